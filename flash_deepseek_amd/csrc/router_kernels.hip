// router_kernels.hip -- router logits and route() for DeepSeek-V3 noaux_tc
// routing (infer.m:350-353, 376, 920-991).
//
// Exactness.  Indices must match the reference bit for bit, so both halves
// of the router are defined operation by operation:
//  - logits: partial t of 256 accumulates float4 chunks t, t+256, ... with
//    one fma per element; the partials are reduced by an xor butterfly per
//    wave and the four wave sums combined as (s0 + s1) + (s2 + s3).  The C
//    restatement (oracle) sums in this same order.
//  - sigmoid: 1/(1 + expf(-x)) with expf evaluated as a double-precision
//    exp built from fma/mul/add (exp_det) and rounded once; float division
//    and addition are IEEE, so the CPU and GPU agree bit for bit.
//  - route: the reference's sequential semantics (running top-2 per group,
//    strict-> group passes with lowest index winning ties, replace-the-
//    first-minimum slot scan over experts in index order, weights summed in
//    slot order) are reproduced by one wave: top-2 by a multiset butterfly,
//    group choice by uniform passes, and the slot scan by ballots that jump
//    straight to the next expert able to displace the current minimum.
#include "fdm_internal.h"

namespace fdm {

__device__ __noinline__ double exp_det(double x) {
#pragma clang fp contract(off)
  if (x != x) return x;
  if (x > 709.0) return __builtin_inf();
  if (x < -746.0) return 0.0;
  const double inv_ln2 = 1.4426950408889634;
  const double ln2_hi = 0x1.62e42fefa39efp-1;
  const double ln2_lo = 0x1.abc9e3b39803fp-56;
  const double t = x * inv_ln2;
  const double k = floor(t + 0.5);
  double r = fma(-k, ln2_hi, x);
  r = fma(-k, ln2_lo, r);
  const double inv_fact[14] = {1.0,         1.0,          1.0 / 2,       1.0 / 6,
                               1.0 / 24,    1.0 / 120,    1.0 / 720,     1.0 / 5040,
                               1.0 / 40320, 1.0 / 362880, 1.0 / 3628800, 1.0 / 39916800,
                               1.0 / 479001600, 1.0 / 6227020800.0};
  double p = inv_fact[13];
#pragma unroll
  for (int i = 12; i >= 0; --i) p = fma(p, r, inv_fact[i]);
  return ldexp(p, (int)k);
}

__device__ __forceinline__ float sigmoid_det(float x) {
#pragma clang fp contract(off)
  const float e = (float)exp_det((double)(-x));
  return __fdiv_rn(1.0f, 1.0f + e);
}

__device__ __forceinline__ float load_relaxed(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// route() for one token, executed by one full wave.  Expert i lives in
// lane i % 64 of "chunk" i / 64; group of expert i = i / 32.
// R1 geometry: 256 experts, 8 groups of 32, 4 groups kept.
__device__ void route_wave(const float* logits, const float* bias, int K, float scale,
                          int* __restrict__ idx_out, float* __restrict__ w_out) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  float score[4], choice[4], gs_lane[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = 64 * j + lane;
    score[j] = sigmoid_det(load_relaxed(logits + i));
    choice[j] = score[j] + (bias ? bias[i] : 0.0f);
    // running top-2 of the group = top-2 of the multiset of choices that
    // exceed -1e30 (NaN never enters), padded with -1e30
    float t1 = choice[j] > -1e30f ? choice[j] : -1e30f;
    float t2 = -1e30f;
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) {
      const float o1 = __shfl_xor(t1, m, 32);
      const float o2 = __shfl_xor(t2, m, 32);
      const float n2 = fmaxf(fminf(t1, o1), fmaxf(t2, o2));
      t1 = fmaxf(t1, o1);
      t2 = n2;
    }
    gs_lane[j] = t1 + t2;
  }
  float gs[8];
#pragma unroll
  for (int G = 0; G < 8; ++G) gs[G] = __shfl(gs_lane[G >> 1], (G & 1) * 32);
  unsigned selmask = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    int best = -1;
    float bs = -1e30f;
#pragma unroll
    for (int G = 0; G < 8; ++G) {
      if (!((selmask >> G) & 1u) && gs[G] > bs) {
        bs = gs[G];
        best = G;
      }
    }
    if (best >= 0) selmask |= 1u << best;
  }
  // Slot scan.  Slot k lives in lane k (k < K <= 16).  mu / minslot are the
  // current first minimum; candidates are re-balloted after each insertion.
  float key = -1e30f;
  int id = 0;
  float mu = -1e30f;
  int minslot = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool in_sel = (selmask >> (2 * j + (lane >> 5))) & 1u;
    const float v = in_sel ? choice[j] : -1e30f;
    unsigned long long cand = __ballot(v > mu);
    while (cand) {
      const int l = __ffsll((unsigned long long)cand) - 1;
      const float vl = __shfl(v, l);
      if (lane == minslot) {
        key = vl;
        id = 64 * j + l;
      }
      float kk = lane < K ? key : __builtin_inff();
      kk = fminf(kk, __shfl_xor(kk, 8));
      kk = fminf(kk, __shfl_xor(kk, 4));
      kk = fminf(kk, __shfl_xor(kk, 2));
      kk = fminf(kk, __shfl_xor(kk, 1));
      mu = __shfl(kk, 0);
      const unsigned long long eq = __ballot(lane < K && key == mu);
      minslot = __ffsll((unsigned long long)eq) - 1;
      const unsigned long long later = (l == 63) ? 0ull : (~0ull << (l + 1));
      cand = __ballot(v > mu) & later;
    }
  }
  // Weights: unbiased scores of the picks, normalised in slot order.
  const int jj = id >> 6, ll = id & 63;
  const float s0 = __shfl(score[0], ll), s1 = __shfl(score[1], ll);
  const float s2 = __shfl(score[2], ll), s3 = __shfl(score[3], ll);
  float wv = jj == 0 ? s0 : (jj == 1 ? s1 : (jj == 2 ? s2 : s3));
  float sum = 0.0f;
  for (int k = 0; k < K; ++k) sum += __shfl(wv, k);
  if (sum > 0.0f) {
    const float f = __fdiv_rn(scale, sum);
    wv *= f;
  }
  if (lane < K) {
    idx_out[lane] = id;
    w_out[lane] = wv;
  }
}

// One router logit per (expert, token) in the canonical order; TPW tokens
// share each load of the weight row.
template <int TPW>
__global__ __launch_bounds__(256) void k_router_logits(const float* __restrict__ Wg,
                                                       const float* __restrict__ x, int n_exp,
                                                       int dim, int T,
                                                       float* __restrict__ logits) {
#pragma clang fp contract(off)
  __shared__ float red[4][TPW];
  const int e = blockIdx.x, t0 = blockIdx.y * TPW;
  const int n4 = dim >> 2;
  const float4* w4 = reinterpret_cast<const float4*>(Wg + (size_t)e * dim);
  float acc[TPW];
#pragma unroll
  for (int q = 0; q < TPW; ++q) acc[q] = 0.0f;
  for (int c = threadIdx.x; c < n4; c += 256) {
    const float4 w = w4[c];
#pragma unroll
    for (int q = 0; q < TPW; ++q) {
      if (t0 + q < T) {
        const float4 xv = reinterpret_cast<const float4*>(x + (size_t)(t0 + q) * dim)[c];
        float a = acc[q];
        a = fmaf(w.x, xv.x, a);
        a = fmaf(w.y, xv.y, a);
        a = fmaf(w.z, xv.z, a);
        a = fmaf(w.w, xv.w, a);
        acc[q] = a;
      }
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int q = 0; q < TPW; ++q) {
    float v = acc[q];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = v + __shfl_xor(v, m);
    if (lane == 0) red[wave][q] = v;
  }
  __syncthreads();
  if (threadIdx.x < TPW && t0 + (int)threadIdx.x < T) {
    const int q = threadIdx.x;
    logits[(size_t)(t0 + q) * n_exp + e] = (red[0][q] + red[1][q]) + (red[2][q] + red[3][q]);
  }
}

__global__ __launch_bounds__(256) void k_route(const float* __restrict__ logits,
                                               const float* __restrict__ bias, int T, int K,
                                               int* __restrict__ idx, float* __restrict__ w) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  route_wave(logits + (size_t)t * 256, bias, K, 2.5f, idx + (size_t)t * K, w + (size_t)t * K);
}

// Batch-1 front end of the MoE layer; 256 workgroups, one per expert.
__global__ __launch_bounds__(256) void k_router_layer(const float* __restrict__ Wg,
                                                      const float* __restrict__ bias,
                                                      const float* __restrict__ h, int K,
                                                      float* __restrict__ logits,
                                                      XGroup* __restrict__ xd,
                                                      int* __restrict__ idx,
                                                      float* __restrict__ w,
                                                      int* __restrict__ counter) {
#pragma clang fp contract(off)
  __shared__ float red[4];
  __shared__ int is_last;
  const int e = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // digits of h_post: group e (112 groups of 64 elements)
  if (e < kHidden / 64 && wave == 1) {
    const float v = h[e * 64 + lane];
    int8_t a, b;
    float s, sum;
    make_digits32(v, a, b, s, sum);
    XGroup* g = xd + e;
    g->a[lane] = a;
    g->b[lane] = b;
    if ((lane & 31) == 0) {
      g->s[lane >> 5] = s;
      g->xsum[lane >> 5] = sum;
    }
  }
  const float4* w4 = reinterpret_cast<const float4*>(Wg + (size_t)e * kHidden);
  const float4* x4 = reinterpret_cast<const float4*>(h);
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < kHidden / 1024; ++i) {
    const int c = threadIdx.x + 256 * i;
    const float4 wv = w4[c], xv = x4[c];
    acc = fmaf(wv.x, xv.x, acc);
    acc = fmaf(wv.y, xv.y, acc);
    acc = fmaf(wv.z, xv.z, acc);
    acc = fmaf(wv.w, xv.w, acc);
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) acc = acc + __shfl_xor(acc, m);
  if (lane == 0) red[wave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    logits[e] = (red[0] + red[1]) + (red[2] + red[3]);
    __threadfence();
    const int done = atomicAdd(counter, 1);
    is_last = (done == (int)gridDim.x - 1);
  }
  __syncthreads();
  if (is_last) {
    __threadfence();
    if (wave == 0) route_wave(logits, bias, K, 2.5f, idx, w);
    if (threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

hipError_t launch_router_logits(const float* Wg, const float* x, int n_exp, int dim, int T,
                                float* logits, hipStream_t s) {
  if (T <= 1) {
    hipLaunchKernelGGL(k_router_logits<1>, dim3(n_exp, T), dim3(256), 0, s, Wg, x, n_exp, dim,
                       T, logits);
  } else {
    hipLaunchKernelGGL(k_router_logits<8>, dim3(n_exp, (T + 7) / 8), dim3(256), 0, s, Wg, x,
                       n_exp, dim, T, logits);
  }
  return hipGetLastError();
}

hipError_t launch_route(const float* logits, const float* bias, int T, int K, int* idx, float* w,
                        hipStream_t s) {
  hipLaunchKernelGGL(k_route, dim3((T + 3) / 4), dim3(256), 0, s, logits, bias, T, K, idx, w);
  return hipGetLastError();
}

hipError_t launch_router_layer(const float* Wg, const float* bias, const float* h_post, int K,
                               float* logits, XGroup* xd, int* idx, float* w, int* counter,
                               hipStream_t s) {
  hipLaunchKernelGGL(k_router_layer, dim3(256), dim3(256), 0, s, Wg, bias, h_post, K, logits,
                     xd, idx, w, counter);
  return hipGetLastError();
}

}  // namespace fdm
