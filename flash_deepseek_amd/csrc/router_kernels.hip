// router_kernels.hip -- router logits and route() for DeepSeek-V3 noaux_tc
// routing (infer.m:350-353, 376, 920-991).
//
// Exactness.  Indices must match the reference bit for bit, so the logits
// are defined operation by operation: partial t of 256 accumulates float4
// chunks t, t+256, ... with one fma per element; the partials are reduced
// by an xor butterfly per wave and the four wave sums combined as
// (s0 + s1) + (s2 + s3).  The C restatement (oracle) sums in this same
// order.  route() itself is in route_device.h.
#include "fdm_internal.h"
#include "route_device.h"

namespace fdm {

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

// Dot of one Q4_K group with fp32 activations x64 (the group's 64 values)
// and their two sub-block sums: sum over the group of (d*sc*q - dmin*m)*x.
__device__ __forceinline__ float q4k_group_dot_f32(const u32x4 hdr, const u32x4 q0, const u32x4 q1,
                                                   const Q4KScaleSel& sel,
                                                   const float* __restrict__ x64, float xs0,
                                                   float xs1) {
  const uint32_t wq[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
  const f32x4* xv = reinterpret_cast<const f32x4*>(x64);
  float a0 = 0.0f, a1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t lo = wq[i] & 0x0F0F0F0Fu, hi = (wq[i] >> 4) & 0x0F0F0F0Fu;
    const f32x4 xl = xv[i], xh = xv[8 + i];
    a0 = fmaf((float)(lo & 0xFF), xl.x, a0);
    b0 = fmaf((float)((lo >> 8) & 0xFF), xl.y, b0);
    a0 = fmaf((float)((lo >> 16) & 0xFF), xl.z, a0);
    b0 = fmaf((float)(lo >> 24), xl.w, b0);
    a1 = fmaf((float)(hi & 0xFF), xh.x, a1);
    b1 = fmaf((float)((hi >> 8) & 0xFF), xh.y, b1);
    a1 = fmaf((float)((hi >> 16) & 0xFF), xh.z, a1);
    b1 = fmaf((float)(hi >> 24), xh.w, b1);
  }
  int sc0, m0, sc1, m1;
  q4k_scale_min_pair(hdr.y, hdr.z, hdr.w, sel, sc0, m0, sc1, m1);
  const float d = half_to_float(hdr.x), dmin = half_to_float(hdr.x >> 16);
  const float qx = fmaf((float)sc0, a0 + b0, (float)sc1 * (a1 + b1));
  const float mx = fmaf((float)m0, xs0, (float)m1 * xs1);
  return fmaf(d, qx, -dmin * mx);
}

// Batch-1 front end of the MoE layer, one launch of 512 workgroups:
//  0..255    router row e (4 waves = the 4 canonical runs of 64 partials),
//            stored as its sigmoid score; workgroups 0..27 also produce the
//            digits of h_post (one 64-element group per wave).  Arrival is
//            counted in two levels (16 groups of 16 workgroups, then the 16
//            group finishers), so no counter sees more than 16 atomics; the
//            last workgroup reads the 256 scores and selects the expert SET
//            (route_set_wave) into prov_idx.  The exact reference slot order
//            and weights are produced later, off the critical path, by the
//            gate/up launch.
//  256..511  gate/up + SwiGLU of the shared expert (which needs no routing)
//            for 8 rows each, against fp32 h_post staged in LDS, while the
//            router runs; the activation digits are finished as in k_gateup.
constexpr int kRouterWGs = 256;
constexpr int kArriveGroup = 16;
constexpr int kCounterStride = 64;  // ints between counters (256 bytes)

__global__ __launch_bounds__(256) void k_router_layer(const float* __restrict__ Wg,
                                                      const float* __restrict__ bias,
                                                      const float* __restrict__ h, int K,
                                                      float* __restrict__ scores,
                                                      XGroup* __restrict__ xd,
                                                      int* __restrict__ prov_idx,
                                                      int* __restrict__ counters,
                                                      const uint8_t* __restrict__ shared,
                                                      float* __restrict__ act_s,
                                                      XGroup* __restrict__ act_xd_s,
                                                      int* __restrict__ gu_counters_s) {
#pragma clang fp contract(off)
  __shared__ float xf[kHidden];
  __shared__ float xsum[kHidden / 32];
  __shared__ float red[4];
  __shared__ int flag;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (blockIdx.x >= kRouterWGs) {
    // ---- shared expert gate/up tile ----
    const int tile = blockIdx.x - kRouterWGs;
    const int q = lane >> 4, l16 = lane & 15, g = l16 & 3;
    const int row = tile * 8 + 2 * wave + (q & 1);
    const uint8_t* rowp = shared + (q >= 2 ? kGateBytes : 0) + (size_t)row * kQ4KRowHidden;
    Q4KGroupLoad ld[7];
#pragma unroll
    for (int i = 0; i < 7; ++i) ld[i] = q4k_load_group(rowp + (4 * i + (l16 >> 2)) * kQ4KBlock, g);
    const float4* h4 = reinterpret_cast<const float4*>(h);
    for (int i = threadIdx.x; i < kHidden / 4; i += 256) reinterpret_cast<float4*>(xf)[i] = h4[i];
    __syncthreads();
    if (threadIdx.x < kHidden / 32) {
      float sacc = 0.0f;
      for (int k = 0; k < 32; ++k) sacc += xf[32 * threadIdx.x + k];
      xsum[threadIdx.x] = sacc;
    }
    __syncthreads();
    const Q4KScaleSel sel = q4k_scale_sel(g);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 7; ++i) {
      const int G = 16 * i + l16;
      u32x4 hd;
      hd.x = quad_bcast<0>(ld[i].hdr_part);
      hd.y = quad_bcast<1>(ld[i].hdr_part);
      hd.z = quad_bcast<2>(ld[i].hdr_part);
      hd.w = quad_bcast<3>(ld[i].hdr_part);
      acc += q4k_group_dot_f32(hd, ld[i].q0, ld[i].q1, sel, xf + 64 * G, xsum[2 * G],
                               xsum[2 * G + 1]);
      __builtin_amdgcn_sched_barrier(0);
    }
    acc = sum16(acc);
    const float up = __shfl(acc, (lane + 32) & 63);
    if (lane == 0 || lane == 16) {
      store_agent(act_s + row, silu_mul(acc, up));
      wait_stores_done();
    }
    __syncthreads();
    int* cnt = gu_counters_s + (tile >> 2);
    if (threadIdx.x == 0) flag = (arrive_agent(cnt) == 3);
    __syncthreads();
    if (flag && threadIdx.x < 32) {
      const float v = load_agent(act_s + (tile >> 2) * 32 + threadIdx.x);
      int8_t a, b;
      float sc, sum;
      make_digits32(v, a, b, sc, sum);
      XGroup* xg = act_xd_s + (tile >> 3);
      const int half = (tile >> 2) & 1;
      xg->a[32 * half + threadIdx.x] = a;
      xg->b[32 * half + threadIdx.x] = b;
      if (threadIdx.x == 0) {
        xg->s[half] = sc;
        xg->xsum[half] = sum;
        reset_agent(cnt);
      }
    }
    return;
  }
  // ---- router row e ----
  const int e = blockIdx.x;
  const int t = 64 * wave + lane;  // canonical partial index
  const float4* w4 = reinterpret_cast<const float4*>(Wg + (size_t)e * kHidden);
  const float4* x4 = reinterpret_cast<const float4*>(h);
  float4 wv[kHidden / 1024], xv[kHidden / 1024];
#pragma unroll
  for (int i = 0; i < kHidden / 1024; ++i) {
    wv[i] = w4[t + 256 * i];
    xv[i] = x4[t + 256 * i];
  }
  if (e < kHidden / 256) {
    const int G = 4 * e + wave;
    const float v = h[G * 64 + lane];
    int8_t a, b;
    float sc, sum;
    make_digits32(v, a, b, sc, sum);
    XGroup* gx = xd + G;
    gx->a[lane] = a;
    gx->b[lane] = b;
    if ((lane & 31) == 0) {
      gx->s[lane >> 5] = sc;
      gx->xsum[lane >> 5] = sum;
    }
  }
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < kHidden / 1024; ++i) {
    acc = fmaf(wv[i].x, xv[i].x, acc);
    acc = fmaf(wv[i].y, xv[i].y, acc);
    acc = fmaf(wv[i].z, xv[i].z, acc);
    acc = fmaf(wv[i].w, xv[i].w, acc);
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) acc = acc + __shfl_xor(acc, m);
  if (lane == 0) red[wave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    store_agent(scores + e, sigmoid_det((red[0] + red[1]) + (red[2] + red[3])));
    wait_stores_done();
    int* grp = counters + kCounterStride * (1 + e / kArriveGroup);
    int last = 0;
    if (arrive_agent(grp) == kArriveGroup - 1) {
      reset_agent(grp);
      last = arrive_agent(counters) == kRouterWGs / kArriveGroup - 1;
    }
    flag = last;
  }
  __syncthreads();
  if (flag && wave == 0) {
    float sc[4], bj[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      sc[j] = load_agent(scores + 64 * j + lane);
      bj[j] = bias ? bias[64 * j + lane] : 0.0f;
    }
    route_set_wave(sc, bj, K, prov_idx);
    if (lane == 0) reset_agent(counters);
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
                               float* scores, XGroup* xd, int* prov_idx, int* counters,
                               const uint8_t* shared, float* act_s, XGroup* act_xd_s,
                               int* gu_counters_s, hipStream_t s) {
  const int grid = kRouterWGs + (shared ? kFfn / 8 : 0);
  hipLaunchKernelGGL(k_router_layer, dim3(grid), dim3(256), 0, s, Wg, bias, h_post, K, scores,
                     xd, prov_idx, counters, shared, act_s, act_xd_s, gu_counters_s);
  return hipGetLastError();
}

}  // namespace fdm
