// router_kernels.hip -- router logits and route() for DeepSeek-V3 noaux_tc
// routing (infer.m:350-353, 376, 920-991).
//
// Exactness.  Indices must match the reference bit for bit, so the logits
// are defined operation by operation: partial t of 256 accumulates float4
// chunks t, t+256, ... with one fma per element; the partials are reduced
// as by an xor butterfly per wave (lane 0 adds the same pairs in the same
// order, through lane permutes and DPP shifts: wave_sum_lane0) and the four
// wave sums combined as (s0 + s1) + (s2 + s3).  The C restatement (oracle) sums in this same
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
  for (int q = 0; q < TPW; ++q) acc[q] = wave_sum_lane0(acc[q]);
  if (lane == 0) {
#pragma unroll
    for (int q = 0; q < TPW; ++q) red[wave][q] = acc[q];
  }
  __syncthreads();
  if (threadIdx.x < TPW && t0 + (int)threadIdx.x < T) {
    const int q = threadIdx.x;
    logits[(size_t)(t0 + q) * n_exp + e] = (red[0][q] + red[1][q]) + (red[2][q] + red[3][q]);
  }
}

// The same logits for a block of EPB experts x TPW tokens per workgroup:
// each weight chunk and each token chunk is loaded once per block and used
// EPB (TPW) times, so the L2 traffic of many tokens is (n_exp / EPB) token
// reads + (T / TPW) weight reads instead of n_exp token reads.  Every
// logit is still its own canonical chain: partial t over chunks t, t+256, ...
// with one fma per element, butterfly, (s0 + s1) + (s2 + s3).
template <int EPB, int TPW>
__global__ __launch_bounds__(256) void k_router_logits_blk(const float* __restrict__ Wg,
                                                           const float* __restrict__ x, int n_exp,
                                                           int dim, int T,
                                                           float* __restrict__ logits) {
#pragma clang fp contract(off)
  __shared__ float red[4][EPB][TPW];
  const int e0 = blockIdx.x * EPB, t0 = blockIdx.y * TPW;
  const int n4 = dim >> 2;
  float acc[EPB][TPW];
#pragma unroll
  for (int k = 0; k < EPB; ++k)
#pragma unroll
    for (int q = 0; q < TPW; ++q) acc[k][q] = 0.0f;
  for (int c = threadIdx.x; c < n4; c += 256) {
    float4 xv[TPW];
#pragma unroll
    for (int q = 0; q < TPW; ++q)
      xv[q] = reinterpret_cast<const float4*>(x + (size_t)min(t0 + q, T - 1) * dim)[c];
#pragma unroll
    for (int k = 0; k < EPB; ++k) {
      const float4 w = reinterpret_cast<const float4*>(Wg + (size_t)(e0 + k) * dim)[c];
#pragma unroll
      for (int q = 0; q < TPW; ++q) {
        float a = acc[k][q];
        a = fmaf(w.x, xv[q].x, a);
        a = fmaf(w.y, xv[q].y, a);
        a = fmaf(w.z, xv[q].z, a);
        a = fmaf(w.w, xv[q].w, a);
        acc[k][q] = a;
      }
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // every logit's butterfly sum into lane 0 (the same adds in the same
  // order), without lane exchanges through the LDS crossbar
#pragma unroll
  for (int k = 0; k < EPB; ++k)
#pragma unroll
    for (int q = 0; q < TPW; ++q) acc[k][q] = wave_sum_lane0(acc[k][q]);
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < EPB; ++k)
#pragma unroll
      for (int q = 0; q < TPW; ++q) red[wave][k][q] = acc[k][q];
  }
  __syncthreads();
  if (threadIdx.x < EPB * TPW) {
    const int k = threadIdx.x / TPW, q = threadIdx.x % TPW;
    if (t0 + q < T)
      logits[(size_t)(t0 + q) * n_exp + e0 + k] = (red[0][k][q] + red[1][k][q]) + (red[2][k][q] + red[3][k][q]);
  }
}

__global__ __launch_bounds__(256) void k_route(const float* __restrict__ logits,
                                               const float* __restrict__ bias, int T, int K,
                                               int* __restrict__ idx, float* __restrict__ w) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  route_wave(logits + (size_t)t * 256, bias, K, 2.5f, idx + (size_t)t * K, w + (size_t)t * K);
}

hipError_t launch_router_logits(const float* Wg, const float* x, int n_exp, int dim, int T,
                                float* logits, hipStream_t s) {
  if (T <= 1) {
    hipLaunchKernelGGL(k_router_logits<1>, dim3(n_exp, T), dim3(256), 0, s, Wg, x, n_exp, dim,
                       T, logits);
  } else if (T >= 16 && n_exp % 8 == 0) {
    hipLaunchKernelGGL((k_router_logits_blk<8, 8>), dim3(n_exp / 8, (T + 7) / 8), dim3(256), 0, s, Wg, x,
                       n_exp, dim, T, logits);
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

}  // namespace fdm
