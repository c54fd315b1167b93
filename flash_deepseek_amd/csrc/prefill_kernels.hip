// prefill_kernels.hip -- rms_norm (infer.m:369-374) on the device, bit-exact:
// the tokens of a prefill step (infer.m:1850, 1878-1922) and the attention's
// norms.  Its expert GEMMs are in gemm_kernels.hip.
#include "fdm_internal.h"
#include "planes_device.h"
#include "rms_device.h"

namespace fdm {

// ---- rms_norm: o = x * (1 / sqrt(sum x^2 / d + 1e-6)) * w -------------------------------
// One workgroup per token.  The sum of squares is the reference's
// sequential fma chain, evaluated bit for bit by rms_sumsq_exact (runs of
// integer steps inside a binade, the steps at binade edges and ties walked
// in order); sqrt and division are IEEE; o = (x * inv) * w as infer.m:372.
// At d = 7168 (16-byte aligned rows) every load is a 16-byte vector load
// issued before the sum, so the row's latency is paid once.
__device__ __forceinline__ void rms_norm_row(const float* __restrict__ xr, const float* __restrict__ w,
                                             float* orow, int d, RmsSmem& sm) {
  const int n = (d + kRmsThreads - 1) / kRmsThreads;
  const int i0 = threadIdx.x * n;
  const bool vec = d == kHidden && (reinterpret_cast<uintptr_t>(xr) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(orow) & 15) == 0 &&
                   (!w || (reinterpret_cast<uintptr_t>(w) & 15) == 0);
  float xv[kRmsMaxPer];
  if (vec) {
    constexpr int kV = kHidden / 4 / kRmsThreads;  // 7 vectors per thread
    const f32x4* x4 = reinterpret_cast<const f32x4*>(xr);
    f32x4 xc[kV], wc[kV];
#pragma unroll
    for (int k = 0; k < kV; ++k) {
      const f32x4 v = x4[i0 / 4 + k];  // the thread's 28 consecutive elements
      xv[4 * k] = v.x;
      xv[4 * k + 1] = v.y;
      xv[4 * k + 2] = v.z;
      xv[4 * k + 3] = v.w;
      xc[k] = x4[threadIdx.x + kRmsThreads * k];  // coalesced, for the output
      wc[k] = w ? reinterpret_cast<const f32x4*>(w)[threadIdx.x + kRmsThreads * k] : f32x4{1.0f, 1.0f, 1.0f, 1.0f};
    }
    const float inv = rms_inv(rms_sumsq_exact(xv, d, sm), d);
#pragma unroll
    for (int k = 0; k < kV; ++k) {
      f32x4 v;
      v.x = xc[k].x * inv;
      v.y = xc[k].y * inv;
      v.z = xc[k].z * inv;
      v.w = xc[k].w * inv;
      if (w) {
        v.x = v.x * wc[k].x;
        v.y = v.y * wc[k].y;
        v.z = v.z * wc[k].z;
        v.w = v.w * wc[k].w;
      }
      reinterpret_cast<f32x4*>(orow)[threadIdx.x + kRmsThreads * k] = v;
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < kRmsMaxPer; ++j) {
    const float v = xr[min(i0 + j, d - 1)];  // every slot loads; past the row it is a zero step
    xv[j] = (j < n && i0 + j < d) ? v : 0.0f;
  }
  const float inv = rms_inv(rms_sumsq_exact(xv, d, sm), d);
  for (int i = threadIdx.x; i < d; i += kRmsThreads) {
    const float v = xr[i] * inv;
    orow[i] = w ? v * w[i] : v;
  }
}

__global__ __launch_bounds__(kRmsThreads) void k_rms_norm(const float* __restrict__ x,
                                                          const float* __restrict__ w, float* o, int d) {
  __shared__ RmsSmem sm;
  rms_norm_row(x + (size_t)blockIdx.x * d, w, o + (size_t)blockIdx.x * d, d, sm);
}

// rms_norm of one token of 7168 (bit-exact, as k_rms_norm), then the one
// fp16 plane of the normalised row that the prefill's grouped GEMMs read
// (planes_device.h): thread sb re-reads sub-block sb of the row this
// workgroup has just written (its own stores, visible after the barrier).
__global__ __launch_bounds__(kRmsThreads) void k_rms_norm_planes(const float* __restrict__ x,
                                                                 const float* __restrict__ w, float* o,
                                                                 size_t T, _Float16* __restrict__ xp,
                                                                 float* __restrict__ xs, float* __restrict__ xe) {
  constexpr int NSB = kHidden / 32;
  static_assert(NSB <= kRmsThreads, "a sub-block per thread");
  __shared__ RmsSmem sm;
  __shared__ float red[kRmsThreads / 64];
  const size_t row = blockIdx.x;
  float* orow = o + row * kHidden;
  rms_norm_row(x + row * kHidden, w, orow, kHidden, sm);
  __syncthreads();
  const int sb = threadIdx.x;
  f32x4 v[8];
  float m = 0.0f;
  if (sb < NSB) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = reinterpret_cast<const f32x4*>(orow + 32 * sb)[i];
    m = subblock_absmax(v);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  if (sb >= NSB) return;
  const int sh = planes_shift(m);
  if (sb == 0) xe[row] = ldexpf(1.0f, -sh);
  xs[row * NSB + sb] = planes_subblock<1>(v, sh, xp + row * kHidden + 32 * sb, T * kHidden);
}

hipError_t launch_rms_norm_planes(const float* x, const float* w, float* o, int T, _Float16* xp, float* xs,
                                  float* xe, hipStream_t s) {
  hipLaunchKernelGGL(k_rms_norm_planes, dim3(T), dim3(kRmsThreads), 0, s, x, w, o, (size_t)T, xp, xs, xe);
  return hipGetLastError();
}

// Two independent rows of different widths in one launch (the attention's
// q_a and kv_a norms): workgroup 0 and 1.
__global__ __launch_bounds__(kRmsThreads) void k_rms_norm_pair(const float* __restrict__ x0,
                                                               const float* __restrict__ w0, float* o0, int d0,
                                                               const float* __restrict__ x1,
                                                               const float* __restrict__ w1, float* o1, int d1) {
  __shared__ RmsSmem sm;
  if (blockIdx.x == 0)
    rms_norm_row(x0, w0, o0, d0, sm);
  else
    rms_norm_row(x1, w1, o1, d1, sm);
}

hipError_t launch_rms_norm_pair(const float* x0, const float* w0, float* o0, int d0, const float* x1,
                                const float* w1, float* o1, int d1, hipStream_t s) {
  hipLaunchKernelGGL(k_rms_norm_pair, dim3(2), dim3(kRmsThreads), 0, s, x0, w0, o0, d0, x1, w1, o1, d1);
  return hipGetLastError();
}

hipError_t launch_rms_norm(const float* x, const float* w, float* o, int T, int d, hipStream_t s) {
  hipLaunchKernelGGL(k_rms_norm, dim3(T), dim3(kRmsThreads), 0, s, x, w, o, d);
  return hipGetLastError();
}

}  // namespace fdm
