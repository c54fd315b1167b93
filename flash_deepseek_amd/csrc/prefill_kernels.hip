// prefill_kernels.hip -- rms_norm (infer.m:369-374) on the device, bit-exact:
// the tokens of a prefill step (infer.m:1850, 1878-1922) and of standalone
// calls (fdm_rms_norm).  Its expert GEMMs are in gemm_kernels.hip.
#include "fdm_internal.h"
#include "planes_device.h"
#include "rms_device.h"

namespace fdm {

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

hipError_t launch_rms_norm(const float* x, const float* w, float* o, int T, int d, hipStream_t s) {
  hipLaunchKernelGGL(k_rms_norm, dim3(T), dim3(kRmsThreads), 0, s, x, w, o, d);
  return hipGetLastError();
}

}  // namespace fdm
