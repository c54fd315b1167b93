// prefill_kernels.hip -- rms_norm of the tokens of a prefill step (and of
// the attention's norms): rms_norm (infer.m:369-374) on the device,
// bit-exact.  Prefill runs h <- h + MoE(rms_norm(h, w_l)) per layer
// (infer.m:1850, 1878-1922); its expert GEMMs are in gemm_kernels.hip.
#include "fdm_internal.h"

namespace fdm {

// ---- rms_norm: h_post = x * (1 / sqrt(sum x^2 / d + 1e-6)) * w ---------------------------
// One workgroup per token.  The sum of squares is taken in index order by
// one thread with one fused multiply-add per element, as the reference's
// loop compiles (infer.m:369-374: clang contracts `ss += x[i]*x[i]`), so
// h_post -- and with it the routing -- is bit-exact; sqrt and division are
// IEEE.
__global__ __launch_bounds__(256) void k_rms_norm(const float* __restrict__ x,
                                                  const float* __restrict__ w, float* __restrict__ o,
                                                  int d, float eps) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float row[kHidden];
  __shared__ float inv_s;
  const float* xr = x + (size_t)blockIdx.x * d;
  for (int i = threadIdx.x; i < d; i += 256) row[i] = xr[i];
  __syncthreads();
  if (threadIdx.x == 0) {
    // the reference's loop as compiled: ss = fma(x_i, x_i, ss) in index order
    // (clang contracts `ss += x[i]*x[i]`); one dependent chain, fed 16
    // values at a time from LDS so the reads run ahead of it
    float ss = 0.0f;
    const int n64 = d / 64;
    const f32x4* r4 = reinterpret_cast<const f32x4*>(row);
    f32x4 buf[2][16];  // 64 values per chunk, the next chunk's reads in flight
    if (n64 > 0) {
#pragma unroll
      for (int k = 0; k < 16; ++k) buf[0][k] = r4[k];
    }
    for (int c = 0; c < n64; c += 2) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (c + h >= n64) break;
        if (c + h + 1 < n64) {
#pragma unroll
          for (int k = 0; k < 16; ++k) buf[h ^ 1][k] = r4[16 * (c + h + 1) + k];
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          const f32x4 v = buf[h][k];
          ss = fmaf(v.x, v.x, ss);
          ss = fmaf(v.y, v.y, ss);
          ss = fmaf(v.z, v.z, ss);
          ss = fmaf(v.w, v.w, ss);
        }
      }
    }
    for (int i = 64 * n64; i < d; ++i) ss = fmaf(row[i], row[i], ss);
    inv_s = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, (float)d) + eps));
  }
  __syncthreads();
  const float inv = inv_s;
  for (int i = threadIdx.x; i < d; i += 256) {
    const float v = w ? (row[i] * inv) * w[i] : row[i] * inv;
    o[(size_t)blockIdx.x * d + i] = v;
  }
}

hipError_t launch_rms_norm(const float* x, const float* w, float* o, int T, int d, hipStream_t s) {
  hipLaunchKernelGGL(k_rms_norm, dim3(T), dim3(256), 0, s, x, w, o, d, 1e-6f);
  return hipGetLastError();
}

}  // namespace fdm
