// synth_kernels.hip -- seeded synthetic tensors on the device (benchmark
// inputs).  Same generator as the C restatement (oracle/synth.c):
//   uniform byte p   = byte (p % 8) of splitmix64(seed, p / 8)
//   normal number i  = Box-Muller (cosine branch) of draws 2i, 2i+1
//   Q4_K d, dmin     = fp16(|0.02 N|), draws 2b, 2b+1 of a sub-seed
//   Q6_K d           = fp16(|0.02 N|), draw b of a sub-seed
// Integer streams match the CPU bit for bit; the normals go through the
// device's double log/cos, then are rounded to fp16 by integer steps.
#include "fdm_internal.h"

namespace fdm {

__device__ __forceinline__ uint64_t rand_u64(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ double std_normal(uint64_t seed, uint64_t i) {
  const double u1 = ((double)(rand_u64(seed, 2 * i) >> 11) + 1.0) * 0x1.0p-53;
  const double u2 = (double)(rand_u64(seed, 2 * i + 1) >> 11) * 0x1.0p-53;
  return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

// double -> IEEE half, round to nearest even (same steps as synth.c).
__device__ uint16_t to_half_rne(double v) {
  uint16_t sign = 0;
  if (v < 0) {
    sign = 0x8000;
    v = -v;
  }
  if (v >= 65520.0) return sign | 0x7C00;
  if (v < 0x1.0p-25) return sign;
  int e;
  const double m = frexp(v, &e);
  int exp_h = e - 1 + 15;
  if (exp_h <= 0) return sign | (uint16_t)rint(ldexp(v, 24));
  uint32_t mant = (uint32_t)rint(ldexp(m, 11));
  if (mant == 2048) {
    mant = 1024;
    ++exp_h;
  }
  if (exp_h >= 31) return sign | 0x7C00;
  return sign | (uint16_t)(exp_h << 10) | (uint16_t)(mant - 1024);
}

__global__ __launch_bounds__(256) void k_synth_words(uint64_t* __restrict__ dst, size_t n_words,
                                                     uint64_t seed) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_words; i += stride)
    dst[i] = rand_u64(seed, i);
}

__global__ __launch_bounds__(256) void k_synth_tail(uint8_t* __restrict__ dst, size_t first,
                                                    size_t n, uint64_t seed) {
  const size_t p = first + threadIdx.x;
  if (p < n) dst[p] = (uint8_t)(rand_u64(seed, p >> 3) >> (8 * (p & 7)));
}

__global__ __launch_bounds__(256) void k_patch_q4k(uint8_t* __restrict__ dst, size_t n_blocks,
                                                   uint64_t sub) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x; b < n_blocks; b += stride) {
    const uint16_t d = to_half_rne(fabs(0.02 * std_normal(sub, 2 * b)));
    const uint16_t dm = to_half_rne(fabs(0.02 * std_normal(sub, 2 * b + 1)));
    *reinterpret_cast<uint32_t*>(dst + b * kQ4KBlock) = (uint32_t)d | ((uint32_t)dm << 16);
  }
}

__global__ __launch_bounds__(256) void k_patch_q6k(uint8_t* __restrict__ dst, size_t n_blocks,
                                                   uint64_t sub) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x; b < n_blocks; b += stride) {
    const uint16_t d = to_half_rne(fabs(0.02 * std_normal(sub, b)));
    *reinterpret_cast<uint16_t*>(dst + b * kQ6KBlock + 208) = d;
  }
}

__global__ __launch_bounds__(256) void k_synth_normal(float* __restrict__ dst, size_t n,
                                                      float mean, float std_dev, uint64_t seed) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    dst[i] = (float)((double)mean + (double)std_dev * std_normal(seed, i));
}

static unsigned grid_cap(size_t n) {
  size_t wg = (n + 255) / 256;
  const size_t cap = (size_t)(g_num_cus > 0 ? g_num_cus : 256) * 32;
  if (wg > cap) wg = cap;
  return (unsigned)(wg ? wg : 1);
}

static hipError_t synth_bytes(uint8_t* dst, size_t n, uint64_t seed, hipStream_t s) {
  const size_t words = n / 8;
  if (words)
    hipLaunchKernelGGL(k_synth_words, dim3(grid_cap(words)), dim3(256), 0, s,
                       reinterpret_cast<uint64_t*>(dst), words, seed);
  if (n % 8) hipLaunchKernelGGL(k_synth_tail, dim3(1), dim3(256), 0, s, dst, words * 8, n, seed);
  return hipGetLastError();
}

// sub-seed of field 1, as synth.c: rand_u64(seed, ~1)
static uint64_t host_rand_u64(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

hipError_t launch_synth_q4k(uint8_t* dst, size_t n_blocks, uint64_t seed, hipStream_t s) {
  hipError_t e = synth_bytes(dst, n_blocks * kQ4KBlock, seed, s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_patch_q4k, dim3(grid_cap(n_blocks)), dim3(256), 0, s, dst, n_blocks,
                     host_rand_u64(seed, ~1ull));
  return hipGetLastError();
}

hipError_t launch_synth_q6k(uint8_t* dst, size_t n_blocks, uint64_t seed, hipStream_t s) {
  hipError_t e = synth_bytes(dst, n_blocks * kQ6KBlock, seed, s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_patch_q6k, dim3(grid_cap(n_blocks)), dim3(256), 0, s, dst, n_blocks,
                     host_rand_u64(seed, ~1ull));
  return hipGetLastError();
}

hipError_t launch_synth_normal(float* dst, size_t n, float mean, float std_dev, uint64_t seed,
                               hipStream_t s) {
  hipLaunchKernelGGL(k_synth_normal, dim3(grid_cap(n)), dim3(256), 0, s, dst, n, mean, std_dev,
                     seed);
  return hipGetLastError();
}

}  // namespace fdm
