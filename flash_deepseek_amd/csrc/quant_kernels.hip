// quant_kernels.hip -- device twins of quant.h: fp16_to_fp32,
// dequantize_row_q4_K, dequantize_row_q6_K (quant.c:4-92).
//
// Bit-exactness.  quant.c writes y = d1 * q - m1 and y = d * sc * q.  With
// d a half, d * sc and d1 * q are exact in fp32 (at most 21 significant
// bits), so Q4_K rounds once however the expression is evaluated; the Q6_K
// product (d * sc) * q is evaluated in that order.  Contraction is switched
// off in these kernels anyway so that every expression rounds as written.
// The half-precision scales are decoded by integer construction
// (half_bits_exact), which reproduces quant.c's conversion for every bit
// pattern, NaN payloads included.
#include "fdm_internal.h"

namespace fdm {

__global__ __launch_bounds__(256) void k_fp16_to_fp32(const uint16_t* __restrict__ src,
                                                      float* __restrict__ dst, size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    dst[i] = half_bits_exact(src[i]);
}

// One wave per block.  Lane l: 64-element chunk c = l / 16, qs byte pair
// 32c + 2(l % 16) .. +1 -> elements 64c + 2i, +1 (low nibbles) and
// 64c + 32 + 2i, +1 (high nibbles).
__global__ __launch_bounds__(256) void k_dequant_q4k(const uint8_t* __restrict__ src,
                                                     float* __restrict__ dst, size_t nblocks) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int c = lane >> 4, i = lane & 15;
  const size_t waves = ((size_t)gridDim.x * blockDim.x) >> 6;
  for (size_t b = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6; b < nblocks;
       b += waves) {
    const uint8_t* blk = src + b * kQ4KBlock;
    const uint32_t* h32 = reinterpret_cast<const uint32_t*>(blk);
    const uint32_t dd = h32[0], s0 = h32[1], s1 = h32[2], s2 = h32[3];
    const uint32_t q2 = *reinterpret_cast<const uint16_t*>(blk + 16 + 32 * c + 2 * i);
    int sc_lo, m_lo, sc_hi, m_hi;
    q4k_scale_min_pair(s0, s1, s2, c, sc_lo, m_lo, sc_hi, m_hi);
    const float d = half_bits_exact(dd & 0xFFFFu);
    const float dmin = half_bits_exact(dd >> 16);
    const float mul_lo = d * (float)sc_lo, sub_lo = dmin * (float)m_lo;
    const float mul_hi = d * (float)sc_hi, sub_hi = dmin * (float)m_hi;
    float2 lo, hi;
    lo.x = mul_lo * (float)(q2 & 0xF) - sub_lo;
    lo.y = mul_lo * (float)((q2 >> 8) & 0xF) - sub_lo;
    hi.x = mul_hi * (float)((q2 >> 4) & 0xF) - sub_hi;
    hi.y = mul_hi * (float)((q2 >> 12) & 0xF) - sub_hi;
    float* y = dst + b * kQK + 64 * c + 2 * i;
    *reinterpret_cast<float2*>(y) = lo;
    *reinterpret_cast<float2*>(y + 32) = hi;
  }
}

// One wave per block.  Lane l: half h = l / 32, position p = l % 32 ->
// elements 128h + p + 32k, k = 0..3 (quant.c:63-92).
__global__ __launch_bounds__(256) void k_dequant_q6k(const uint8_t* __restrict__ src,
                                                     float* __restrict__ dst, size_t nblocks) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, p = lane & 31;
  const size_t waves = ((size_t)gridDim.x * blockDim.x) >> 6;
  for (size_t b = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6; b < nblocks;
       b += waves) {
    const uint8_t* blk = src + b * kQ6KBlock;
    const uint32_t ql0 = blk[64 * h + p], ql1 = blk[64 * h + p + 32];
    const uint32_t qh = blk[128 + 32 * h + p];
    const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192 + 8 * h);
    const int is = p >> 4;
    const float d = half_bits_exact((uint32_t)blk[208] | ((uint32_t)blk[209] << 8));
    const int q[4] = {(int)((ql0 & 0xF) | (((qh >> 0) & 3) << 4)) - 32,
                      (int)((ql1 & 0xF) | (((qh >> 2) & 3) << 4)) - 32,
                      (int)((ql0 >> 4) | (((qh >> 4) & 3) << 4)) - 32,
                      (int)((ql1 >> 4) | (((qh >> 6) & 3) << 4)) - 32};
    float* y = dst + b * kQK + 128 * h + p;
#pragma unroll
    for (int k = 0; k < 4; ++k) y[32 * k] = d * (float)sc[is + 2 * k] * (float)q[k];
  }
}

// ---- packed blobs -> the resident expert layout (REL) ----------------------------------
// One thread per Q4_K block of a blob's gate, up or Q4_K down matrix: the
// block's header dwords and its 8 half-groups go to their REL pieces (see
// rel_step / rel_piece).  Blob b of n: src + b * src_stride ->
// dst + b * expert_size.  A Q6_K down matrix goes through k_rel_pack_q6.
__global__ __launch_bounds__(256) void k_rel_pack(const uint8_t* __restrict__ src, size_t src_stride,
                                                  uint8_t* __restrict__ dst, size_t expert_size,
                                                  int n_blobs, int with_down) {
  constexpr int kGuBlocks = kFfn * (kHidden / kQK);  // 57,344 per gate / up matrix
  constexpr int kDnBlocks = kHidden * (kFfn / kQK);  // 57,344 per down matrix
  const int per_blob = 2 * kGuBlocks + (with_down ? kDnBlocks : 0);
  const size_t total = (size_t)n_blobs * per_blob;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int b = (int)(i / per_blob);
    int k = (int)(i % per_blob);
    const uint8_t* sb = src + (size_t)b * src_stride;
    uint8_t* db = dst + (size_t)b * expert_size;
    const u32x4* blk;
    uint8_t* step;
    int L, N;
    if (k < 2 * kGuBlocks) {
      const int m = k / kGuBlocks;  // 0 gate, 1 up
      k %= kGuBlocks;
      const int row = k / (kHidden / kQK), block = k % (kHidden / kQK);
      const size_t mo = (size_t)m * kGateBytes;
      blk = reinterpret_cast<const u32x4*>(sb + mo + (size_t)row * kQ4KRowHidden + block * kQ4KBlock);
      step = const_cast<uint8_t*>(rel_step<false>(db + mo, row, block));
      L = rel_piece<false>(row, block, 0);
      N = kRelGuPieces;
    } else {
      k -= 2 * kGuBlocks;
      const int row = k / (kFfn / kQK), block = k % (kFfn / kQK);
      const size_t mo = 2 * (size_t)kGateBytes;
      blk = reinterpret_cast<const u32x4*>(sb + mo + (size_t)row * kQ4KRowFfn + block * kQ4KBlock);
      step = const_cast<uint8_t*>(rel_step<true>(db + mo, row, block));
      L = rel_piece<true>(row, block, 0);
      N = kRelDnPieces;
    }
    u32x4 v[9];
#pragma unroll
    for (int j = 0; j < 9; ++j) v[j] = blk[j];
    // header dwords g = 0..3 (pieces L + g are consecutive)
    *reinterpret_cast<u32x4*>(step + 32 * N + 4 * L) = v[0];
    // qs of group g: bytes 32 g .. 32 g + 31 of the block's qs = v[1 + 2 g], v[2 + 2 g]
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      *reinterpret_cast<u32x4*>(step + 16 * (L + g)) = v[1 + 2 * g];
      *reinterpret_cast<u32x4*>(step + 16 * N + 16 * (L + g)) = v[2 + 2 * g];
    }
  }
}

// Q6_K down matrices into their resident layout (fdm_device.h): one thread
// per 210-byte block, byte by byte (made once per layer, not a hot path).
__global__ __launch_bounds__(256) void k_rel_pack_q6(const uint8_t* __restrict__ src, size_t src_stride,
                                                     uint8_t* __restrict__ dst, size_t expert_size, int n_blobs) {
  const size_t per = (size_t)kHidden * (kFfn / kQK);  // blocks per matrix
  const size_t total = per * (size_t)n_blobs;
  const size_t off = 2 * (size_t)kGateBytes;
  for (size_t k = (size_t)blockIdx.x * blockDim.x + threadIdx.x; k < total; k += (size_t)gridDim.x * blockDim.x) {
    const size_t n = k / per, kb = k % per;
    const int row = (int)(kb / (kFfn / kQK)), block = (int)(kb % (kFfn / kQK));
    const uint8_t* b = src + n * src_stride + off + (size_t)row * kQ6KRowFfn + (size_t)block * kQ6KBlock;
    uint8_t* st = dst + n * expert_size + off + rel6_step_off(row, block);
    const int bi = rel6_block_index(row, block);
    for (int h = 0; h < 2; ++h) {
      const int p = 2 * bi + h;
      for (int i = 0; i < 64; ++i) st[kRel6Ql + (i >> 4) * 2048 + 16 * p + (i & 15)] = b[64 * h + i];
      for (int i = 0; i < 32; ++i) st[kRel6Qh + (i >> 4) * 2048 + 16 * p + (i & 15)] = b[128 + 32 * h + i];
      for (int i = 0; i < 8; ++i) st[kRel6Sc + 8 * p + i] = b[192 + 8 * h + i];
    }
    st[kRel6D + 2 * bi] = b[208];
    st[kRel6D + 2 * bi + 1] = b[209];
  }
}

static unsigned grid_for_waves(size_t waves) {
  size_t wg = (waves + 3) / 4;
  const size_t cap = (size_t)(g_num_cus > 0 ? g_num_cus : 256) * 16;
  if (wg > cap) wg = cap;
  return (unsigned)(wg ? wg : 1);
}

hipError_t launch_fp16_to_fp32(const uint16_t* src, float* dst, size_t n, hipStream_t s) {
  size_t wg = (n + 255) / 256;
  const size_t cap = (size_t)(g_num_cus > 0 ? g_num_cus : 256) * 16;
  if (wg > cap) wg = cap;
  hipLaunchKernelGGL(k_fp16_to_fp32, dim3((unsigned)(wg ? wg : 1)), dim3(256), 0, s, src, dst, n);
  return hipGetLastError();
}

hipError_t launch_dequant_q4k(const uint8_t* src, float* dst, size_t n_blocks, hipStream_t s) {
  hipLaunchKernelGGL(k_dequant_q4k, dim3(grid_for_waves(n_blocks)), dim3(256), 0, s, src, dst,
                     n_blocks);
  return hipGetLastError();
}

hipError_t launch_dequant_q6k(const uint8_t* src, float* dst, size_t n_blocks, hipStream_t s) {
  hipLaunchKernelGGL(k_dequant_q6k, dim3(grid_for_waves(n_blocks)), dim3(256), 0, s, src, dst,
                     n_blocks);
  return hipGetLastError();
}

hipError_t launch_rel_pack(const uint8_t* src, size_t src_stride, uint8_t* dst, size_t expert_size,
                           int n_blobs, bool down_q6, hipStream_t s) {
  const size_t blocks = (size_t)n_blobs * (down_q6 ? 2 : 3) * 57344;
  size_t wg = (blocks + 255) / 256;
  const size_t cap = (size_t)(g_num_cus > 0 ? g_num_cus : 256) * 32;
  if (wg > cap) wg = cap;
  hipLaunchKernelGGL(k_rel_pack, dim3((unsigned)(wg ? wg : 1)), dim3(256), 0, s, src, src_stride, dst,
                     expert_size, n_blobs, down_q6 ? 0 : 1);
  if (hipError_t e = hipGetLastError()) return e;
  if (!down_q6) return hipSuccess;
  // the Q6_K down matrices: their own resident layout
  const size_t q6_blocks = (size_t)n_blobs * 57344;
  size_t wg6 = (q6_blocks + 255) / 256;
  if (wg6 > cap) wg6 = cap;
  hipLaunchKernelGGL(k_rel_pack_q6, dim3((unsigned)(wg6 ? wg6 : 1)), dim3(256), 0, s, src, src_stride, dst,
                     expert_size, n_blobs);
  return hipGetLastError();
}

}  // namespace fdm
