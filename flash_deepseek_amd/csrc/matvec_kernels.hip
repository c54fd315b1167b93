// matvec_kernels.hip -- activation digits and the fused dequant matvecs
// y = deq(W) . x for Q4_K and Q6_K weights: the MI355X counterparts of
// dequant_matvec_q4k / dequant_matvec_q6k (shaders.metal:43-179).
//
// Mapping (wave64).  Sixteen lanes own one output row; a wave computes four
// rows and a 256-thread workgroup sixteen.  A Q4_K row of in_dim columns has
// in_dim/64 "groups" (a quarter block: 32 qs bytes + the block header), lane
// l of the row takes groups l, l+16, l+32, ... so one 16-byte load per lane
// covers the row contiguously across the 16 lanes.  The activation digits
// of the whole x (in_dim/64 records of 208 bytes) are staged in LDS once
// per workgroup; every row of the workgroup reads them from there.  The
// 16-lane partial sums are reduced with xor shuffles.
#include "fdm_internal.h"

namespace fdm {

// One wave per 64-element group: lanes 0-31 and 32-63 are the two
// sub-blocks.
__global__ __launch_bounds__(256) void k_xdigits(const float* __restrict__ x, size_t n_groups,
                                                 XGroup* __restrict__ xd) {
  const int lane = threadIdx.x & 63;
  const size_t G = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  if (G >= n_groups) return;  // whole wave exits together
  const float v = x[G * 64 + lane];
  int8_t a, b, c;
  float s, sum;
  make_digits3(v, a, b, c, s, sum);
  XGroup* g = xd + G;
  g->a[lane] = a;
  g->b[lane] = b;
  g->c[lane] = c;
  if ((lane & 31) == 0) {
    g->s[lane >> 5] = s;
    g->xsum[lane >> 5] = sum;
  }
}

// GPL = groups per lane (in_dim / 1024) when known at compile time, 0 for
// any in_dim that is a multiple of 256.
template <int GPL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void k_matvec_q4k(const uint8_t* __restrict__ W,
                                                    const XGroup* __restrict__ xd,
                                                    float* __restrict__ y, int rows, int gr) {
  extern __shared__ XGroup xs[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = blockIdx.x * 16 + wave * 4 + (lane >> 4);
  const int l16 = lane & 15, g = l16 & 3;
  const Q4KScaleSel sel = q4k_scale_sel(g);
  float acc = 0.0f;
  if constexpr (GPL > 0) {
    // the digit records first, then the weights: the records land first
    XStage<16 * GPL> st;
    st.load(xd, gr);
    u32x4 hdr[GPL], q0[GPL], q1[GPL];
    const uint8_t* rp = W + (size_t)min(row, rows - 1) * (size_t)(gr >> 2) * kQ4KBlock;
#pragma unroll
    for (int t = 0; t < GPL; ++t) {
      const uint8_t* bp = rp + (size_t)(4 * t + (l16 >> 2)) * kQ4KBlock;
      hdr[t] = *reinterpret_cast<const u32x4_a4*>(bp);
      q0[t] = *reinterpret_cast<const u32x4_a4*>(bp + 16 + 32 * g);
      q1[t] = *reinterpret_cast<const u32x4_a4*>(bp + 32 + 32 * g);
    }
    st.store(xs, gr);
    __syncthreads();
    if (row < rows) {
#pragma unroll
      for (int t = 0; t < GPL; ++t) {
        acc += q4k_group_dot(hdr[t], q0[t], q1[t], sel, &xs[16 * t + l16]);
        // keep each group's LDS reads next to its math (bounds live registers)
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  } else {
    xstage_copy(xs, xd, gr);
    __syncthreads();
    if (row < rows) {
      const uint8_t* rp = W + (size_t)row * (size_t)(gr >> 2) * kQ4KBlock;
      for (int G = l16; G < gr; G += 16) {
        const uint8_t* bp = rp + (size_t)(G >> 2) * kQ4KBlock;
        const u32x4 hdr = *reinterpret_cast<const u32x4_a4*>(bp);
        const u32x4 q0 = *reinterpret_cast<const u32x4_a4*>(bp + 16 + 32 * g);
        const u32x4 q1 = *reinterpret_cast<const u32x4_a4*>(bp + 32 + 32 * g);
        acc += q4k_group_dot(hdr, q0, q1, sel, &xs[G]);
      }
    }
  }
  acc = sum16(acc);
  if (row < rows && l16 == 0) y[row] = acc;
}

// Load the n dwords starting at byte address p (p is 2-byte aligned) into
// out[0..n), reading only dword-aligned words inside [p - 2, p + 4n + 2).
template <int N>
__device__ __forceinline__ void load_realigned(const uint8_t* p, uint32_t* out) {
  const uintptr_t addr = reinterpret_cast<uintptr_t>(p);
  const uint32_t sh = addr & 3u;
  const uint32_t* a = reinterpret_cast<const uint32_t*>(addr - sh);
  uint32_t w[N + 1];
#pragma unroll
  for (int i = 0; i < N; ++i) w[i] = a[i];
  w[N] = sh ? a[N] : 0u;
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = funnel(w[i], w[i + 1], sh);
}

// One 128-element half (h) of the Q6_K block at `blk`; xg points at the
// two XGroups of the half's activations.  Returns the half's dot product.
__device__ __forceinline__ float q6k_half(const uint8_t* blk, int h,
                                          const XGroup* __restrict__ xg) {
  uint32_t ql[16], qh[8], sc[2];
  load_realigned<16>(blk + 64 * h, ql);
  load_realigned<8>(blk + 128 + 32 * h, qh);
  const uint16_t* s16 = reinterpret_cast<const uint16_t*>(blk + 192 + 8 * h);
  sc[0] = (uint32_t)s16[0] | ((uint32_t)s16[1] << 16);
  sc[1] = (uint32_t)s16[2] | ((uint32_t)s16[3] << 16);
  const float d = half_to_float(*reinterpret_cast<const uint16_t*>(blk + 208));
  return d * q6k_half_dot(ql, qh, sc, xg, xg + 1);
}

// Q6_K: a lane owns 128-element halves of blocks; half-blocks per row =
// in_dim / 128, lane l of the row takes halves l, l+16, ...
template <int HPL>
__global__ __launch_bounds__(256) void k_matvec_q6k(const uint8_t* __restrict__ W,
                                                    const XGroup* __restrict__ xd,
                                                    float* __restrict__ y, int rows, int gr) {
  extern __shared__ XGroup xs[];
  xstage_copy(xs, xd, gr);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = blockIdx.x * 16 + wave * 4 + (lane >> 4);
  const int l16 = lane & 15;
  const int hr = gr >> 1;  // halves per row
  float acc = 0.0f;
  if (row < rows) {
    const uint8_t* rp = W + (size_t)row * (size_t)(gr >> 2) * kQ6KBlock;
    if constexpr (HPL > 0) {
#pragma unroll
      for (int t = 0; t < HPL; ++t) {
        const int hb = 16 * t + l16;
        acc += q6k_half(rp + (size_t)(hb >> 1) * kQ6KBlock, hb & 1, &xs[2 * hb]);
      }
    } else {
      for (int hb = l16; hb < hr; hb += 16)
        acc += q6k_half(rp + (size_t)(hb >> 1) * kQ6KBlock, hb & 1, &xs[2 * hb]);
    }
  }
  acc = sum16(acc);
  if (row < rows && l16 == 0) y[row] = acc;
}

hipError_t launch_xdigits(const float* x, size_t n_groups, XGroup* xd, hipStream_t s) {
  const size_t wg = (n_groups + 3) / 4;
  hipLaunchKernelGGL(k_xdigits, dim3((unsigned)wg), dim3(256), 0, s, x, n_groups, xd);
  return hipGetLastError();
}

hipError_t launch_matvec_q4k(const uint8_t* W, const XGroup* xd, float* y, int rows, int in_dim,
                             hipStream_t s) {
  const int gr = in_dim / 64;
  const dim3 grid((rows + 15) / 16), block(256);
  const size_t lds = (size_t)gr * sizeof(XGroup);
  if (in_dim == 7168)
    hipLaunchKernelGGL(k_matvec_q4k<7>, grid, block, lds, s, W, xd, y, rows, gr);
  else if (in_dim == 2048)
    hipLaunchKernelGGL(k_matvec_q4k<2>, grid, block, lds, s, W, xd, y, rows, gr);
  else
    hipLaunchKernelGGL(k_matvec_q4k<0>, grid, block, lds, s, W, xd, y, rows, gr);
  return hipGetLastError();
}

hipError_t launch_matvec_q6k(const uint8_t* W, const XGroup* xd, float* y, int rows, int in_dim,
                             hipStream_t s) {
  const int gr = in_dim / 64;
  const dim3 grid((rows + 15) / 16), block(256);
  const size_t lds = (size_t)gr * sizeof(XGroup);
  if (in_dim == 2048)
    hipLaunchKernelGGL(k_matvec_q6k<1>, grid, block, lds, s, W, xd, y, rows, gr);
  else
    hipLaunchKernelGGL(k_matvec_q6k<0>, grid, block, lds, s, W, xd, y, rows, gr);
  return hipGetLastError();
}

}  // namespace fdm
