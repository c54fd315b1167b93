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

// ---- one launch (Q6_K): the digits of x, then the rows -------------------------------
// Work list of 128-thread workgroups: [digit items: two 64-element groups
// each, one per wave] [row items: 8 rows each, 16 lanes per row].  A row
// item requests its weights first, then waits for the digit flag (set by
// the last digit item to arrive), stages the records with coherent 16-byte
// loads and finishes; the digits' latency hides behind the weight loads and
// no second launch is paid.  Digit items never wait, so the grid drains
// whatever the dispatch order; the flag wait is bounded as well (a wait that
// gives up records the epoch in the error flag, which fdm_stream_sync reports).

__device__ __forceinline__ int mv_digit_items(int gr) { return (gr + 1) / 2; }

__device__ __forceinline__ void mv_digit_item(const MatvecArgs& a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = 2 * blockIdx.x + wave;
  if (G < a.gr) publish_digit_group(a.x[64 * G + lane], a.xd + G);
  wait_stores_done();
  __syncthreads();
  if (threadIdx.x == 0 && arrive_agent(a.counter) == mv_digit_items(a.gr) - 1) {
    reset_agent(a.counter);
    store_u32_agent(a.flag, a.epoch);
  }
}

// Thread 0 polls the digit flag; every thread returns after it is set (or
// after the bounded wait gave up).
__device__ __forceinline__ void mv_wait_digits(const MatvecArgs& a) {
  if (threadIdx.x == 0) {
    for (unsigned n = 0; load_u32_agent(a.flag) != a.epoch; ++n) {
      if (n >= a.spin_limit || ((n & 63) == 63 && load_u32_agent(a.err) == a.epoch)) {
        store_u32_agent(a.err, a.epoch);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  __syncthreads();
}

// The first n records of a.xd into LDS: every 16-byte load (coherent, sc1)
// is issued before the first store.
template <int N>
__device__ __forceinline__ void mv_stage(const MatvecArgs& a, XGroup* xs) {
  constexpr int kVec = N * (int)sizeof(XGroup) / 16;
  constexpr int kPer = (kVec + 127) / 128;
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.xd, 0, N * (int)sizeof(XGroup), 0x00020000);
  u32x4 v[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) v[k] = __builtin_amdgcn_raw_buffer_load_b128(r, (threadIdx.x + 128 * k) * 16, 0, 16);
#pragma unroll
  for (int k = 0; k < kPer; ++k)
    if (threadIdx.x + 128 * k < kVec) reinterpret_cast<u32x4*>(xs)[threadIdx.x + 128 * k] = v[k];
  __syncthreads();
}

// Q6_K, in_dim = 2048 HPL: lane l16 of a row takes 128-element halves l16 + 16 t.
template <int HPL>
__global__ __launch_bounds__(128) void k_matvec1_q6k(MatvecArgs a) {
  __shared__ XGroup xs[32 * HPL];
  const int nd = mv_digit_items(a.gr);
  if ((int)blockIdx.x < nd) {
    mv_digit_item(a);
    return;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = 8 * ((int)blockIdx.x - nd) + 4 * wave + (lane >> 4);
  const int l16 = lane & 15;
  const uint8_t* rp = a.W + (size_t)min(row, a.rows - 1) * (size_t)(a.gr / 4) * kQ6KBlock;
  Q6KHalfLoad l6[HPL];
#pragma unroll
  for (int t = 0; t < HPL; ++t) {
    const int hb = 16 * t + l16;
    l6[t] = q6k_load_half(rp + (size_t)(hb >> 1) * kQ6KBlock, hb & 1);
  }
  mv_wait_digits(a);
  mv_stage<32 * HPL>(a, xs);
  float acc = 0.0f;
#pragma unroll
  for (int t = 0; t < HPL; ++t) {
    acc += q6k_half_dot_ld(l6[t], &xs[2 * (16 * t + l16)]);
    __builtin_amdgcn_sched_barrier(0);
  }
  acc = sum16(acc);
  if (row < a.rows && l16 == 0) a.y[row] = acc;
}

bool matvec1_supported(bool q6, int in_dim) {
  return q6 && in_dim % 2048 == 0 && in_dim / 2048 >= 1 && in_dim / 2048 <= 3;
}

hipError_t launch_matvec1(const MatvecArgs& a, bool q6, hipStream_t s) {
  if (!q6) return hipErrorInvalidValue;  // Q4_K takes the column-part kernel below
  const dim3 grid((unsigned)((a.gr + 1) / 2 + (a.rows + 7) / 8)), block(128);
  switch (a.gr * 64 / 2048) {
    case 1: hipLaunchKernelGGL(k_matvec1_q6k<1>, grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL(k_matvec1_q6k<2>, grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL(k_matvec1_q6k<3>, grid, block, 0, s, a); break;
  }
  return hipGetLastError();
}

// ---- one launch by column parts (Q4_K, in_dim = 1024 P) -------------------------------
// Items of 256 threads, part-major: (part p, 16-row block).  (Row-block-major
// order, where a row block's P items read its whole rows together, measured
// no faster.)  An item turns its
// part's 1024 activations into digit records itself (4 KB of x: no hand-off
// before the math), contracts its 16 rows x 4 blocks (16 lanes per row, one
// 64-element group each) and publishes each row's partial sum as a tagged
// word.  The items of the last part then take the earlier parts' partials of
// their rows (bounded waits; those items precede them in the list) and write
// y = ((p_0 + p_1) + ...) + p_(P-1).
template <int P>
__global__ __launch_bounds__(256) void k_matvec2_q4k(Matvec2Args a) {
  __shared__ XGroup xs[16];
  __shared__ float own[16];
  const int nb = (a.rows + 15) / 16;
  const int p = blockIdx.x / nb, rb = blockIdx.x - p * nb;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = 16 * rb + 4 * wave + (lane >> 4);
  const int l16 = lane & 15, g = l16 & 3;
  const uint8_t* bp = a.W + ((size_t)min(row, a.rows - 1) * (4 * P) + 4 * p + (l16 >> 2)) * kQ4KBlock;
  // x before the weights: loads return in order, so the digits are made
  // while the weights are still in flight
  float xv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) xv[i] = a.x[1024 * p + 64 * (4 * wave + i) + lane];
  const Q4KGroupLoad ld = q4k_load_group(bp, g);
#pragma unroll
  for (int i = 0; i < 4; ++i) digits_to_lds(xv[i], xs[4 * wave + i]);
  __syncthreads();
  const float acc = sum16(q4k_group_dot_ld(ld, q4k_scale_sel(g), &xs[l16]));
  if (p < P - 1) {
    if (l16 == 0 && row < a.rows) put_tagged(a.part + (size_t)p * a.rows + row, a.epoch, __float_as_uint(acc));
    return;
  }
  if (l16 == 0) own[4 * wave + (lane >> 4)] = acc;
  __syncthreads();
  const int r = 16 * rb + (int)threadIdx.x;
  if (threadIdx.x >= 16 || r >= a.rows) return;
  // the earlier parts' partials of row r: every load in flight at once,
  // again for those not yet published
  uint64_t v[P > 1 ? P - 1 : 1];
#pragma unroll
  for (int q = 0; q < P - 1; ++q) v[q] = get_tagged(a.part + (size_t)q * a.rows + r);
  for (unsigned n = 0;; ++n) {
    bool all = true;
#pragma unroll
    for (int q = 0; q < P - 1; ++q) all = all && tag_is(v[q], a.epoch);
    if (all) break;
    if (n >= a.spin_limit || ((n & 63) == 63 && load_u32_agent(a.err) == a.epoch)) {
      store_u32_agent(a.err, a.epoch);
      break;
    }
    __builtin_amdgcn_s_sleep(2);
#pragma unroll
    for (int q = 0; q < P - 1; ++q)
      if (!tag_is(v[q], a.epoch)) v[q] = get_tagged(a.part + (size_t)q * a.rows + r);
  }
  float sum = 0.0f;
#pragma unroll
  for (int q = 0; q < P - 1; ++q) sum = q == 0 ? tagged_f(v[q]) : sum + tagged_f(v[q]);
  a.y[r] = P == 1 ? own[threadIdx.x] : sum + own[threadIdx.x];
}

// ---- one launch in fp32 (Q4_K, in_dim = 1024, 2048 or 7168) -----------------------------
// (Measured on MI355X, 2048 x 7168: 5.3 us against 6.7 us for the
// column-part digit kernel below; a row over two waves, 6.1 us.)
// No activation digits and no hand-off between workgroups: at batch 1 a
// single matvec is latency-bound (8 MB streams in ~1.4 us), and the digit
// records (each workgroup making the digits of its columns, then a second
// round trip to add the column parts) cost more than the math they save.
// Here every workgroup stages the whole x in LDS once (with each 32-element
// sub-block's fp32 sum for the Q4_K min term; 16 bytes of padding per
// 64-element group, so the lanes of a wave, one group each, read distinct
// banks), and each row is contracted by
// LPR lanes in fp32: lane i of a row takes the row's 64-element groups
// i, i + LPR, ..; a group's 32 qs bytes are two sub-blocks (low nibbles:
// elements 0-31, high: 32-63), each dotted with x as sum_k q_k x_k in fp32
// (the nibbles widened two at a time by the fp8 conversion), then
//   d (sc0 S0 + sc1 S1) - dmin (m0 X0 + m1 X1)
// as dequant_matvec_q4k (shaders.metal:43-99) in fp32; the row's lane
// partials are added by DPP into its first lane.  All loads of a workgroup
// (its rows' weights and x) are issued before any math.
template <int LPR, int GPL, int NG>
__global__ __launch_bounds__(256) void k_matvec3_q4k(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                     float* __restrict__ y, int rows) {
  constexpr int ng = NG;
  extern __shared__ float xsh[];  // x, 68 floats per 64-element group (bank padding), then the sub-block sums [2 ng]
  float* xss = xsh + kXPad * ng;
  static_assert(LPR == 16 || LPR == 32 || LPR == 64, "lanes per row");
  constexpr int RPW = 64 / LPR;  // rows per wave
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane % LPR;
  const int row = blockIdx.x * (4 * RPW) + wave * RPW + lane / LPR;
  const int rr = min(row, rows - 1);
  const int g = li & 3;
  // x first (its LDS copy waits for these loads only), then the weights of
  // the lane's groups (clamped: groups past the row load a valid group and
  // contribute 0); each group's math waits for its own loads
  constexpr int kNv = 16 * NG / 256;  // float4s of x per thread
  static_assert(kNv * 256 == 16 * NG, "x in whole 256-thread steps");
  f32x4 xv[kNv];
#pragma unroll
  for (int i = 0; i < kNv; ++i) xv[i] = reinterpret_cast<const f32x4*>(x)[threadIdx.x + 256 * i];
  Q4KGroupLoad ld[GPL];
#pragma unroll
  for (int k = 0; k < GPL; ++k) {
    const int G = min(li + k * LPR, ng - 1);
    ld[k] = q4k_load_group(W + ((size_t)rr * (ng >> 2) + (G >> 2)) * kQ4KBlock, g);
  }
  // x into LDS; each sub-block's sum by the eight threads that hold it
#pragma unroll
  for (int i = 0; i < kNv; ++i) {
    const int v = threadIdx.x + 256 * i;
    *reinterpret_cast<f32x4*>(xsh + kXPad * (v >> 4) + 4 * (v & 15)) = xv[i];
    float sb = (xv[i].x + xv[i].y) + (xv[i].z + xv[i].w);
    sb = sb + dpp_row_shl<1>(sb);
    sb = sb + dpp_row_shl<2>(sb);
    sb = sb + dpp_row_shl<4>(sb);
    if ((v & 7) == 0) xss[v >> 3] = sb;
  }
  __syncthreads();
  const float qscale = q4k_fp8_qscale();
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < GPL; ++k) {
    const int G = li + k * LPR, Gc = min(G, ng - 1);
    const float part = q4k_group_dot_f32(ld[k], q4k_quad_hdr(ld[k]), g, xsh + kXPad * Gc, xss[2 * Gc],
                                         xss[2 * Gc + 1], qscale);
    acc += G < ng ? part : 0.0f;
  }
  // the row's LPR lanes into its first lane
  if constexpr (LPR == 64) {
    acc = wave_sum_lane0(acc);
  } else {
    // LPR = 32: rows 1 and 3 of 16 lanes into rows 0 and 2 (permlane16_swap)
    if constexpr (LPR == 32)
      acc = acc + __uint_as_float(__builtin_amdgcn_permlane16_swap(__float_as_uint(acc), __float_as_uint(acc), false, false)[1]);
    acc = sum16(acc);
  }
  if (li == 0 && row < rows) y[row] = acc;
}

bool matvec3_supported(int in_dim) { return in_dim == 1024 || in_dim == 2048 || in_dim == 7168; }

hipError_t launch_matvec3_q4k(const uint8_t* W, const float* x, float* y, int rows, int in_dim, hipStream_t s) {
  const int ng = in_dim / 64;
  const size_t lds = (size_t)ng * kXPad * 4 + (size_t)ng * 2 * 4;
  if (in_dim == 7168) {
    hipLaunchKernelGGL((k_matvec3_q4k<64, 2, 112>), dim3((rows + 3) / 4), dim3(256), lds, s, W, x, y, rows);
  } else if (in_dim == 2048) {
    hipLaunchKernelGGL((k_matvec3_q4k<32, 1, 32>), dim3((rows + 7) / 8), dim3(256), lds, s, W, x, y, rows);
  } else if (in_dim == 1024) {
    hipLaunchKernelGGL((k_matvec3_q4k<16, 1, 16>), dim3((rows + 15) / 16), dim3(256), lds, s, W, x, y, rows);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

bool matvec2_supported(int in_dim, int rows, size_t part_words) {
  const int P = in_dim / 1024;
  return in_dim % 1024 == 0 && P >= 1 && P <= 7 && (size_t)(P - 1) * (size_t)rows <= part_words;
}

hipError_t launch_matvec2_q4k(const Matvec2Args& a, int in_dim, hipStream_t s) {
  const int P = in_dim / 1024;
  const dim3 grid((unsigned)(P * ((a.rows + 15) / 16))), block(256);
  switch (P) {
    case 1: hipLaunchKernelGGL(k_matvec2_q4k<1>, grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL(k_matvec2_q4k<2>, grid, block, 0, s, a); break;
    case 3: hipLaunchKernelGGL(k_matvec2_q4k<3>, grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL(k_matvec2_q4k<4>, grid, block, 0, s, a); break;
    case 5: hipLaunchKernelGGL(k_matvec2_q4k<5>, grid, block, 0, s, a); break;
    case 6: hipLaunchKernelGGL(k_matvec2_q4k<6>, grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL(k_matvec2_q4k<7>, grid, block, 0, s, a); break;
  }
  return hipGetLastError();
}

}  // namespace fdm
