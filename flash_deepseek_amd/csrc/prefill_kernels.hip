// prefill_kernels.hip -- prefill of T tokens through a stack of MoE layers:
// h <- h + MoE(rms_norm(h, w_l)) per layer (rms_norm: infer.m:369-374; the
// MoE branch and residual: infer.m:1850, 1878-1922).  The experts run as a
// grouped GEMM: per distinct expert, its tokens' activations [n x 7168]
// against the expert's Q4_K rows, dequantised to bf16 in registers (the
// MFMA A operand) and contracted on v_mfma_f32_16x16x32_bf16 with fp32
// accumulation.  One MFMA K step (32) is exactly one Q4_K sub-block, so a
// step needs one (scale, min) pair per row.
//
// Routing stays exact: the router reads the fp32 normalised activations
// (bit-exact rms_norm, sequential sum as the reference's loop) through the
// same kernels as decode; only the expert GEMMs use bf16 operands.  The
// GEMM inputs x enter as a bf16 pair x = hi + lo (hi = bf16(x), lo =
// bf16(x - hi), two MFMAs): Q4_K weights carry a large common offset
// (-dmin * m per sub-block), which turns the 2^-9 rounding of a single bf16
// x into output errors of up to a few 1e-2; the pair leaves ~2^-16.  The
// weights and the SwiGLU activations are single bf16 (their rounding costs
// ~1e-3).
//
// Batched decode runs the same GEMMs at pair precision: the dequantised
// weight w enters as hi = bf16(w) and lo = bf16(w - hi) (16 significant
// bits) and every activation as a bf16 pair, contracted as hi*hi + hi*lo +
// lo*hi (three MFMAs per step; the lo*lo term is below 2^-16).  Outputs then
// carry ~1e-5 relative error, inside decode's 1e-3 bar, and each expert's
// weights are dequantised once per 32-token chunk instead of once per token.
#include "fdm_internal.h"

namespace fdm {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));

constexpr int kPTokens = 64;                       // tokens per shared-expert item and per down chunk

// One lane's share of one Q4_K block for the MFMA A operand.  Lane (c16, j)
// of a wave holds row c16 and the 32 qs bytes 32 j .. 32 j + 31, i.e. all of
// sub-blocks 2 j (low nibbles) and 2 j + 1 (high nibbles), as two whole
// 16-byte pieces of the resident expert layout (q0: bytes 32 j .. +15, q1:
// 32 j + 16 .. +31; rel_step / rel_piece), plus the block header.  The four
// lanes of a row then read one contiguous 64-byte run per instruction.
struct Q4KLane {
  u32x4 hdr;
  u32x4 q0, q1;
};

template <bool DOWN>
__device__ __forceinline__ Q4KLane q4k_lane_load(const uint8_t* mat, int row, int block, int j) {
  constexpr int N = DOWN ? kRelDnPieces : kRelGuPieces;
  const uint8_t* st = rel_step<DOWN>(mat, row, block);
  const int L = rel_piece<DOWN>(row, block, 0);
  Q4KLane r;
  r.hdr = *reinterpret_cast<const u32x4*>(st + 32 * N + 4 * L);
  r.q0 = *reinterpret_cast<const u32x4*>(st + 16 * (L + j));
  r.q1 = *reinterpret_cast<const u32x4*>(st + 16 * N + 16 * (L + j));
  return r;
}

// The lane's 8 weights of MFMA step M (0..7) of a block: sub-block
// s = 2 j + (M >> 2), elements 8 (M & 3) .. 8 (M & 3) + 7 of it, i.e. block
// elements 64 j + 32 (M >> 2) + 8 (M & 3) + 0..7 (k-piece 8 j + M of the
// block; the B operand reads the same piece), as d*sc*q - dmin*m in fp32
// after the dequant of quant.c:49-57, then bf16: hi = bf16(w) and, with PAIR,
// the remainder lo = bf16(w - hi).
struct W8 {
  bf16x8 hi, lo;
};

template <int M, bool PAIR>
__device__ __forceinline__ W8 q4k_lane_w(const Q4KLane& r, int j) {
  constexpr int H = M >> 2, R = M & 3;
  // get_scale_min_k4(s) (quant.c:26-34) on the 12 scale bytes hdr.y|z|w for
  // the lane's s = 2 j + H: byte s & 3 of each word; s >= 4 when j >= 2
  const uint32_t sh = 8u * (uint32_t)((2 * j + H) & 3);
  const uint32_t b0 = (r.hdr.y >> sh) & 0xFFu, b1 = (r.hdr.z >> sh) & 0xFFu, b2 = (r.hdr.w >> sh) & 0xFFu;
  // branch-free select (a conditional here becomes divergent branches)
  const uint32_t up = 0u - (uint32_t)(j >> 1);
  const int sc = (int)((((b2 & 0xFu) | ((b0 >> 6) << 4)) & up) | ((b0 & 63u) & ~up));
  const int m = (int)((((b2 >> 4) | ((b1 >> 6) << 4)) & up) | ((b1 & 63u) & ~up));
  const float d1 = half_to_float(r.hdr.x) * (float)sc;
  const float m1 = half_to_float(r.hdr.x >> 16) * (float)m;
  const u32x4& q = R < 2 ? r.q0 : r.q1;
  const uint32_t w0 = q[2 * (R & 1)], w1 = q[2 * (R & 1) + 1];
  uint32_t lo = H ? (w0 >> 4) & 0x0F0F0F0Fu : w0 & 0x0F0F0F0Fu;
  uint32_t hi = H ? (w1 >> 4) & 0x0F0F0F0Fu : w1 & 0x0F0F0F0Fu;
  // Opaque to the optimiser: otherwise it folds the mask into one bit-field
  // extract per nibble instead of converting bytes 1..3 in place.
  asm("" : "+v"(lo), "+v"(hi));
  f32x8 v;
  v[0] = d1 * (float)(lo & 0xFF) - m1;
  v[1] = d1 * (float)((lo >> 8) & 0xFF) - m1;
  v[2] = d1 * (float)((lo >> 16) & 0xFF) - m1;
  v[3] = d1 * (float)(lo >> 24) - m1;
  v[4] = d1 * (float)(hi & 0xFF) - m1;
  v[5] = d1 * (float)((hi >> 8) & 0xFF) - m1;
  v[6] = d1 * (float)((hi >> 16) & 0xFF) - m1;
  v[7] = d1 * (float)(hi >> 24) - m1;
  W8 o;
  o.hi = __builtin_convertvector(v, bf16x8);
  if constexpr (PAIR) o.lo = __builtin_convertvector(v - __builtin_convertvector(o.hi, f32x8), bf16x8);
  return o;
}

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// GEMM work item y of a grid: y < D: the y-th distinct routed expert (all
// its pair rows, in chunks of kPTokens); y >= 256: chunk y - 256 of the
// shared expert (tokens [64 c, 64 c + 64)).  Returns false for an empty y.
struct PItem {
  const uint8_t* blob;
  int first, count;  // B rows [first, first + count) (pair rows or shared rows)
  bool shared;
};

__device__ __forceinline__ bool prefill_item(const PrefillArgs& p, int y, PItem& it) {
  const int D = *p.n_distinct;
  if (y < 256) {
    if (y >= D) return false;
    const int e = p.distinct[y];
    it.blob = p.experts + (size_t)e * p.expert_size;
    it.first = p.seg_start[e];
    it.count = p.seg_start[e + 1] - it.first;
    it.shared = false;
    return true;
  }
  const int c = y - 256;
  if (!p.shared || c * kPTokens >= p.T) return false;
  it.blob = p.shared;
  it.first = c * kPTokens;
  it.count = min(kPTokens, p.T - it.first);
  it.shared = true;
  return true;
}

}  // namespace

// ---- rms_norm: h_post = x * (1 / sqrt(sum x^2 / d + 1e-6)) * w ---------------------------
// One workgroup per token.  The sum of squares is taken in index order by
// one thread with one fused multiply-add per element, as the reference's
// loop compiles (infer.m:369-374: clang contracts `ss += x[i]*x[i]`), so
// h_post -- and with it the routing -- is bit-exact; sqrt and division are
// IEEE.  Also
// writes the bf16 pair (hi, lo) of h_post for the expert GEMMs when xb is
// not null (hi at xb, lo at xb + T*d).
__global__ __launch_bounds__(256) void k_rms_norm(const float* __restrict__ x,
                                                  const float* __restrict__ w, float* __restrict__ o,
                                                  __bf16* __restrict__ xb, int d, float eps) {
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
    if (xb) {
      const __bf16 hi = (__bf16)v;
      xb[(size_t)blockIdx.x * d + i] = hi;
      xb[(size_t)(gridDim.x + blockIdx.x) * d + i] = (__bf16)(v - (float)hi);
    }
  }
}

// ---- grouped GEMMs: shared structure ---------------------------------------------------------
// A workgroup of kPWaves waves owns kPM = 16 kPWaves weight rows (wave w:
// rows 16 w .. 16 w + 15, the A operand built from Q4_K in registers) and
// walks the item's tokens in chunks (NB blocks of 16 tokens; only the
// chunk's non-empty blocks do work).  Per Q4_K block (256 k) the chunk's B
// tile -- NH halves (the hi/lo bf16 pair, or one) x 16 NB token rows x 256
// bf16 -- is copied global -> LDS by the waves' direct LDS loads into one of
// two buffers, so block b + 1 streams in while block b is contracted and one
// barrier per block suffices.  The next block's A words are loaded at the
// same point.
//
// LDS B rows are 512 B, unpadded; piece p (16 B, k = 8 p .. 8 p + 7) of token
// row t sits at slot p ^ (t & 15).  An MFMA read (lanes 0..15: tokens
// 16 nb + 0..15, one piece) then touches 16 distinct 16-byte bank groups.
constexpr int kPWaves = 8;
constexpr int kPM = 16 * kPWaves;                 // rows per workgroup
constexpr int kPGuTokens = 32;                    // gate/up chunk (two A operands per wave)
constexpr int kPRowB = kQK * 2;                   // LDS token row, bytes
// B offsets are 32-bit: the largest, (T K + T) activation rows of 4 KiB at
// K = 16, stays far below 4 GiB for the C API's cap of T <= 512 tokens.
static_assert((size_t)512 * 17 * kFfn * 2 < (1ull << 31), "32-bit B offsets");

// Direct LDS staging of one chunk: round k of wave w fills compact rows
// 2 (w + 8 k) and 2 (w + 8 k) + 1 of the (half, token) space (half h, token
// t < 16 NB: row h 16 NB + t); LDS row of (h, t) is h HT + t.  Rows past the
// chunk's n_tok repeat its last token (their C columns are never written).
template <int NB, int NH, int HT>
struct BDma {
  static constexpr int kRounds = NH * NB;  // 16 NB rows per half, 2 rows per wave round
  uint32_t src[kRounds];                   // lane's global byte offset in block 0
};

template <int NB, int NH, int HT>
__device__ __forceinline__ BDma<NB, NH, HT> bdma_init(const int* trow, int n_tok, uint32_t row_bytes,
                                                      uint32_t half_bytes) {
  BDma<NB, NH, HT> d;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < BDma<NB, NH, HT>::kRounds; ++k) {
    const int rho = 2 * (wave + kPWaves * k) + (lane >> 5);
    const int h = rho / (16 * NB), t = rho - h * 16 * NB;
    const uint32_t piece = (uint32_t)((lane & 31) ^ (t & 15));
    d.src[k] = h * half_bytes + (uint32_t)trow[min(t, n_tok - 1)] * row_bytes + 16u * piece;
  }
  return d;
}

// One 16-byte direct global -> LDS load per lane.  (A plain function: the
// host compilation pass rejects the builtin inside some template
// instantiations, not inside a non-template body.)
__device__ __forceinline__ void lds_dma16(const void* gsrc, void* lds_dst) {
  __builtin_amdgcn_global_load_lds(gsrc, lds_dst, 16, 0, 0);
}

template <int NB, int NH, int HT>
__device__ __forceinline__ void bdma_issue(const BDma<NB, NH, HT>& d, const __bf16* src, __bf16* buf, int b) {
  const uint8_t* base = reinterpret_cast<const uint8_t*>(src) + (size_t)b * kPRowB;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < BDma<NB, NH, HT>::kRounds; ++k) {
    const int rho0 = 2 * (wave + kPWaves * k);  // wave-uniform
    const int h = rho0 / (16 * NB), t0 = rho0 - h * 16 * NB;
    lds_dma16(base + d.src[k], reinterpret_cast<uint8_t*>(buf) + (h * HT + t0) * kPRowB);
  }
}

// The wave's direct LDS loads (and every other global load) have landed.
__device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// B operand of MFMA step M from the LDS tile: token row tok = 16 nb + c16 of
// half h, k-piece 8 j + M of the current block (the pieces q4k_lane_w<M>
// dequantises for lane j).
template <int HT>
__device__ __forceinline__ bf16x8 lds_b(const __bf16* bs, int h, int nb, int c16, int M, int j) {
  const int t = 16 * nb + c16;
  return *reinterpret_cast<const bf16x8*>(reinterpret_cast<const uint8_t*>(bs) + (h * HT + t) * kPRowB +
                                           16 * ((8 * j + M) ^ c16));
}

// ---- grouped gate/up GEMM + SwiGLU --------------------------------------------------------
// Item rows: gate AND up rows kPM tile .. +kPM-1 (two A operands per K
// step) against the item's tokens as bf16 (hi, lo) pairs; act = silu(g) * u
// goes out as bf16 rows (the B operand of the down GEMM).  One chunk of
// n_tok <= 16 NB tokens.  The two B buffers are distinct LDS arrays and the
// block loop is unrolled by two, so the compiler can tell that the reads of
// one buffer do not depend on the direct loads still landing in the other.
constexpr int kPGuBuf = 2 * kPGuTokens * kQK;  // bf16 per gate/up B buffer

template <int NB, bool PAIR>
__device__ __forceinline__ void pgateup_block(const __bf16* cur, const Q4KLane& gl, const Q4KLane& ul,
                                              f32x4 (&ag)[NB], f32x4 (&au)[NB], int c16, int j) {
#define FDM_PGU_STEP(S)                                                  \
  {                                                                      \
    const W8 ga = q4k_lane_w<S, PAIR>(gl, j), ua = q4k_lane_w<S, PAIR>(ul, j); \
    _Pragma("unroll") for (int nb = 0; nb < NB; ++nb) {                  \
      const bf16x8 bh = lds_b<kPGuTokens>(cur, 0, nb, c16, S, j);        \
      const bf16x8 bl = lds_b<kPGuTokens>(cur, 1, nb, c16, S, j);        \
      ag[nb] = mfma16(ga.hi, bl, mfma16(ga.hi, bh, ag[nb]));             \
      au[nb] = mfma16(ua.hi, bl, mfma16(ua.hi, bh, au[nb]));             \
      if constexpr (PAIR) {                                              \
        ag[nb] = mfma16(ga.lo, bh, ag[nb]);                              \
        au[nb] = mfma16(ua.lo, bh, au[nb]);                              \
      }                                                                  \
    }                                                                    \
  }                                                                      \
  __builtin_amdgcn_sched_barrier(0);
  FDM_PGU_STEP(0) FDM_PGU_STEP(1) FDM_PGU_STEP(2) FDM_PGU_STEP(3)
  FDM_PGU_STEP(4) FDM_PGU_STEP(5) FDM_PGU_STEP(6) FDM_PGU_STEP(7)
#undef FDM_PGU_STEP
}

template <int NB, bool PAIR>
__device__ __forceinline__ void pgateup_chunk(const PrefillArgs& p, const PItem& it, __bf16* bs0, __bf16* bs1,
                                              const int* trow, int t0, int n_tok) {
  constexpr int kBlocks = kHidden / kQK;  // 28, even
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane >> 4, c16 = lane & 15;
  const int arow = blockIdx.x * kPM + wave * 16 + c16;  // the lane's A row
  const uint8_t* gbase = it.blob;
  const uint8_t* ubase = it.blob + kGateBytes;
  const BDma<NB, 2, kPGuTokens> dma =
      bdma_init<NB, 2, kPGuTokens>(trow, n_tok, kHidden * 2, (uint32_t)p.T * kHidden * 2);
  f32x4 ag[NB], au[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    ag[nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    au[nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  __syncthreads();  // both buffers free: the previous chunk's last block is read
  bdma_issue(dma, p.xb, bs0, 0);
  Q4KLane gn = q4k_lane_load<false>(gbase, arow, 0, j), un = q4k_lane_load<false>(ubase, arow, 0, j);
  for (int b = 0; b < kBlocks; b += 2) {
    // Even block b from bs0 while b + 1 lands in bs1; odd block b + 1 from
    // bs1 while b + 2 lands in bs0 (the last pair re-stages block 27 into
    // the idle buffer: branch-free, so the compiler's wait counts stay exact).
    Q4KLane gl = gn, ul = un;
    wait_vm();
    __syncthreads();  // block b staged by every wave; bs1 read by all (block b - 1)
    bdma_issue(dma, p.xb, bs1, b + 1);
    gn = q4k_lane_load<false>(gbase, arow, b + 1, j);
    un = q4k_lane_load<false>(ubase, arow, b + 1, j);
    pgateup_block<NB, PAIR>(bs0, gl, ul, ag, au, c16, j);
    gl = gn;
    ul = un;
    const int b2 = min(b + 2, kBlocks - 1);
    wait_vm();
    __syncthreads();  // block b + 1 staged; bs0 read by all (block b)
    bdma_issue(dma, p.xb, bs0, b2);
    gn = q4k_lane_load<false>(gbase, arow, b2, j);
    un = q4k_lane_load<false>(ubase, arow, b2, j);
    pgateup_block<NB, PAIR>(bs1, gl, ul, ag, au, c16, j);
  }
  wait_vm();  // the re-staged copy has landed before the buffers are reused
  // C of a 16x16 block: lane (c16, j) holds token column c16, rows 4 j .. 4 j + 3.
  const int P = p.T * p.K;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int t = nb * 16 + c16;
    if (t >= n_tok) continue;
    const int orow = it.shared ? P + it.first + t0 + t : it.first + t0 + t;
    const size_t off = (size_t)orow * kFfn + blockIdx.x * kPM + wave * 16 + 4 * j;
    f32x4 a;
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = silu_mul(ag[nb][i], au[nb][i]);
    if (PAIR && p.actf) {
      *reinterpret_cast<f32x4*>(p.actf + off) = a;
      continue;
    }
    const bf16x4 hi = __builtin_convertvector(a, bf16x4);
    *reinterpret_cast<bf16x4*>(p.actb + off) = hi;
    if (PAIR)
      *reinterpret_cast<bf16x4*>(p.actb + p.act_rows * kFfn + off) =
          __builtin_convertvector(a - __builtin_convertvector(hi, f32x4), bf16x4);
  }
}

template <bool PAIR>
__device__ __forceinline__ void pgateup_body(const PrefillArgs& p, __bf16* bs0, __bf16* bs1, int* trow) {
  PItem it;
  if (!prefill_item(p, blockIdx.y, it)) return;
  for (int t0 = 0; t0 < it.count; t0 += kPGuTokens) {
    const int n_tok = min(kPGuTokens, it.count - t0);
    __syncthreads();  // the previous chunk's trow is no longer read
    if (threadIdx.x < n_tok)
      trow[threadIdx.x] = it.shared ? it.first + t0 + threadIdx.x : p.pair_tok[it.first + t0 + threadIdx.x];
    __syncthreads();
    if (n_tok > 16)
      pgateup_chunk<2, PAIR>(p, it, bs0, bs1, trow, t0, n_tok);
    else
      pgateup_chunk<1, PAIR>(p, it, bs0, bs1, trow, t0, n_tok);
  }
}

// ---- grouped down GEMM ----------------------------------------------------------------------
// Item rows: down rows kPM tile .. +kPM-1 against the item's bf16
// activation rows (contiguous; at pair precision hi and lo planes); fp32
// outputs.  Two B buffers of kPDnTok<PAIR> token rows per plane (the same
// LDS either way), as the gate/up GEMM.
template <bool PAIR>
constexpr int kPDnTok = PAIR ? kPTokens / 2 : kPTokens;  // tokens per down chunk
constexpr int kPDnBuf = kPTokens * kQK;                   // bf16 per down B buffer (both precisions)

template <int NB, bool PAIR>
__device__ __forceinline__ void pdown_block(const __bf16* cur, const Q4KLane& dl, f32x4 (&acc)[NB], int c16,
                                            int j) {
  constexpr int HT = kPDnTok<PAIR>;
#define FDM_PDN_STEP(S)                                                                  \
  {                                                                                      \
    const W8 da = q4k_lane_w<S, PAIR>(dl, j);                                            \
    _Pragma("unroll") for (int nb = 0; nb < NB; ++nb) {                                  \
      const bf16x8 bh = lds_b<HT>(cur, 0, nb, c16, S, j);                                \
      acc[nb] = mfma16(da.hi, bh, acc[nb]);                                              \
      if constexpr (PAIR) {                                                              \
        acc[nb] = mfma16(da.hi, lds_b<HT>(cur, 1, nb, c16, S, j), acc[nb]);              \
        acc[nb] = mfma16(da.lo, bh, acc[nb]);                                            \
      }                                                                                  \
    }                                                                                    \
  }                                                                                      \
  __builtin_amdgcn_sched_barrier(0);
  FDM_PDN_STEP(0) FDM_PDN_STEP(1) FDM_PDN_STEP(2) FDM_PDN_STEP(3)
  FDM_PDN_STEP(4) FDM_PDN_STEP(5) FDM_PDN_STEP(6) FDM_PDN_STEP(7)
#undef FDM_PDN_STEP
}

template <int NB, bool PAIR>
__device__ __forceinline__ void pdown_chunk(const PrefillArgs& p, const PItem& it, __bf16* bs0, __bf16* bs1,
                                            const int* trow, int row0, int n_tok) {
  constexpr int kBlocks = kFfn / kQK;  // 8, even
  constexpr int NH = PAIR ? 2 : 1, HT = kPDnTok<PAIR>;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane >> 4, c16 = lane & 15;
  const int arow = blockIdx.x * kPM + wave * 16 + c16;
  const uint8_t* dbase = it.blob + 2 * (size_t)kGateBytes;
  const BDma<NB, NH, HT> dma =
      bdma_init<NB, NH, HT>(trow, n_tok, kFfn * 2, PAIR ? (uint32_t)(p.act_rows * kFfn * 2) : 0u);
  f32x4 acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  __syncthreads();
  bdma_issue(dma, p.actb, bs0, 0);
  Q4KLane dn = q4k_lane_load<true>(dbase, arow, 0, j);
  for (int b = 0; b < kBlocks; b += 2) {
    Q4KLane dl = dn;
    wait_vm();
    __syncthreads();
    bdma_issue(dma, p.actb, bs1, b + 1);
    dn = q4k_lane_load<true>(dbase, arow, b + 1, j);
    pdown_block<NB, PAIR>(bs0, dl, acc, c16, j);
    dl = dn;
    const int b2 = min(b + 2, kBlocks - 1);
    wait_vm();
    __syncthreads();
    bdma_issue(dma, p.actb, bs0, b2);
    dn = q4k_lane_load<true>(dbase, arow, b2, j);
    pdown_block<NB, PAIR>(bs1, dl, acc, c16, j);
  }
  wait_vm();
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int t = nb * 16 + c16;
    if (t >= n_tok) continue;
    *reinterpret_cast<f32x4*>(p.eo + (size_t)(row0 + t) * kHidden + blockIdx.x * kPM + wave * 16 + 4 * j) =
        acc[nb];
  }
}

template <bool PAIR>
__device__ __forceinline__ void pdown_body(const PrefillArgs& p, __bf16* bs0, __bf16* bs1, int* trow) {
  constexpr int CT = kPDnTok<PAIR>;
  PItem it;
  if (!prefill_item(p, blockIdx.y, it)) return;
  const int P = p.T * p.K;
  const int base = it.shared ? P + it.first : it.first;  // first activation row
  for (int t0 = 0; t0 < it.count; t0 += CT) {
    const int n_tok = min(CT, it.count - t0);
    __syncthreads();
    if (threadIdx.x < n_tok) trow[threadIdx.x] = base + t0 + threadIdx.x;
    __syncthreads();
    switch ((n_tok + 15) >> 4) {
      case 1: pdown_chunk<1, PAIR>(p, it, bs0, bs1, trow, base + t0, n_tok); break;
      case 2: pdown_chunk<2, PAIR>(p, it, bs0, bs1, trow, base + t0, n_tok); break;
      case 3: if constexpr (!PAIR) pdown_chunk<3, PAIR>(p, it, bs0, bs1, trow, base + t0, n_tok); break;
      default: if constexpr (!PAIR) pdown_chunk<4, PAIR>(p, it, bs0, bs1, trow, base + t0, n_tok); break;
    }
  }
}

__global__ __launch_bounds__(kPWaves * 64) __attribute__((amdgpu_waves_per_eu(4))) void k_pgateup(
    PrefillArgs p) {
  __shared__ __attribute__((aligned(16))) __bf16 bs0[kPGuBuf];
  __shared__ __attribute__((aligned(16))) __bf16 bs1[kPGuBuf];
  __shared__ int trow[kPGuTokens];
  pgateup_body<false>(p, bs0, bs1, trow);
}
__global__ __launch_bounds__(kPWaves * 64) __attribute__((amdgpu_waves_per_eu(4))) void k_pgateup_pair(
    PrefillArgs p) {
  __shared__ __attribute__((aligned(16))) __bf16 bs0[kPGuBuf];
  __shared__ __attribute__((aligned(16))) __bf16 bs1[kPGuBuf];
  __shared__ int trow[kPGuTokens];
  pgateup_body<true>(p, bs0, bs1, trow);
}
__global__ __launch_bounds__(kPWaves * 64) __attribute__((amdgpu_waves_per_eu(4))) void k_pdown(
    PrefillArgs p) {
  __shared__ __attribute__((aligned(16))) __bf16 bs0[kPDnBuf];
  __shared__ __attribute__((aligned(16))) __bf16 bs1[kPDnBuf];
  __shared__ int trow[kPTokens];
  pdown_body<false>(p, bs0, bs1, trow);
}
__global__ __launch_bounds__(kPWaves * 64) __attribute__((amdgpu_waves_per_eu(4))) void k_pdown_pair(
    PrefillArgs p) {
  __shared__ __attribute__((aligned(16))) __bf16 bs0[kPDnBuf];
  __shared__ __attribute__((aligned(16))) __bf16 bs1[kPDnBuf];
  __shared__ int trow[kPTokens];
  pdown_body<true>(p, bs0, bs1, trow);
}

// x -> (hi, lo) bf16 pair planes
__global__ __launch_bounds__(256) void k_bf16_pair(const float* __restrict__ x, __bf16* __restrict__ xb,
                                                   size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  const __bf16 hi = (__bf16)v;
  xb[i] = hi;
  xb[n + i] = (__bf16)(v - (float)hi);
}

hipError_t launch_rms_norm(const float* x, const float* w, float* o, __bf16* xb, int T, int d,
                           hipStream_t s) {
  hipLaunchKernelGGL(k_rms_norm, dim3(T), dim3(256), 0, s, x, w, o, xb, d, 1e-6f);
  return hipGetLastError();
}

hipError_t launch_prefill_experts(const PrefillArgs& p, bool pair, hipStream_t s) {
  const int items = 256 + (p.shared ? (p.T + kPTokens - 1) / kPTokens : 0);
  if (pair)
    hipLaunchKernelGGL(k_pgateup_pair, dim3(kFfn / kPM, items), dim3(kPWaves * 64), 0, s, p);
  else
    hipLaunchKernelGGL(k_pgateup, dim3(kFfn / kPM, items), dim3(kPWaves * 64), 0, s, p);
  if (hipError_t e = hipGetLastError()) return e;
  if (pair && p.actf) return hipSuccess;  // the down runs on the dot4 kernels
  if (pair)
    hipLaunchKernelGGL(k_pdown_pair, dim3(kHidden / kPM, items), dim3(kPWaves * 64), 0, s, p);
  else
    hipLaunchKernelGGL(k_pdown, dim3(kHidden / kPM, items), dim3(kPWaves * 64), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_bf16_pair(const float* x, __bf16* xb, size_t n, hipStream_t s) {
  hipLaunchKernelGGL(k_bf16_pair, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, xb, n);
  return hipGetLastError();
}

}  // namespace fdm
