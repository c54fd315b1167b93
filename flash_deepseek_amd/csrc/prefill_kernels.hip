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
#include "fdm_internal.h"

namespace fdm {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));

constexpr int kPTokens = 64;                       // tokens per GEMM item (4 N blocks)
constexpr int kPNBlocks = kPTokens / 16;
constexpr int kPGuTile = 64;                       // gate (and up) rows per gate/up workgroup
constexpr int kPDnTile = 64;                       // down rows per down workgroup

// One lane's share of one Q4_K block for the MFMA A operand: the header and
// the 8 qs bytes of each 64-element group that hold the lane's elements
// (k = 32 s + 8 j .. +8 of sub-block s, j = lane / 16: bytes 32 (s/2) + 8 j,
// low nibbles for even s, high for odd s).
struct Q4KLane {
  u32x4 hdr;
  uint2 qs[4];
};

__device__ __forceinline__ Q4KLane q4k_lane_load(const uint8_t* blk, int j) {
  Q4KLane r;
  r.hdr = *reinterpret_cast<const u32x4_a4*>(blk);
#pragma unroll
  for (int g = 0; g < 4; ++g) r.qs[g] = *reinterpret_cast<const uint2*>(blk + 16 + 32 * g + 8 * j);
  return r;
}

// The lane's 8 weights of sub-block S as bf16 (d*sc*q - dmin*m, rounded once
// to bf16 after the fp32 dequant of quant.c:49-57).
template <int S>
__device__ __forceinline__ bf16x8 q4k_lane_bf16(const Q4KLane& r) {
  const uint32_t s0 = r.hdr.y, s1 = r.hdr.z, s2 = r.hdr.w;
  // get_scale_min_k4(S) (quant.c:26-34) on the 12 scale bytes s0|s1|s2
  int sc, m;
  if (S < 4) {
    sc = (int)((s0 >> (8 * S)) & 63u);
    m = (int)((s1 >> (8 * S)) & 63u);
  } else {
    const uint32_t b = (s2 >> (8 * (S - 4))) & 0xFFu;
    sc = (int)((b & 0xFu) | (((s0 >> (8 * (S - 4))) >> 6 & 3u) << 4));
    m = (int)((b >> 4) | (((s1 >> (8 * (S - 4))) >> 6 & 3u) << 4));
  }
  const float d1 = half_to_float(r.hdr.x) * (float)sc;
  const float m1 = half_to_float(r.hdr.x >> 16) * (float)m;
  const uint2 w = r.qs[S >> 1];
  const uint32_t lo = (S & 1) ? (w.x >> 4) & 0x0F0F0F0Fu : w.x & 0x0F0F0F0Fu;
  const uint32_t hi = (S & 1) ? (w.y >> 4) & 0x0F0F0F0Fu : w.y & 0x0F0F0F0Fu;
  f32x8 v;
  v[0] = d1 * (float)(lo & 0xFF) - m1;
  v[1] = d1 * (float)((lo >> 8) & 0xFF) - m1;
  v[2] = d1 * (float)((lo >> 16) & 0xFF) - m1;
  v[3] = d1 * (float)(lo >> 24) - m1;
  v[4] = d1 * (float)(hi & 0xFF) - m1;
  v[5] = d1 * (float)((hi >> 8) & 0xFF) - m1;
  v[6] = d1 * (float)((hi >> 16) & 0xFF) - m1;
  v[7] = d1 * (float)(hi >> 24) - m1;
  return __builtin_convertvector(v, bf16x8);
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
// one thread, as the reference's loop (infer.m:369-374), so h_post -- and
// with it the routing -- is bit-exact; sqrt and division are IEEE.  Also
// writes the bf16 pair (hi, lo) of h_post for the expert GEMMs when xb is
// not null (hi at xb, lo at xb + T*d).
__global__ __launch_bounds__(256) void k_rms_norm(const float* __restrict__ x,
                                                  const float* __restrict__ w, float* __restrict__ o,
                                                  __bf16* __restrict__ xb, int d, float eps) {
#pragma clang fp contract(off)
  __shared__ float row[kHidden];
  __shared__ float inv_s;
  const float* xr = x + (size_t)blockIdx.x * d;
  for (int i = threadIdx.x; i < d; i += 256) row[i] = xr[i];
  __syncthreads();
  if (threadIdx.x == 0) {
    float ss = 0.0f;
    for (int i = 0; i < d; ++i) ss += row[i] * row[i];
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

// ---- grouped gate/up GEMM + SwiGLU --------------------------------------------------------
// Workgroup (tile, y): rows 64 tile .. +63 of gate AND up of item y; wave w
// owns rows 16 w .. 16 w + 15 of both (two A operands per K step) and all
// the item's tokens, 64 at a time (4 N blocks).  act = silu(g) * u goes out
// as bf16 rows (the B operand of the down GEMM).
__global__ __launch_bounds__(256) void k_pgateup(PrefillArgs p) {
  PItem it;
  if (!prefill_item(p, blockIdx.y, it)) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane >> 4, c16 = lane & 15;
  const int r = blockIdx.x * kPGuTile + wave * 16 + c16;  // the lane's A row
  const uint8_t* grow = it.blob + (size_t)r * kQ4KRowHidden;
  const uint8_t* urow = it.blob + kGateBytes + (size_t)r * kQ4KRowHidden;
  const int P = p.T * p.K;
  for (int t0 = 0; t0 < it.count; t0 += kPTokens) {
    // B rows of the 4 N blocks: token (or pair) row of column c16
    const __bf16* brow[kPNBlocks];
    bool bval[kPNBlocks];
    const size_t lo_off = (size_t)p.T * kHidden;  // lo half of the pair
#pragma unroll
    for (int nb = 0; nb < kPNBlocks; ++nb) {
      const int t = t0 + nb * 16 + c16;
      bval[nb] = t < it.count;
      const int tok = !bval[nb] ? 0 : it.shared ? it.first + t : p.pair_tok[it.first + t];
      brow[nb] = p.xb + (size_t)tok * kHidden + 8 * j;
    }
    f32x4 ag[kPNBlocks], au[kPNBlocks];
#pragma unroll
    for (int nb = 0; nb < kPNBlocks; ++nb) {
      ag[nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      au[nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    for (int b = 0; b < kHidden / kQK; ++b) {
      const Q4KLane gl = q4k_lane_load(grow + b * kQ4KBlock, j);
      const Q4KLane ul = q4k_lane_load(urow + b * kQ4KBlock, j);
#define FDM_PGU_STEP(S)                                                                   \
  {                                                                                       \
    const bf16x8 ga = q4k_lane_bf16<S>(gl), ua = q4k_lane_bf16<S>(ul);                    \
    _Pragma("unroll") for (int nb = 0; nb < kPNBlocks; ++nb) {                            \
      bf16x8 bh = {}, bl = {};                                                            \
      if (bval[nb]) {                                                                     \
        const __bf16* q_ = brow[nb] + b * kQK + 32 * (S);                                 \
        bh = *reinterpret_cast<const bf16x8*>(q_);                                        \
        bl = *reinterpret_cast<const bf16x8*>(q_ + lo_off);                               \
      }                                                                                   \
      ag[nb] = mfma16(ga, bl, mfma16(ga, bh, ag[nb]));                                    \
      au[nb] = mfma16(ua, bl, mfma16(ua, bh, au[nb]));                                    \
    }                                                                                     \
  }
      FDM_PGU_STEP(0) FDM_PGU_STEP(1) FDM_PGU_STEP(2) FDM_PGU_STEP(3)
      FDM_PGU_STEP(4) FDM_PGU_STEP(5) FDM_PGU_STEP(6) FDM_PGU_STEP(7)
#undef FDM_PGU_STEP
    }
    // C of a 16x16 block: lane (c16, j) holds token column c16, rows 4 j .. 4 j + 3
#pragma unroll
    for (int nb = 0; nb < kPNBlocks; ++nb) {
      const int t = t0 + nb * 16 + c16;
      if (t >= it.count) continue;
      const int orow = it.shared ? P + it.first + t : it.first + t;
      bf16x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = (__bf16)silu_mul(ag[nb][i], au[nb][i]);
      *reinterpret_cast<bf16x4*>(p.actb + (size_t)orow * kFfn + blockIdx.x * kPGuTile + wave * 16 +
                                 4 * j) = o;
    }
  }
}

// ---- grouped down GEMM ----------------------------------------------------------------------
// Workgroup (tile, y): down rows 64 tile .. +63 of item y (wave w: rows
// 16 w .. +15) against the item's bf16 activation rows; fp32 outputs.
__global__ __launch_bounds__(256) void k_pdown(PrefillArgs p) {
  PItem it;
  if (!prefill_item(p, blockIdx.y, it)) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane >> 4, c16 = lane & 15;
  const int r = blockIdx.x * kPDnTile + wave * 16 + c16;
  const uint8_t* drow = it.blob + 2 * (size_t)kGateBytes + (size_t)r * kQ4KRowFfn;
  const int P = p.T * p.K;
  const int base = it.shared ? P + it.first : it.first;  // first activation row
  for (int t0 = 0; t0 < it.count; t0 += kPTokens) {
    const __bf16* brow[kPNBlocks];
    bool bval[kPNBlocks];
#pragma unroll
    for (int nb = 0; nb < kPNBlocks; ++nb) {
      const int t = t0 + nb * 16 + c16;
      bval[nb] = t < it.count;
      brow[nb] = p.actb + (size_t)(bval[nb] ? base + t : 0) * kFfn + 8 * j;
    }
    f32x4 acc[kPNBlocks];
#pragma unroll
    for (int nb = 0; nb < kPNBlocks; ++nb) acc[nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int b = 0; b < kFfn / kQK; ++b) {
      const Q4KLane dl = q4k_lane_load(drow + b * kQ4KBlock, j);
#define FDM_PDN_STEP(S)                                                                   \
  {                                                                                       \
    const bf16x8 da = q4k_lane_bf16<S>(dl);                                               \
    _Pragma("unroll") for (int nb = 0; nb < kPNBlocks; ++nb) {                            \
      bf16x8 bv = {};                                                                     \
      if (bval[nb]) bv = *reinterpret_cast<const bf16x8*>(brow[nb] + b * kQK + 32 * (S)); \
      acc[nb] = mfma16(da, bv, acc[nb]);                                                  \
    }                                                                                     \
  }
      FDM_PDN_STEP(0) FDM_PDN_STEP(1) FDM_PDN_STEP(2) FDM_PDN_STEP(3)
      FDM_PDN_STEP(4) FDM_PDN_STEP(5) FDM_PDN_STEP(6) FDM_PDN_STEP(7)
#undef FDM_PDN_STEP
    }
#pragma unroll
    for (int nb = 0; nb < kPNBlocks; ++nb) {
      const int t = t0 + nb * 16 + c16;
      if (t >= it.count) continue;
      *reinterpret_cast<f32x4*>(p.eo + (size_t)(base + t) * kHidden + blockIdx.x * kPDnTile +
                                wave * 16 + 4 * j) = acc[nb];
    }
  }
}

hipError_t launch_rms_norm(const float* x, const float* w, float* o, __bf16* xb, int T, int d,
                           hipStream_t s) {
  hipLaunchKernelGGL(k_rms_norm, dim3(T), dim3(256), 0, s, x, w, o, xb, d, 1e-6f);
  return hipGetLastError();
}

hipError_t launch_prefill_experts(const PrefillArgs& p, hipStream_t s) {
  const int items = 256 + (p.shared ? (p.T + kPTokens - 1) / kPTokens : 0);
  hipLaunchKernelGGL(k_pgateup, dim3(kFfn / kPGuTile, items), dim3(256), 0, s, p);
  if (hipError_t e = hipGetLastError()) return e;
  hipLaunchKernelGGL(k_pdown, dim3(kHidden / kPDnTile, items), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace fdm
