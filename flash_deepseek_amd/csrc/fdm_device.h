// fdm_device.h -- device-side building blocks shared by the gfx950 kernels.
//
// Activation digits.  A matvec against K-quant weights does, per weight, a
// nibble (or 6-bit) unpack and a multiply-accumulate.  Done in fp32 that is
// ~2.4 VALU instructions per weight, which at 8 TB/s of 4.5-bit weights
// would keep the vector ALUs of all 256 CUs almost fully busy.  Instead the
// activation vector x is split once per 32-element sub-block j into three
// int8 "digits" against a power-of-two scale s_j (the smallest with
// max|x| / s_j <= 127, so x / s_j is exact):
//   t = x / s_j,  a = rint(t),  b = rint((t - a) * 254),
//   c = rint(((t - a) * 254 - b) * 254),
//   x ~= s_j * (a + b / 254 + c / 254^2),  |x - x'| <= s_j / 129032
// i.e. at most max|x| * 2^-23 per element: the precision of an fp32 product
// relative to the sub-block's largest element.  The weights' integer quants
// meet the digits in v_dot4_i32_i8 (four 8-bit products per instruction,
// exact int32 sums), and the block scales are applied once per sub-block in
// fp32.  The sub-block sums sum_j x (exact fp32 order) carry the Q4_K min
// term.
//
// Digits of 64 consecutive elements live in one 208-byte record (XGroup),
// matching one Q4_K "group" (32 qs bytes = sub-blocks 2g and 2g+1).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fdm {

constexpr int kQK = 256;
constexpr int kQ4KBlock = 144;
constexpr int kQ6KBlock = 210;
constexpr int kHidden = 7168;
constexpr int kFfn = 2048;
constexpr int kGateBytes = 57344 * kQ4KBlock;       // 8,257,536
constexpr int kDownQ4KBytes = 57344 * kQ4KBlock;    // 8,257,536
constexpr int kDownQ6KBytes = 57344 * kQ6KBlock;    // 12,042,240
constexpr int kQ4KRowHidden = kHidden / kQK * kQ4KBlock;  // 4032 B: gate/up row
constexpr int kQ4KRowFfn = kFfn / kQK * kQ4KBlock;        // 1152 B: down row (Q4_K)
constexpr int kQ6KRowFfn = kFfn / kQK * kQ6KBlock;        // 1680 B: down row (Q6_K)

struct __attribute__((aligned(16))) XGroup {
  int8_t a[64];    // first digit of elements 0..63
  int8_t b[64];    // second digit (units of 1/254)
  int8_t c[64];    // third digit (units of 1/254^2)
  float s[2];      // digit scale of sub-blocks 0 (elements 0-31) and 1 (32-63)
  float xsum[2];   // fp32 sum of the 32 elements of each sub-block
};
static_assert(sizeof(XGroup) == 208, "XGroup must be 208 bytes");
constexpr int kXGroupVec = sizeof(XGroup) / 16;  // 16-byte vectors per record (13)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// 4-byte aligned 16-byte vector: legal dwordx4 access at any dword address.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
  if (__builtin_constant_p(c) && c == 0) {
    // the first product of a chain: the three-operand form with an inline
    // zero accumulator (the compiler otherwise picks the two-operand
    // accumulating form and first moves 0 into its destination)
    int r;
    __asm__("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
  }
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Half bits -> float through the hardware converter (exact for every finite
// half, subnormals included: f16 denormals are not flushed by default).
__device__ __forceinline__ float half_to_float(uint32_t bits16) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xFFFFu));
  return (float)h;
}

// Half bits -> float by integer construction, bit-identical to quant.c:4-24
// for every input including signalling-NaN payloads.
__device__ __forceinline__ float half_bits_exact(uint32_t h) {
  uint32_t sign = (h >> 15) << 31;
  uint32_t e = (h >> 10) & 0x1Fu;
  uint32_t f = h & 0x3FFu;
  uint32_t bits;
  if (e == 0x1Fu) {
    bits = sign | 0x7F800000u | (f << 13);
  } else if (e != 0) {
    bits = sign | ((e + 112u) << 23) | (f << 13);
  } else if (f == 0) {
    bits = sign;
  } else {
    // leading one of the 10-bit fraction at bit p: value = f * 2^-24
    uint32_t p = 31u - __builtin_clz(f);  // 0..9
    uint32_t shift = 10u - p;
    bits = sign | ((113u - shift) << 23) | (((f << shift) & 0x3FFu) << 13);
  }
  return __builtin_bit_cast(float, bits);
}

// 6-bit scale and min of sub-blocks 2g and 2g+1 of a Q4_K block
// (quant.c:26-34).  s0/s1/s2 are the 12 scale bytes as three dwords.
// Sub-blocks 0-3 (g < 2) keep scale/min in the low six bits of bytes 0-3 /
// 4-7; sub-blocks 4-7 (g >= 2) take their low nibble from bytes 8-11 and
// their top two bits from bits 6-7 of bytes 0-3 / 4-7.  Written without
// branches: a lane's g is fixed, so the selectors below are per-lane
// constants and every lane runs the same instructions.
struct Q4KScaleSel {
  bool lowg;        // g < 2
  uint32_t width;   // 6 or 4 bits taken from the "low" source
  uint32_t off_sc;  // bit offset of sc_lo in its source (sc_hi: +8)
  uint32_t off_m;   // bit offset of m_lo in its source (m_hi: +8)
  uint32_t sh;      // 16 * (g & 1)
  uint32_t hmask;   // 0x30 when the top two bits come from bytes 0-7
};

__device__ __forceinline__ Q4KScaleSel q4k_scale_sel(int g) {
  Q4KScaleSel t;
  t.lowg = g < 2;
  t.sh = (uint32_t)(g & 1) * 16u;
  t.width = t.lowg ? 6u : 4u;
  t.off_sc = t.sh;
  t.off_m = t.lowg ? t.sh : t.sh + 4u;
  t.hmask = t.lowg ? 0u : 0x30u;
  return t;
}

__device__ __forceinline__ void q4k_scale_min_pair(uint32_t s0, uint32_t s1, uint32_t s2,
                                                   const Q4KScaleSel& t, int& sc_lo, int& m_lo,
                                                   int& sc_hi, int& m_hi) {
  const uint32_t A = t.lowg ? s0 : s2;
  const uint32_t B = t.lowg ? s1 : s2;
  sc_lo = (int)(__builtin_amdgcn_ubfe(A, t.off_sc, t.width) | ((s0 >> (t.sh + 2u)) & t.hmask));
  m_lo = (int)(__builtin_amdgcn_ubfe(B, t.off_m, t.width) | ((s1 >> (t.sh + 2u)) & t.hmask));
  sc_hi = (int)(__builtin_amdgcn_ubfe(A, t.off_sc + 8u, t.width) | ((s0 >> (t.sh + 10u)) & t.hmask));
  m_hi = (int)(__builtin_amdgcn_ubfe(B, t.off_m + 8u, t.width) | ((s1 >> (t.sh + 10u)) & t.hmask));
}

__device__ __forceinline__ void q4k_scale_min_pair(uint32_t s0, uint32_t s1, uint32_t s2, int g,
                                                   int& sc_lo, int& m_lo, int& sc_hi,
                                                   int& m_hi) {
  q4k_scale_min_pair(s0, s1, s2, q4k_scale_sel(g), sc_lo, m_lo, sc_hi, m_hi);
}

// One XGroup held in registers (52 VGPRs): digits a, b, c and {s0, s1, xsum0, xsum1}.
struct XDig {
  i32x4 a0, a1, a2, a3, b0, b1, b2, b3, c0, c1, c2, c3;
  f32x4 meta;
};

__device__ __forceinline__ XDig load_xdig(const XGroup* __restrict__ xg) {
  const i32x4* av = reinterpret_cast<const i32x4*>(xg->a);
  const i32x4* bv = reinterpret_cast<const i32x4*>(xg->b);
  const i32x4* cv = reinterpret_cast<const i32x4*>(xg->c);
  XDig x;
  x.a0 = av[0];
  x.a1 = av[1];
  x.a2 = av[2];
  x.a3 = av[3];
  x.b0 = bv[0];
  x.b1 = bv[1];
  x.b2 = bv[2];
  x.b3 = bv[3];
  x.c0 = cv[0];
  x.c1 = cv[1];
  x.c2 = cv[2];
  x.c3 = cv[3];
  x.meta = *reinterpret_cast<const f32x4*>(xg->s);
  return x;
}

// The three int32 digit sums of one sub-block, folded into units of s:
// A + B / 254 + C / 254^2 (each sum is exact; the fold rounds twice).
__device__ __forceinline__ float digit_fold(int A, int B, int C) {
  constexpr float k1 = 1.0f / 254.0f, k2 = 1.0f / 64516.0f;
  return fmaf((float)B, k1, fmaf((float)C, k2, (float)A));
}

// Dot product of one Q4_K group (qs bytes 32g..32g+31 of a block, i.e.
// elements 64g..64g+63) with the digits of the matching 64 activations.
//   hdr = first 16 bytes of the block: d | dmin | scales[0..11]
//   q0, q1 = the group's 32 qs bytes
// Returns sum over the 64 elements of (d*sc*q - dmin*m) * x.
__device__ __forceinline__ float q4k_group_dot(const u32x4 hdr, const u32x4 q0, const u32x4 q1,
                                               const Q4KScaleSel& sel, const XDig& x) {
  const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
  const uint32_t alo[8] = {(uint32_t)x.a0.x, (uint32_t)x.a0.y, (uint32_t)x.a0.z, (uint32_t)x.a0.w,
                           (uint32_t)x.a1.x, (uint32_t)x.a1.y, (uint32_t)x.a1.z, (uint32_t)x.a1.w};
  const uint32_t ahi[8] = {(uint32_t)x.a2.x, (uint32_t)x.a2.y, (uint32_t)x.a2.z, (uint32_t)x.a2.w,
                           (uint32_t)x.a3.x, (uint32_t)x.a3.y, (uint32_t)x.a3.z, (uint32_t)x.a3.w};
  const uint32_t blo[8] = {(uint32_t)x.b0.x, (uint32_t)x.b0.y, (uint32_t)x.b0.z, (uint32_t)x.b0.w,
                           (uint32_t)x.b1.x, (uint32_t)x.b1.y, (uint32_t)x.b1.z, (uint32_t)x.b1.w};
  const uint32_t bhi[8] = {(uint32_t)x.b2.x, (uint32_t)x.b2.y, (uint32_t)x.b2.z, (uint32_t)x.b2.w,
                           (uint32_t)x.b3.x, (uint32_t)x.b3.y, (uint32_t)x.b3.z, (uint32_t)x.b3.w};
  const uint32_t clo[8] = {(uint32_t)x.c0.x, (uint32_t)x.c0.y, (uint32_t)x.c0.z, (uint32_t)x.c0.w,
                           (uint32_t)x.c1.x, (uint32_t)x.c1.y, (uint32_t)x.c1.z, (uint32_t)x.c1.w};
  const uint32_t chi[8] = {(uint32_t)x.c2.x, (uint32_t)x.c2.y, (uint32_t)x.c2.z, (uint32_t)x.c2.w,
                           (uint32_t)x.c3.x, (uint32_t)x.c3.y, (uint32_t)x.c3.z, (uint32_t)x.c3.w};
  int A0 = 0, B0 = 0, C0 = 0, A1 = 0, B1 = 0, C1 = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t lo = w[i] & 0x0F0F0F0Fu;
    const uint32_t hi = (w[i] >> 4) & 0x0F0F0F0Fu;
    A0 = sdot4(lo, alo[i], A0);
    B0 = sdot4(lo, blo[i], B0);
    C0 = sdot4(lo, clo[i], C0);
    A1 = sdot4(hi, ahi[i], A1);
    B1 = sdot4(hi, bhi[i], B1);
    C1 = sdot4(hi, chi[i], C1);
  }
  int sc0, m0, sc1, m1;
  q4k_scale_min_pair(hdr.y, hdr.z, hdr.w, sel, sc0, m0, sc1, m1);
  const float d = half_to_float(hdr.x);
  const float dmin = half_to_float(hdr.x >> 16);
  const f32x4 meta = x.meta;
  const float f0 = meta.x * digit_fold(A0, B0, C0);
  const float f1 = meta.y * digit_fold(A1, B1, C1);
  const float qx = fmaf((float)sc0, f0, (float)sc1 * f1);
  const float mx = fmaf((float)m0, meta.z, (float)m1 * meta.w);
  return fmaf(d, qx, -dmin * mx);
}

// The same from a record in LDS, read in quarters (qs bytes 0-15, then
// 16-31, each with the digits of its low-nibble and then of its high-nibble
// elements), so at most 12 registers of digits are live at a time.
__device__ __forceinline__ float q4k_group_dot(const u32x4 hdr, const u32x4 q0, const u32x4 q1,
                                               const Q4KScaleSel& sel,
                                               const XGroup* __restrict__ xg) {
  const i32x4* av = reinterpret_cast<const i32x4*>(xg->a);
  const i32x4* bv = reinterpret_cast<const i32x4*>(xg->b);
  const i32x4* cv = reinterpret_cast<const i32x4*>(xg->c);
  int A[2] = {0, 0}, B[2] = {0, 0}, C[2] = {0, 0};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      // n = 0: low nibbles (sub-block 0, digits 16h..16h+15); n = 1: high
      // nibbles (sub-block 1, digits 32 + 16h ..)
      const u32x4 q = h ? q1 : q0;
      const i32x4 a = av[2 * n + h], b = bv[2 * n + h], c = cv[2 * n + h];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t v = n ? (q[i] >> 4) & 0x0F0F0F0Fu : q[i] & 0x0F0F0F0Fu;
        A[n] = sdot4(v, (uint32_t)a[i], A[n]);
        B[n] = sdot4(v, (uint32_t)b[i], B[n]);
        C[n] = sdot4(v, (uint32_t)c[i], C[n]);
      }
      // the sums are complete here: the quarter's digits are dead before
      // the next quarter's are read
      __asm__ volatile("" : "+v"(A[n]), "+v"(B[n]), "+v"(C[n]));
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  const int A0 = A[0], B0 = B[0], C0 = C[0], A1 = A[1], B1 = B[1], C1 = C[1];
  const f32x4 meta = *reinterpret_cast<const f32x4*>(xg->s);
  int sc0, m0, sc1, m1;
  q4k_scale_min_pair(hdr.y, hdr.z, hdr.w, sel, sc0, m0, sc1, m1);
  const float d = half_to_float(hdr.x);
  const float dmin = half_to_float(hdr.x >> 16);
  const float f0 = meta.x * digit_fold(A0, B0, C0);
  const float f1 = meta.y * digit_fold(A1, B1, C1);
  const float qx = fmaf((float)sc0, f0, (float)sc1 * f1);
  const float mx = fmaf((float)m0, meta.z, (float)m1 * meta.w);
  return fmaf(d, qx, -dmin * mx);
}

// A workgroup's copy of n (<= MAXN) digit records from global memory into
// LDS in one round trip: every 16-byte load of a thread is issued (load)
// before any is stored (store).  Issue the loads ahead of a kernel's weight
// loads: loads complete in order, so the stores then wait for the records
// only, and each weight group is used as soon as it arrives.
template <int MAXN>
struct XStage {
  static constexpr int kSteps = (MAXN * kXGroupVec + 255) / 256;
  u32x4 v[kSteps];
  __device__ __forceinline__ void load(const XGroup* __restrict__ src, int n) {
    const u32x4* s = reinterpret_cast<const u32x4*>(src);
#pragma unroll
    for (int k = 0; k < kSteps; ++k) {
      const int i = threadIdx.x + 256 * k;
      if (i < n * kXGroupVec) v[k] = s[i];
    }
  }
  __device__ __forceinline__ void store(XGroup* __restrict__ dst, int n) const {
    u32x4* d = reinterpret_cast<u32x4*>(dst);
#pragma unroll
    for (int k = 0; k < kSteps; ++k) {
      const int i = threadIdx.x + 256 * k;
      if (i < n * kXGroupVec) d[i] = v[k];
    }
  }
};

// Any number of records, XStage<112> at a time (for lengths known only at
// run time).
__device__ __forceinline__ void xstage_copy(XGroup* __restrict__ dst, const XGroup* __restrict__ src, int n) {
  for (int b = 0; b < n; b += 112) {
    XStage<112> st;
    st.load(src + b, min(112, n - b));
    st.store(dst + b, min(112, n - b));
  }
}

// Broadcast lane `src` of each group of four lanes to the whole quad (DPP
// quad_perm [src,src,src,src]; no LDS traffic).
template <int SRC>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
  constexpr int ctrl = SRC | (SRC << 2) | (SRC << 4) | (SRC << 6);
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, ctrl, 0xF, 0xF, false);
}

// The weight bytes one lane needs for one Q4_K group.  The four lanes that
// share a block (groups g = 0..3 of it, consecutive lanes) each load one
// dword of the 16-byte block header and exchange them by DPP, instead of
// all four loading the whole header.
struct Q4KGroupLoad {
  uint32_t hdr_part;  // header dword g of the block
  u32x4 q0, q1;       // the group's 32 qs bytes
};

__device__ __forceinline__ Q4KGroupLoad q4k_load_group(const uint8_t* blk, int g) {
  Q4KGroupLoad r;
  r.hdr_part = *reinterpret_cast<const uint32_t*>(blk + 4 * g);
  r.q0 = *reinterpret_cast<const u32x4_a4*>(blk + 16 + 32 * g);
  r.q1 = *reinterpret_cast<const u32x4_a4*>(blk + 32 + 32 * g);
  return r;
}

// Every lane of the quad must call this (it exchanges header dwords).
__device__ __forceinline__ u32x4 q4k_quad_hdr(const Q4KGroupLoad& r) {
  u32x4 h;
  h.x = quad_bcast<0>(r.hdr_part);
  h.y = quad_bcast<1>(r.hdr_part);
  h.z = quad_bcast<2>(r.hdr_part);
  h.w = quad_bcast<3>(r.hdr_part);
  return h;
}

__device__ __forceinline__ float q4k_group_dot_ld(const Q4KGroupLoad& r, const Q4KScaleSel& sel,
                                                  const XGroup* __restrict__ xg) {
  return q4k_group_dot(q4k_quad_hdr(r), r.q0, r.q1, sel, xg);
}

__device__ __forceinline__ float q4k_group_dot_ld(const Q4KGroupLoad& r, const Q4KScaleSel& sel, const XDig& x) {
  return q4k_group_dot(q4k_quad_hdr(r), r.q0, r.q1, sel, x);
}

// ---- fp32 dot of one Q4_K group with x held in LDS -------------------------------------
// x in LDS as 68 floats per 64-element group (16 bytes of padding, so the
// lanes of a wave, one group each, read distinct banks), the fp32 sum of
// each 32-element sub-block beside it.  Returns
//   d (sc0 S0 + sc1 S1) - dmin (m0 X0 + m1 X1),  S = sum_k q_k x_k in fp32,
// dequant_matvec_q4k's arithmetic (shaders.metal:43-99) in fp32.  A nibble
// q read as an fp8 (e4m3) byte is q * 2^-c exactly (q < 16: exponent field 0
// or 1), so the fp8 conversion widens two nibbles per instruction; the
// products are summed on that scale and qscale = 2^c is folded into d.
constexpr int kXPad = 68;
__device__ __forceinline__ float q4k_fp8_qscale() { return 1.0f / __builtin_amdgcn_cvt_pk_f32_fp8(1, false)[0]; }
__device__ __forceinline__ float q4k_group_dot_f32(const Q4KGroupLoad& ld, const u32x4 hdr, int g,
                                                   const float* __restrict__ x0, float xsum0, float xsum1,
                                                   float qscale) {
  const uint32_t w[8] = {ld.q0.x, ld.q0.y, ld.q0.z, ld.q0.w, ld.q1.x, ld.q1.y, ld.q1.z, ld.q1.w};
  float S0 = 0.0f, S1 = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(x0 + 4 * i);
    const f32x4 b = *reinterpret_cast<const f32x4*>(x0 + 32 + 4 * i);
    const int lo = (int)(w[i] & 0x0F0F0F0Fu), hi = (int)((w[i] >> 4) & 0x0F0F0F0Fu);
    const auto l01 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false), l23 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
    const auto h01 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false), h23 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
    S0 = fmaf(l01[0], a.x, S0);
    S0 = fmaf(l01[1], a.y, S0);
    S0 = fmaf(l23[0], a.z, S0);
    S0 = fmaf(l23[1], a.w, S0);
    S1 = fmaf(h01[0], b.x, S1);
    S1 = fmaf(h01[1], b.y, S1);
    S1 = fmaf(h23[0], b.z, S1);
    S1 = fmaf(h23[1], b.w, S1);
  }
  int sc0, m0, sc1, m1;
  q4k_scale_min_pair(hdr.y, hdr.z, hdr.w, q4k_scale_sel(g), sc0, m0, sc1, m1);
  const float d = half_to_float(hdr.x) * qscale, dmin = half_to_float(hdr.x >> 16);
  const float qx = fmaf((float)sc0, S0, (float)sc1 * S1);
  const float mx = fmaf((float)m0, xsum0, (float)m1 * xsum1);
  return fmaf(d, qx, -dmin * mx);
}

// R rows' groups (the same group position g in every row) against ONE
// digit record in LDS: each quarter of the record (12 registers of digits)
// is read once and applied to all R rows, so a lane's LDS traffic is one
// record instead of R.  Sub-block by sub-block (low nibbles, then high), so
// only one sub-block's int32 sums are live.  out[r] = the group's dot of row r,
// the same arithmetic as q4k_group_dot.
template <int R>
__device__ __forceinline__ void q4k_group_dot_rows(const Q4KGroupLoad (&ld)[R], const Q4KScaleSel& sel,
                                                   const XGroup* __restrict__ xg, float (&out)[R]) {
  const i32x4* av = reinterpret_cast<const i32x4*>(xg->a);
  const i32x4* bv = reinterpret_cast<const i32x4*>(xg->b);
  const i32x4* cv = reinterpret_cast<const i32x4*>(xg->c);
  float f0[R];
#pragma unroll
  for (int n = 0; n < 2; ++n) {
    int A[R], B[R], C[R];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const i32x4 a = av[2 * n + h], b = bv[2 * n + h], c = cv[2 * n + h];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const u32x4 q = h ? ld[r].q1 : ld[r].q0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t v = n ? (q[i] >> 4) & 0x0F0F0F0Fu : q[i] & 0x0F0F0F0Fu;
          const bool first = h == 0 && i == 0;
          A[r] = sdot4(v, (uint32_t)a[i], first ? 0 : A[r]);
          B[r] = sdot4(v, (uint32_t)b[i], first ? 0 : B[r]);
          C[r] = sdot4(v, (uint32_t)c[i], first ? 0 : C[r]);
        }
      }
    }
    const f32x4 meta = *reinterpret_cast<const f32x4*>(xg->s);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float f = (n ? meta.y : meta.x) * digit_fold(A[r], B[r], C[r]);
      if (n == 0) {
        f0[r] = f;
      } else {
        const u32x4 hdr = q4k_quad_hdr(ld[r]);
        int sc0, m0, sc1, m1;
        q4k_scale_min_pair(hdr.y, hdr.z, hdr.w, sel, sc0, m0, sc1, m1);
        const float d = half_to_float(hdr.x);
        const float dmin = half_to_float(hdr.x >> 16);
        const float qx = fmaf((float)sc0, f0[r], (float)sc1 * f);
        const float mx = fmaf((float)m0, meta.z, (float)m1 * meta.w);
        out[r] = fmaf(d, qx, -dmin * mx);
      }
    }
  }
}


// ---- the resident expert layout (REL) ---------------------------------------------------
// Experts of a resident layer are stored with each Q4_K matrix permuted so
// that every load instruction of the dot4 kernels reads whole contiguous
// lines: in the packed layout a half-wave's 16-byte loads hit every other
// 16 bytes of several rows, so lines are fetched twice and the streaming
// ("nt") cache policy cannot be used; in REL a half-wave (gate/up) or a
// wave (down) reads one contiguous run, and nontemporal loads stream ~20%
// faster.  The values are untouched: REL is a permutation of the packed
// blob's bytes, made once when a layer becomes resident.
//  gate / up [2048 x 7168] (28 blocks per row): step (row / 2, block / 4),
//    N = 32 pieces, at ((row / 2) * 7 + block / 4) * 1152.
//  down Q4_K [7168 x 2048] (8 blocks per row): step (block / 4, row / 4),
//    N = 64 pieces, at ((block / 4) * 1792 + row / 4) * 2304.
//  Inside a step (36 N bytes): the first 16 qs bytes of group g of each
//  piece at 16 L, the last 16 at 16 N + 16 L, header dword g at 32 N + 4 L,
//  where L = (block % 4) * 4 R + (row % R) * 4 + g (R = 2 rows for gate /
//  up, 4 for down): one block of a step's rows fills whole 128-byte lines of
//  q0 and of q1, so a kernel that walks the blocks one at a time (the
//  grouped GEMMs) reads every line at once instead of half of it now and
//  the other half a block later, after the L2 may have dropped it.  A Q6_K
//  down matrix has a layout of its own (below).
constexpr int kRelGuPieces = 32;
constexpr int kRelDnPieces = 64;

template <bool DOWN>
__device__ __forceinline__ const uint8_t* rel_step(const uint8_t* mat, int row, int block) {
  constexpr size_t kStep = 36 * (DOWN ? kRelDnPieces : kRelGuPieces);
  return mat + (DOWN ? ((size_t)(block >> 2) * (kHidden / 4) + (row >> 2))
                     : ((size_t)(row >> 1) * (kHidden / 1024) + (block >> 2))) * kStep;
}

template <bool DOWN>
__device__ __forceinline__ int rel_piece(int row, int block, int g) {
  return DOWN ? (block & 3) * 16 + (row & 3) * 4 + g : (block & 3) * 8 + (row & 1) * 4 + g;
}

// Group g of block `block` of row `row` of a REL matrix, by nontemporal loads.
template <bool DOWN>
__device__ __forceinline__ Q4KGroupLoad rel_load_group(const uint8_t* mat, int row, int block, int g) {
  constexpr int N = DOWN ? kRelDnPieces : kRelGuPieces;
  const uint8_t* s = rel_step<DOWN>(mat, row, block);
  const int L = rel_piece<DOWN>(row, block, g);
  Q4KGroupLoad r;
  r.hdr_part = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(s + 32 * N + 4 * L));
  r.q0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(s + 16 * L));
  r.q1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(s + 16 * N + 16 * L));
  return r;
}

// ---- the resident layout of a Q6_K down matrix ---------------------------------------------
// A Q6_K down matrix [7168 x 2048] (8 blocks of 210 B per row) of a resident
// layer is stored in steps of 16 rows x 4 blocks (64 blocks, 13,440 B = 105
// whole 128-byte lines) at ((block / 4) * 448 + row / 16) * 13,440, so a
// column part of 4 blocks is one contiguous run of steps.  Inside a step the
// block's bytes are split by kind and every kind is aligned: with the block
// index b = (row % 16 / 4) * 16 + (block % 4) * 4 + row % 4 and the piece
// p = 2 b + half (a half is 128 weights: ql bytes 64 h .. 64 h + 63, qh
// bytes 128 + 32 h .., scales 192 + 8 h .. of the packed block),
//   ql chunk j (16 B, j < 4) of piece p at j * 2048 + 16 p
//   qh chunk j (j < 2) at 8192 + j * 2048 + 16 p
//   the half's 8 scales at 12288 + 8 p
//   d of block b at 13312 + 2 b
// so the 32 pieces of 4 rows x 4 blocks are consecutive: a wave's load of
// them reads one contiguous 512-byte run per chunk, and no word needs the
// byte realignment of the packed 210-byte blocks.  The values are untouched:
// every byte of the packed blob has one place in the step.
constexpr int kRel6Step = 13440;
constexpr int kRel6Ql = 0, kRel6Qh = 8192, kRel6Sc = 12288, kRel6D = 13312;

__host__ __device__ __forceinline__ size_t rel6_step_off(int row, int block) {
  return ((size_t)(block >> 2) * (kHidden / 16) + (size_t)(row >> 4)) * kRel6Step;
}
__host__ __device__ __forceinline__ int rel6_block_index(int row, int block) {
  return ((row & 15) >> 2) * 16 + (block & 3) * 4 + (row & 3);
}

// The words one lane needs for one 128-element half of a Q6_K block, aligned.
struct Q6KHalfW {
  uint32_t ql[16], qh[8], sc[2];
  uint32_t d;  // the block's fp16 d in the low 16 bits
};

__device__ __forceinline__ Q6KHalfW q6k_rel_load_half(const uint8_t* mat, int row, int block, int half) {
  const uint8_t* s = mat + rel6_step_off(row, block);
  const int b = rel6_block_index(row, block), p = 2 * b + half;
  Q6KHalfW r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(s + kRel6Ql + j * 2048 + 16 * p));
    r.ql[4 * j] = v.x;
    r.ql[4 * j + 1] = v.y;
    r.ql[4 * j + 2] = v.z;
    r.ql[4 * j + 3] = v.w;
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(s + kRel6Qh + j * 2048 + 16 * p));
    r.qh[4 * j] = v.x;
    r.qh[4 * j + 1] = v.y;
    r.qh[4 * j + 2] = v.z;
    r.qh[4 * j + 3] = v.w;
  }
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 sc = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(s + kRel6Sc + 8 * p));
  r.sc[0] = sc.x;
  r.sc[1] = sc.y;
  const uint32_t dw = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(s + kRel6D + 4 * (b >> 1)));
  r.d = (b & 1) ? dw >> 16 : dw;
  return r;
}

// funnel: the 4 bytes starting `byte_shift` (0..3) bytes into the 8-byte
// little-endian pair (lo, hi).
__device__ __forceinline__ uint32_t funnel(uint32_t lo, uint32_t hi, uint32_t byte_shift) {
  return __builtin_amdgcn_alignbyte(hi, lo, byte_shift);
}

// Dot product of one 128-element half of a Q6_K block (quant.c:63-92) with
// the digits of its activations.  The half's bytes are passed already
// realigned: ql[16] (64 bytes), qh[8] (32 bytes), sc[2] (8 int8 scales).
// x0 covers elements 0..63 of the half, x1 elements 64..127.
// Returns sum over the 128 elements of d*sc*(q-32) * x, without the d.
__device__ __forceinline__ float q6k_half_dot(const uint32_t* ql, const uint32_t* qh,
                                              const uint32_t* sc, const XGroup* __restrict__ x0,
                                              const XGroup* __restrict__ x1) {
  const uint32_t* a0 = reinterpret_cast<const uint32_t*>(x0->a);
  const uint32_t* b0 = reinterpret_cast<const uint32_t*>(x0->b);
  const uint32_t* c0 = reinterpret_cast<const uint32_t*>(x0->c);
  const uint32_t* a1 = reinterpret_cast<const uint32_t*>(x1->a);
  const uint32_t* b1 = reinterpret_cast<const uint32_t*>(x1->b);
  const uint32_t* c1 = reinterpret_cast<const uint32_t*>(x1->c);
  // quarter k covers elements 32k..32k+31 of the half (k = 0..3), scale
  // half s = l / 16: the integer sums of one quarter are complete (and
  // folded) before the next quarter's begin, so only six are live.
  const float xs[4] = {x0->s[0], x0->s[1], x1->s[0], x1->s[1]};
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t* ak = (k < 2 ? a0 : a1) + 8 * (k & 1);
    const uint32_t* bk = (k < 2 ? b0 : b1) + 8 * (k & 1);
    const uint32_t* ck = (k < 2 ? c0 : c1) + 8 * (k & 1);
    int A[2] = {0, 0}, B[2] = {0, 0}, C[2] = {0, 0};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int s = i >> 2;
      const uint32_t wl = ql[i], wl2 = ql[8 + i], wh = qh[i];
      // Each byte becomes 4*(q-32) as int8: the 6-bit q sits in bits 2..7 and
      // flipping bit 7 subtracts 128.
      uint32_t v;
      if (k == 0) v = (((wl & 0x0F0F0F0Fu) << 2) | ((wh & 0x03030303u) << 6)) ^ 0x80808080u;
      else if (k == 1) v = (((wl2 & 0x0F0F0F0Fu) << 2) | ((wh & 0x0C0C0C0Cu) << 4)) ^ 0x80808080u;
      else if (k == 2) v = (((wl >> 2) & 0x3C3C3C3Cu) | ((wh & 0x30303030u) << 2)) ^ 0x80808080u;
      else v = (((wl2 >> 2) & 0x3C3C3C3Cu) | (wh & 0xC0C0C0C0u)) ^ 0x80808080u;
      A[s] = sdot4(v, ak[i], A[s]);
      B[s] = sdot4(v, bk[i], B[s]);
      C[s] = sdot4(v, ck[i], C[s]);
    }
    // scales sc[2k + s]: byte (2k + s) of the 8 scale bytes, as int8
    const uint32_t word = sc[k >> 1];
    const int sh = (k & 1) * 16;
    const int sa = (int)(int8_t)((word >> sh) & 0xFF);
    const int sb = (int)(int8_t)((word >> (sh + 8)) & 0xFF);
    // |sc * sum| < 2^31: 128 * 16 * 128 * 127 per scale half
    const int ia = sa * A[0] + sb * A[1];
    const int ib = sa * B[0] + sb * B[1];
    const int ic = sa * C[0] + sb * C[1];
    acc = fmaf(xs[k], digit_fold(ia, ib, ic), acc);
  }
  return acc * 0.25f;
}

// Raw words of one 128-element half of a Q6_K block, loaded from
// dword-aligned addresses (a block starts at any even byte offset).
struct Q6KHalfLoad {
  uint32_t ql[17], qh[9];
  uint32_t sc[2];
  uint32_t d;
  uint32_t shift;
};

__device__ __forceinline__ Q6KHalfLoad q6k_load_half(const uint8_t* blk, int h) {
  Q6KHalfLoad r;
  const uintptr_t a0 = reinterpret_cast<uintptr_t>(blk + 64 * h);
  r.shift = a0 & 3u;
  const uint32_t* p = reinterpret_cast<const uint32_t*>(a0 - r.shift);
#pragma unroll
  for (int i = 0; i < 16; ++i) r.ql[i] = p[i];
  r.ql[16] = r.shift ? p[16] : 0u;
  const uint32_t* ph =
      reinterpret_cast<const uint32_t*>(reinterpret_cast<uintptr_t>(blk + 128 + 32 * h) - r.shift);
#pragma unroll
  for (int i = 0; i < 8; ++i) r.qh[i] = ph[i];
  r.qh[8] = r.shift ? ph[8] : 0u;
  const uint16_t* s16 = reinterpret_cast<const uint16_t*>(blk + 192 + 8 * h);
  r.sc[0] = (uint32_t)s16[0] | ((uint32_t)s16[1] << 16);
  r.sc[1] = (uint32_t)s16[2] | ((uint32_t)s16[3] << 16);
  r.d = *reinterpret_cast<const uint16_t*>(blk + 208);
  return r;
}

__device__ __forceinline__ float q6k_half_dot_w(const Q6KHalfW& r, const XGroup* __restrict__ xg) {
  return half_to_float(r.d) * q6k_half_dot(r.ql, r.qh, r.sc, xg, xg + 1);
}

__device__ __forceinline__ float q6k_half_dot_ld(const Q6KHalfLoad& r,
                                                 const XGroup* __restrict__ xg) {
  uint32_t ql[16], qh[8];
#pragma unroll
  for (int i = 0; i < 16; ++i) ql[i] = funnel(r.ql[i], r.ql[i + 1], r.shift);
#pragma unroll
  for (int i = 0; i < 8; ++i) qh[i] = funnel(r.qh[i], r.qh[i + 1], r.shift);
  return half_to_float(r.d) * q6k_half_dot(ql, qh, r.sc, xg, xg + 1);
}

// v of lane i + N of the same 16-lane row (DPP row_shl:N; 0 past the row).
template <int N>
__device__ __forceinline__ float dpp_row_shl(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + N, 0xF, 0xF, true));
}

// Sum of v over an aligned group of L lanes (L = 2, 4, 8 or 16, inside one
// 16-lane row) into the group's first lane by DPP row shifts: lane i adds
// lane i + m, m = L/2 .. 1, so the first lane gets exactly what the xor
// butterfly gives it (the same pairs, in the same order).
template <int L>
__device__ __forceinline__ float group_sum_first(float v) {
  static_assert(L == 2 || L == 4 || L == 8 || L == 16, "a power of two inside a DPP row");
  if constexpr (L >= 16) v = v + dpp_row_shl<8>(v);
  if constexpr (L >= 8) v = v + dpp_row_shl<4>(v);
  if constexpr (L >= 4) v = v + dpp_row_shl<2>(v);
  v = v + dpp_row_shl<1>(v);
  return v;
}

// The sum of v over the 64 lanes of a wave, in lane 0: at each step m = 32,
// 16, 8, 4, 2, 1 lane i < m adds lane i + m, so lane 0 adds exactly the pairs,
// in the same order, that the xor butterfly v += shfl_xor(v, m) adds in its
// lane 0 (the same bits).  m = 32 and 16 by v_permlane32_swap /
// v_permlane16_swap (element 1 of the swap of v with itself holds lane i + 32
// in lanes 0-31, lane i + 16 in lanes 0-15), the rest by DPP row shifts: VALU
// only, no lane exchange through the LDS crossbar.  Other lanes hold partial
// sums.
__device__ __forceinline__ float wave_sum_lane0(float v) {
  const uint32_t u32 = __float_as_uint(v);
  v = v + __uint_as_float(__builtin_amdgcn_permlane32_swap(u32, u32, false, false)[1]);
  const uint32_t u16 = __float_as_uint(v);
  v = v + __uint_as_float(__builtin_amdgcn_permlane16_swap(u16, u16, false, false)[1]);
  v = v + dpp_row_shl<8>(v);
  v = v + dpp_row_shl<4>(v);
  v = v + dpp_row_shl<2>(v);
  v = v + dpp_row_shl<1>(v);
  return v;
}

// Sum over the 16 lanes of a row group (lanes 16r..16r+15) into the group's
// first lane (lane 16r), the value the xor butterfly over 8, 4, 2, 1 gives it
// (group_sum_first); the other lanes hold partial sums, so callers read the
// first lanes only.
__device__ __forceinline__ float sum16(float v) { return group_sum_first<16>(v); }

// Cross-workgroup hand-off inside one kernel (arrival counters).  The few
// values handed over are written with agent-scope stores (written through
// past the per-XCD L2) and read with agent-scope loads, so the writer only
// has to wait for its stores to be acknowledged before bumping the counter.
// A __threadfence() would do the same but write back and invalidate the
// whole L2 of the XCD, once per workgroup.
__device__ __forceinline__ void store_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores_done() { __builtin_amdgcn_s_waitcnt(0); }
__device__ __forceinline__ int arrive_agent(int* counter) {
  return __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void reset_agent(int* counter) {
  __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned load_u32_agent(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_u32_agent(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// Reduction of v over each half-wave (lanes 0-31 and 32-63) by DPP: row
// shifts within rows of 16, then row_bcast:15 folds rows 0/2 into rows 1/3;
// every lane receives its half's result (readlane of lane 31 / 63).
template <bool MAX>
__device__ __forceinline__ float half_reduce(float v) {
  const auto op = [](float x, float y) { return MAX ? fmaxf(x, y) : x + y; };
  const int fill = MAX ? __float_as_int(-__builtin_inff()) : 0;
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(fill, __float_as_int(v), 0x111, 0xF, 0xF, false)));
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(fill, __float_as_int(v), 0x112, 0xF, 0xF, false)));
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(fill, __float_as_int(v), 0x114, 0xF, 0xF, false)));
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(fill, __float_as_int(v), 0x118, 0xF, 0xF, false)));
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(fill, __float_as_int(v), 0x142, 0xA, 0xF, false)));
  const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
  const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
  return (threadIdx.x & 32) ? hi : lo;
}

// Digits of the 32 elements of one sub-block.  Called by all 64 lanes of a
// wave; each half-wave (lanes 0-31, 32-63) is one sub-block and each lane
// holds one element v.  Returns the a / b / c digits for the lane and the
// sub-block's scale and fp32 sum (summed in one fixed order, so every
// caller gets the same bits for the same elements).
//   s = 2^e, the smallest power of two with max|v| / s <= 127: t = v / s is
//   exact, a = rint(t), r = t - a (exact), b = rint(254 r), u = 254 r - b
//   (one rounding, by fma), c = rint(254 u).  |t - (a + b/254 + c/254^2)|
//   <= (0.5 + 2^-17) / 254^2.
__device__ __forceinline__ void make_digits3(float v, int8_t& a_out, int8_t& b_out, int8_t& c_out,
                                             float& s_out, float& sum_out) {
  const float amax = half_reduce<true>(fabsf(v));
  const float sum = half_reduce<false>(v);
  int a = 0, b = 0, c = 0;
  float s;
  if (amax > 0.0f && amax <= 3.4028234e38f) {
    // amax = m * 2^E, m in [1, 2): s = 2^(E - 6) unless m > 127/64, then 2^(E - 5)
    int E;
    const float m = frexpf(amax, &E);  // amax = m * 2^E, m in [0.5, 1)
    int e = E - 7;                     // amax / 2^e = 128 m in [64, 128)
    if (m * 128.0f > 127.0f) e += 1;   // keep max |t| <= 127
    s = ldexpf(1.0f, e);
    const float t = ldexpf(v, -e);  // exact: a power-of-two scaling of a normal result
    const float ra = rintf(t);
    const float r = t - ra;         // exact, |r| <= 0.5
    const float rb = rintf(r * 254.0f);
    const float u = fmaf(r, 254.0f, -rb);  // |u| <= 0.5 + 2^-17
    const float rc = fminf(fmaxf(rintf(u * 254.0f), -127.0f), 127.0f);
    a = (int)ra;
    b = (int)rb;
    c = (int)rc;
  } else {
    // all zero: s = 0 gives exact zeros; inf/NaN: propagate a NaN scale
    s = (amax == 0.0f) ? 0.0f : __builtin_nanf("");
  }
  a_out = (int8_t)a;
  b_out = (int8_t)b;
  c_out = (int8_t)c;
  s_out = s;
  sum_out = sum;
}

// The digit record of one 64-element group, by the whole wave (lane l holds
// element l), published for other workgroups: agent-scope dword stores (four
// lanes' digits packed per dword), followed by the caller's wait for the
// stores and its flag.
__device__ __forceinline__ void publish_digit_group(float v, XGroup* xg) {
  const int lane = threadIdx.x & 63;
  int8_t da, db, dc;
  float ds, dsum;
  make_digits3(v, da, db, dc, ds, dsum);
  const int l = lane & 31, sub = lane >> 5;
  auto pack4 = [](int8_t d) {
    const unsigned u = (uint8_t)d;
    return u | (__shfl_down(u, 1, 32) << 8) | (__shfl_down(u, 2, 32) << 16) | (__shfl_down(u, 3, 32) << 24);
  };
  const unsigned wa = pack4(da), wb = pack4(db), wc = pack4(dc);
  if ((l & 3) == 0) {
    store_u32_agent(reinterpret_cast<unsigned*>(xg->a) + 8 * sub + l / 4, wa);
    store_u32_agent(reinterpret_cast<unsigned*>(xg->b) + 8 * sub + l / 4, wb);
    store_u32_agent(reinterpret_cast<unsigned*>(xg->c) + 8 * sub + l / 4, wc);
  }
  if (l == 0) {
    store_agent(&xg->s[sub], ds);
    store_agent(&xg->xsum[sub], dsum);
  }
}

// ---- tagged words -------------------------------------------------------------------------
// {epoch, payload} in one 64-bit word written by one agent-scope store: a
// reader's load is its own readiness check (tag == this call's epoch) and
// nothing is ever cleared.
__device__ __forceinline__ void put_tagged(uint64_t* p, unsigned epoch, uint32_t bits) {
  __hip_atomic_store(p, ((uint64_t)epoch << 32) | bits, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t get_tagged(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool tag_is(uint64_t v, unsigned epoch) {
  return (unsigned)(v >> 32) == epoch;
}
__device__ __forceinline__ float tagged_f(uint64_t v) { return __uint_as_float((uint32_t)v); }
__device__ __forceinline__ int tagged_i(uint64_t v) { return (int)(uint32_t)v; }


// Digits of the 64 elements held by one wave (lane l: element l) into LDS
// record g (two sub-blocks of 32, one per half-wave).
__device__ __forceinline__ void digits_to_lds(float v, XGroup& g) {
  const int lane = threadIdx.x & 63;
  int8_t da, db, dc;
  float ds, dsum;
  make_digits3(v, da, db, dc, ds, dsum);
  g.a[lane] = da;
  g.b[lane] = db;
  g.c[lane] = dc;
  if ((lane & 31) == 0) {
    g.s[lane >> 5] = ds;
    g.xsum[lane >> 5] = dsum;
  }
}

}  // namespace fdm
