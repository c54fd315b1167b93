// rms_device.h -- the sum of squares of rms_norm (infer.m:369-374) on one
// 256-thread workgroup, bit for bit, without its 7,168 dependent steps.
//
// The reference's loop compiles to one chain ss <- fma(x_i, x_i, ss) in
// index order (clang contracts `ss += x[i]*x[i]`).  Each step rounds
// ss + x_i^2 (exact product) to float.  While ss stays inside one binade
// [2^e, 2^(e+1)) its grid is u = 2^(e-23) and ss is a multiple of u, so the
// step is ss + u * rint(x_i^2 / u) -- independent of ss -- unless the sum
// leaves the binade or x_i^2 / u is a tie (then round-half-even looks at
// ss).  The chain is therefore a sum of integers inside each binade, and
// only the steps near a binade boundary (and ties) need the real fma:
//
//  1. P_i = sum_{j<i} x_j^2, summed in float (a block scan), approximates
//     the true chain value before step i: every step of the chain rounds by
//     at most 2^-24 of the running sum, so |ss_i - sum_{j<i} x_j^2| <=
//     i 2^-24 ss_i <= 2^-11 ss_i (d <= 8192), and the float prefix adds
//     less than 2^-18 more.
//  2. Step i is a "run" step when P_i and P_i + x_i^2 both lie inside one
//     binade with a relative margin of 2^-10 to its ends (so the true ss_i
//     and ss_(i+1) lie in it too), P_i >= 2^-100 (normal grid) and
//     x_i^2 / u is safely away from a tie; it then adds
//     K_i = rint(x_i^2 / u) < 2^24.  Every other step is "risky" (the first
//     step always is: P_0 = 0).  x_i^2 / u is formed exactly in floats:
//     x^2 = h + l with h = x*x, l = fma(x, x, -h) (exact for |x| >= 2^-40,
//     smaller x are risky), both scaled by 2^(24-E); K = rint(h'), and the
//     step is risky unless |(h' - K) + l'| < 1/2 - 2^-23 -- (h' - K) is
//     exact and the rounded sum is within 2^-26 of the true fraction, so a
//     step that passes has |fraction| < 1/2 and K is the exact rint.  A risky step keeps the
//     binade exponent E of P_i in its LDS slot (bit 31 set), so the list of
//     risky steps needs no second pass over the prefix.
//  3. Consecutive run steps share one binade, so a run adds exactly
//     u * (sum of its K) -- one float addition, exact because the result
//     stays on the grid inside the binade.  The K are summed mod 2^32 (a
//     run's sum is < 2^24, so differences of the prefix are exact).  The
//     risky steps, in order, are walked by one lane:
//     ss <- ss + c_k; ss <- fma(x_r, x_r, ss).
//
// Inputs with more than kRmsMaxRisky risky steps (sums that stay below
// 2^-100, ties everywhere) take the plain chain instead, as do non-finite
// inputs (every step after them is risky).
#pragma once

#include "fdm_device.h"

namespace fdm {

constexpr int kRmsThreads = 256;
constexpr int kRmsMaxPer = kHidden / kRmsThreads;  // elements per thread at d = 7168 (28)
constexpr int kRmsMaxRisky = 512;

struct alignas(16) RmsSmem {
  unsigned k[kHidden];        // per element: K_i of a run step, kRmsRisky | (E + 256) for a risky step (16-byte aligned)
  float rx[kRmsMaxRisky];     // risky steps in order: x_r,
  unsigned rq[kRmsMaxRisky];  //   sum of K before r (mod 2^32),
  int re[kRmsMaxRisky];       //   exponent E of P_r (the run before r lies in [2^(E-1), 2^E))
  float rc[kRmsMaxRisky + 1];  // the run added before risky step k (and after the last)
  float wf[4];
  unsigned wk[4];
  int wr[4];
  float ss;
};
constexpr unsigned kRmsRisky = 0x80000000u;  // flag of a risky step's slot; bits 0-15: its E + 256

// DPP move of a 32-bit value (lanes without a source receive 0).
template <int CTRL, int ROW_MASK, typename T>
__device__ __forceinline__ T dpp_zero(T x) {
  int bits;
  __builtin_memcpy(&bits, &x, 4);
  bits = __builtin_amdgcn_update_dpp(0, bits, CTRL, ROW_MASK, 0xF, false);
  T r;
  __builtin_memcpy(&r, &bits, 4);
  return r;
}

// Inclusive scan over the 64 lanes of a wave by DPP: row shifts 1, 2, 4, 8
// within each row of 16 lanes, then row_bcast 15 / 31 carry rows 0 -> 1,
// 2 -> 3 and 1 -> 2, 3 (lanes without a source add 0).
template <typename T>
__device__ __forceinline__ T wave_scan_incl(T v) {
  v = v + dpp_zero<0x111, 0xF>(v);  // row_shr:1
  v = v + dpp_zero<0x112, 0xF>(v);  // row_shr:2
  v = v + dpp_zero<0x114, 0xF>(v);  // row_shr:4
  v = v + dpp_zero<0x118, 0xF>(v);  // row_shr:8
  v = v + dpp_zero<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v = v + dpp_zero<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

// The lanes before this one within the wave, from the inclusive scan: for
// floats the previous lane's inclusive value (DPP wave_shr:1; lane 0
// receives 0) -- inc - v would cancel where v dominates the earlier lanes
// (an outlier), and the prefix would lose the relative accuracy step 2
// relies on -- for integers inc - v (exact).
template <typename T>
__device__ __forceinline__ T lanes_before(T inc, T v) {
  if constexpr (__is_same(T, float))
    return dpp_zero<0x138, 0xF>(inc);
  else
    return inc - v;
}

// Exclusive prefix over the workgroup (256 threads, thread order) of a
// value; the total in *tot.  Ends with every thread past its reads of the
// wave sums (the array may be reused).
template <typename T>
__device__ __forceinline__ T rms_block_excl(T v, T* wsum, T& tot) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const T inc = wave_scan_incl(v);
  if (lane == 63) wsum[wave] = inc;
  __syncthreads();
  T base = T(0), all = T(0);
#pragma unroll
  for (int w = 0; w < kRmsThreads / 64; ++w) {
    const T s = wsum[w];
    base = w < wave ? base + s : base;
    all = all + s;
  }
  tot = all;
  __syncthreads();
  return base + lanes_before(inc, v);
}

// Two exclusive prefixes at once (one pair of barriers).
__device__ __forceinline__ void rms_block_excl2(unsigned v, int c, unsigned* wv, int* wc, unsigned& ex_v, int& ex_c,
                                                unsigned& tot_v, int& tot_c) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const unsigned iv = wave_scan_incl(v);
  const int ic = wave_scan_incl(c);
  if (lane == 63) {
    wv[wave] = iv;
    wc[wave] = ic;
  }
  __syncthreads();
  unsigned bv = 0, av = 0;
  int bc = 0, ac = 0;
#pragma unroll
  for (int w = 0; w < kRmsThreads / 64; ++w) {
    const unsigned sv = wv[w];
    const int sc = wc[w];
    bv = w < wave ? bv + sv : bv;
    bc = w < wave ? bc + sc : bc;
    av += sv;
    ac += sc;
  }
  tot_v = av;
  tot_c = ac;
  ex_v = bv + (iv - v);
  ex_c = bc + (ic - c);
  __syncthreads();
}

// The sum of squares below for one thread layout: FULL when every thread
// holds kRmsMaxPer elements (d = 7168: straight-line code), else the first
// n slots of xv are the thread's (a uniform test per slot).
template <bool FULL>
__device__ __forceinline__ float rms_sumsq_impl(const float (&xv)[kRmsMaxPer], int d, int n, RmsSmem& sm) {
#pragma clang fp contract(off)
  const int t = threadIdx.x;
  const int i0 = t * n;
  auto mine = [&](int j) { return FULL || j < n; };
  // 1. the approximate prefix before the thread's first element
  float tot = 0.0f;
#pragma unroll
  for (int j = 0; j < kRmsMaxPer; ++j)
    if (mine(j)) tot = tot + xv[j] * xv[j];
  float total_f;
  const float base = rms_block_excl(tot, sm.wf, total_f);
  // 2. classify each step; K of the run steps (or the flagged E of a risky
  //    step) into LDS (the thread's slots as 16-byte stores where they are
  //    whole vectors)
  const float lo_margin = 0.5f * (1.0f + 0x1p-10f);  // frexp mantissa of P_i at least this
  const float hi_margin = 1.0f - 0x1p-10f;           // (P_i + x^2) / 2^E at most this
  float p = base;
  unsigned ksum = 0;
  int nrisky = 0;
  unsigned kk[4];
#pragma unroll
  for (int j = 0; j < kRmsMaxPer; ++j) {
    kk[j & 3] = 0u;
    if (mine(j)) {
      const float x = xv[j];
      const float after = p + x * x;
      int E;
      const float m = frexpf(p, &E);  // p = m 2^E, m in [0.5, 1)
      // x^2 / u = h' + l' exactly (u = 2^(E - 24))
      const float h = x * x;
      const float l = fmaf(x, x, -h);
      const float hq = ldexpf(h, 24 - E), lq = ldexpf(l, 24 - E);
      const float K = rintf(hq);
      const float frac = (hq - K) + lq;
      // every test evaluated (no short circuit): one mask per element, no
      // branches in the unrolled loop
      const bool risky = !(p >= 0x1p-100f) | !(after < 0x1p126f) | !(m >= lo_margin) |
                         !(ldexpf(after, -E) <= hi_margin) | !(fabsf(x) >= 0x1p-40f) |
                         !(fabsf(frac) < 0x1.fffffcp-2f);
      const unsigned k = risky ? (kRmsRisky | (unsigned)(E + 256)) : (unsigned)K;
      kk[j & 3] = k;
      if (!FULL) sm.k[i0 + j] = k;
      ksum += risky ? 0u : k;
      nrisky += risky ? 1 : 0;
      p = after;
    }
    if (FULL && (j & 3) == 3)
      *reinterpret_cast<u32x4*>(&sm.k[i0 + j - 3]) = u32x4{kk[0], kk[1], kk[2], kk[3]};
  }
  unsigned ktot;
  int rtot;
  unsigned kbase;
  int rbase;
  rms_block_excl2(ksum, nrisky, sm.wk, sm.wr, kbase, rbase, ktot, rtot);
  if (rtot > kRmsMaxRisky) {
    // too many risky steps for the list: the plain chain by one lane, over
    // the inputs gathered in LDS (in place of the K values)
#pragma unroll
    for (int j = 0; j < kRmsMaxPer; ++j)
      if (mine(j)) sm.k[i0 + j] = __float_as_uint(xv[j]);
    __syncthreads();
    if (t == 0) {
      float ss = 0.0f;
      for (int i = 0; i < d; ++i) ss = fmaf(__uint_as_float(sm.k[i]), __uint_as_float(sm.k[i]), ss);
      sm.ss = ss;
    }
    __syncthreads();
    return sm.ss;
  }
  // 3. the risky steps in order: x, the K sum before them, the binade of P
  unsigned kq = kbase;
  int r = rbase;
  unsigned kv[kRmsMaxPer];  // every K read before the walk over them: one LDS round trip
#pragma unroll
  for (int j = 0; j < kRmsMaxPer; j += 4) {
    if (FULL) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(&sm.k[i0 + j]);
      kv[j] = v.x;
      kv[j + 1] = v.y;
      kv[j + 2] = v.z;
      kv[j + 3] = v.w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) kv[j + i] = mine(j + i) ? sm.k[i0 + j + i] : 0u;
    }
  }
  if (nrisky > 0) {
#pragma unroll
    for (int j = 0; j < kRmsMaxPer; ++j) {
      if (mine(j)) {
        const unsigned k = kv[j];
        const bool isr = (k & kRmsRisky) != 0u;
        if (isr) {
          sm.rx[r] = xv[j];
          sm.rq[r] = kq;
          sm.re[r] = (int)(k & 0xFFFFu) - 256;
        }
        kq += isr ? 0u : k;
        r += isr ? 1 : 0;
      }
    }
  }
  __syncthreads();
  // 4. the run before each risky step, and the final run, as exact floats
  for (int k = t; k <= rtot; k += kRmsThreads) {
    unsigned q1;
    int E;
    if (k < rtot) {
      q1 = sm.rq[k];
      E = sm.re[k];
    } else {
      q1 = ktot;
      (void)frexpf(total_f, &E);
    }
    const unsigned q0 = k > 0 ? sm.rq[k - 1] : 0u;
    const unsigned run = q1 - q0;  // < 2^24 when not 0: a run stays in one binade
    sm.rc[k] = run ? ldexpf((float)run, E - 24) : 0.0f;
  }
  __syncthreads();
  // 5. the walk: one lane, two dependent operations per risky step
  if (t == 0) {
    float ss = 0.0f;
#pragma unroll 4
    for (int k = 0; k < rtot; ++k) {
      ss = ss + sm.rc[k];
      ss = fmaf(sm.rx[k], sm.rx[k], ss);
    }
    sm.ss = ss + sm.rc[rtot];
  }
  __syncthreads();
  return sm.ss;
}

// The reference's sum of squares of x[0..d) (d <= 7168), as a float, in
// every thread.  Thread t passes its elements t*n .. t*n+n-1 (n = ceil(d /
// 256)) in xv[0..n), zeros for those past d (steps that leave the chain
// unchanged: fma(0, 0, ss) = ss, K = 0).
__device__ __forceinline__ float rms_sumsq_exact(const float (&xv)[kRmsMaxPer], int d, RmsSmem& sm) {
  const int n = (d + kRmsThreads - 1) / kRmsThreads;
  return n == kRmsMaxPer ? rms_sumsq_impl<true>(xv, d, n, sm) : rms_sumsq_impl<false>(xv, d, n, sm);
}

// 1 / sqrt(ss / d + 1e-6) with IEEE operations, as infer.m:371.  HIP's
// float `/` and sqrtf are correctly rounded (clang's default
// -fhip-fp32-correctly-rounded-divide-sqrt); __fsqrt_rn is not (it is the
// hardware square root, off by an ulp for a few percent of inputs).
__device__ __forceinline__ float rms_inv(float ss, int d) {
#pragma clang fp contract(off)
  return 1.0f / sqrtf(ss / (float)d + 1e-6f);
}

// The thread layout of rms_sumsq_exact at d = 7168 (thread t: elements
// 28 t .. 28 t + 27) from coalesced 16-byte loads (thread t: vectors t,
// t + 256, .., each wave instruction one contiguous 1 KB), turned around
// through sm.k: loaded directly, a wave's 16-byte loads lie 112 bytes apart,
// seven times the cache-line requests of the same bytes.  c receives the
// coalesced vectors (times mul when MUL).  sm.k is free again once the
// caller's rms_sumsq_exact passes its first barrier.
template <bool MUL>
__device__ __forceinline__ void rms_stage_7168(const f32x4* __restrict__ x4, float mul, float (&xv)[kRmsMaxPer],
                                               f32x4 (&c)[kRmsMaxPer / 4], RmsSmem& sm) {
  constexpr int kV = kRmsMaxPer / 4;
#pragma unroll
  for (int k = 0; k < kV; ++k) {
    c[k] = x4[threadIdx.x + kRmsThreads * k];
    if (MUL) c[k] = c[k] * mul;
  }
  f32x4* st = reinterpret_cast<f32x4*>(sm.k);
#pragma unroll
  for (int k = 0; k < kV; ++k) st[threadIdx.x + kRmsThreads * k] = c[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kV; ++k) {
    const f32x4 v = st[threadIdx.x * kV + k];
    xv[4 * k] = v.x;
    xv[4 * k + 1] = v.y;
    xv[4 * k + 2] = v.z;
    xv[4 * k + 3] = v.w;
  }
}

// ---- rms_norm: o = x * (1 / sqrt(sum x^2 / d + 1e-6)) * w -------------------------------
// (x = xr * mul elementwise: mul = 1 leaves xr as it is; the attention
// passes the scale its raw projections still owe)
// One workgroup per token.  The sum of squares is the reference's
// sequential fma chain, evaluated bit for bit by rms_sumsq_exact (runs of
// integer steps inside a binade, the steps at binade edges and ties walked
// in order); sqrt and division are IEEE; o = (x * inv) * w as infer.m:372.
// At d = 7168 (16-byte aligned rows) every load is a 16-byte vector load
// issued before the sum, so the row's latency is paid once.
__device__ __forceinline__ void rms_norm_row(const float* __restrict__ xr, const float* __restrict__ w,
                                             float* orow, int d, RmsSmem& sm, float mul = 1.0f) {
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
    for (int k = 0; k < kV; ++k)
      wc[k] = w ? reinterpret_cast<const f32x4*>(w)[threadIdx.x + kRmsThreads * k] : f32x4{1.0f, 1.0f, 1.0f, 1.0f};
    rms_stage_7168<true>(x4, mul, xv, xc, sm);  // xc: the coalesced vectors, for the output
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
    const float v = xr[min(i0 + j, d - 1)] * mul;  // every slot loads; past the row it is a zero step
    xv[j] = (j < n && i0 + j < d) ? v : 0.0f;
  }
  const float inv = rms_inv(rms_sumsq_exact(xv, d, sm), d);
  for (int i = threadIdx.x; i < d; i += kRmsThreads) {
    const float v = (xr[i] * mul) * inv;
    orow[i] = w ? v * w[i] : v;
  }
}

// The exact 1 / rms of x[0..d) = xr * mul (d <= 7168) in every thread of
// the workgroup, as rms_norm_row computes it; read in the thread layout of
// rms_sumsq_exact (16-byte loads at d = 7168 when xr is 16-byte aligned).
__device__ __forceinline__ float rms_norm_inv(const float* __restrict__ xr, int d, RmsSmem& sm, float mul = 1.0f) {
  const int n = (d + kRmsThreads - 1) / kRmsThreads;
  const int i0 = threadIdx.x * n;
  float xv[kRmsMaxPer];
  if (d == kHidden && (reinterpret_cast<uintptr_t>(xr) & 15) == 0) {
    f32x4 c[kRmsMaxPer / 4];
    rms_stage_7168<true>(reinterpret_cast<const f32x4*>(xr), mul, xv, c, sm);
  } else {
#pragma unroll
    for (int j = 0; j < kRmsMaxPer; ++j) {
      const float v = xr[min(i0 + j, d - 1)] * mul;  // every slot loads; past the row it is a zero step
      xv[j] = (j < n && i0 + j < d) ? v : 0.0f;
    }
  }
  return rms_inv(rms_sumsq_exact(xv, d, sm), d);
}

}  // namespace fdm
