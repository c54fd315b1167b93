// route_device.h -- device-side route() of DeepSeek-V3 noaux_tc routing
// (infer.m:920-991) for one token per wave, shared by the router kernels and
// the expert kernels (which finish the exact slot order off the critical
// path).  Every operation is defined so that the result equals the
// reference's sequential C bit for bit:
//  - sigmoid: 1/(1 + expf(-x)) with expf evaluated as a double-precision
//    exp built from fma/mul/add (exp_det) and rounded once; float division
//    and addition are IEEE.
//  - running top-2 per group by a multiset butterfly, group choice by
//    uniform strict-> passes (lowest index wins ties), the replace-the-
//    first-minimum slot scan by ballots that jump straight to the next
//    expert able to displace the current minimum, weights summed in slot
//    order.
#pragma once

#include <climits>

#include "fdm_device.h"

namespace fdm {

__device__ __forceinline__ double exp_det(double x) {
#pragma clang fp contract(off)
  if (x != x) return x;
  if (x > 709.0) return __builtin_inf();
  if (x < -746.0) return 0.0;
  const double inv_ln2 = 1.4426950408889634;
  const double ln2_hi = 0x1.62e42fefa39efp-1;
  const double ln2_lo = 0x1.abc9e3b39803fp-56;
  const double t = x * inv_ln2;
  const double k = floor(t + 0.5);
  double r = fma(-k, ln2_hi, x);
  r = fma(-k, ln2_lo, r);
  const double inv_fact[14] = {1.0,         1.0,          1.0 / 2,       1.0 / 6,
                               1.0 / 24,    1.0 / 120,    1.0 / 720,     1.0 / 5040,
                               1.0 / 40320, 1.0 / 362880, 1.0 / 3628800, 1.0 / 39916800,
                               1.0 / 479001600, 1.0 / 6227020800.0};
  double p = inv_fact[13];
#pragma unroll
  for (int i = 12; i >= 0; --i) p = fma(p, r, inv_fact[i]);
  return ldexp(p, (int)k);
}

__device__ __forceinline__ float sigmoid_det(float x) {
#pragma clang fp contract(off)
  const float e = (float)exp_det((double)(-x));
  return __fdiv_rn(1.0f, 1.0f + e);
}

__device__ __forceinline__ float load_relaxed(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// DPP row shift (row_shr:n) of a float: lanes with no source in their row
// of 16 receive `fill`.
template <int N>
__device__ __forceinline__ float row_shr(float v, float fill) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(fill), __float_as_int(v), 0x110 | N, 0xF, 0xF, false));
}

// DPP row_bcast:15 of a float into rows 1 and 3: their lanes receive lane
// 15 of the row before (rows 0 and 2 keep v).
__device__ __forceinline__ float row_bcast15(float v, float fill) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(fill), __float_as_int(v), 0x142, 0xA, 0xF, false));
}

// Merge two top-2 multisets (a1 >= a2, b1 >= b2).
__device__ __forceinline__ void top2_merge(float& t1, float& t2, float o1, float o2) {
  const float n2 = fmaxf(fminf(t1, o1), fmaxf(t2, o2));
  t1 = fmaxf(t1, o1);
  t2 = n2;
}

// Order-preserving int image of a non-NaN float (-0 and +0 map together);
// NaN maps below every other key, so it never enters a slot.
__device__ __forceinline__ int sort_key(float f) {
  const int b = __float_as_int(f + 0.0f);
  const int k = b >= 0 ? b : b ^ 0x7FFFFFFF;
  return f != f ? INT_MIN : k;  // selects, no branch
}

// Minimum of an int over the whole wave.
__device__ __forceinline__ int wave_min_i32(int v) {
  v = min(v, __builtin_amdgcn_update_dpp(INT_MAX, v, 0x111, 0xF, 0xF, false));
  v = min(v, __builtin_amdgcn_update_dpp(INT_MAX, v, 0x112, 0xF, 0xF, false));
  v = min(v, __builtin_amdgcn_update_dpp(INT_MAX, v, 0x114, 0xF, 0xF, false));
  v = min(v, __builtin_amdgcn_update_dpp(INT_MAX, v, 0x118, 0xF, 0xF, false));
  const int a = __builtin_amdgcn_readlane(v, 15), b = __builtin_amdgcn_readlane(v, 31);
  const int c = __builtin_amdgcn_readlane(v, 47), d = __builtin_amdgcn_readlane(v, 63);
  return min(min(a, b), min(c, d));
}

// The replace-the-first-minimum slot scan of route() (infer.m:970-990).
// vk: order-preserving keys of the masked choices, expert 64j + lane in
// vk[j]; score: the unbiased sigmoid scores.  Slot k lives in lane k (key,
// id, score; lanes >= K hold a key no slot minimum can be).  The next
// candidate is the first later expert whose key beats the current first
// minimum (a ballot), re-evaluated after every insertion.  On return lane
// k (k < K) holds slot k's expert id and normalised weight.
__device__ __forceinline__ void slot_scan(const int vk[4], const float score[4], int K,
                                          float scale, int& id_out, float& w_out) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int init = sort_key(-1e30f);
  // a slot never filled keeps expert 0, as exp_idx starts zeroed
  int skey = lane < K ? init : INT_MAX;
  int sid = 0;
  float ssc = readlane_f(score[0], 0);
  int mu = init, ms = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    unsigned long long cand = __ballot(vk[j] > mu);
    while (cand) {
      const int l = __ffsll((unsigned long long)cand) - 1;
      const int vl = __builtin_amdgcn_readlane(vk[j], l);
      const float sl = readlane_f(score[j], l);
      if (lane == ms) {
        skey = vl;
        sid = 64 * j + l;
        ssc = sl;
      }
      mu = wave_min_i32(skey);
      ms = __ffsll((unsigned long long)__ballot(skey == mu)) - 1;
      const unsigned long long later = (l == 63) ? 0ull : (~0ull << (l + 1));
      cand = __ballot(vk[j] > mu) & later;
    }
  }
  // Weights: unbiased scores of the picks, summed and scaled in slot order.
  float sum = 0.0f;
  for (int k = 0; k < K; ++k) sum += readlane_f(ssc, k);
  const float f = sum > 0.0f ? __fdiv_rn(scale, sum) : 1.0f;
  id_out = sid;
  w_out = sum > 0.0f ? ssc * f : ssc;
}

// The first half of route() for one token held in registers (lane l holds
// the unbiased sigmoid score of expert 64 j + l in score[j], its bias in
// bj[j]): the order-preserving keys of the choices (score + bias) masked to
// the top-4 groups; experts outside them get the key of -1e30.  R1
// geometry: 256 experts, 8 groups of 32; group of expert i = i / 32 =
// 2j + l / 32 (rows 0-1 of register j are group 2j, rows 2-3 group 2j+1).
//  - group top-2 (infer.m:933-941): the running top-2 of a group is the
//    top-2 of the multiset of its choices above -1e30 (NaN never enters),
//    padded with -1e30.  Each row of 16 lanes is reduced by DPP row shifts,
//    then row_bcast:15 folds row 0 into row 1 and row 2 into row 3, leaving
//    the group's pair in lanes 31 and 63.
//  - group choice (infer.m:944-954): four strict-> passes that start from
//    -1e30 select the top 4 of the groups whose sum exceeds -1e30, by value
//    and then lowest index: a group is chosen iff it is eligible and fewer
//    than 4 eligible groups rank above it (computed for all 8 at once).
__device__ __forceinline__ void route_keys(const float score[4], const float bj[4], int vk[4]) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  float choice[4], t1[4], t2[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    choice[j] = score[j] + bj[j];
    t1[j] = choice[j] > -1e30f ? choice[j] : -1e30f;
    t2[j] = -1e30f;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) top2_merge(t1[j], t2[j], row_shr<1>(t1[j], -1e30f), row_shr<1>(t2[j], -1e30f));
#pragma unroll
  for (int j = 0; j < 4; ++j) top2_merge(t1[j], t2[j], row_shr<2>(t1[j], -1e30f), row_shr<2>(t2[j], -1e30f));
#pragma unroll
  for (int j = 0; j < 4; ++j) top2_merge(t1[j], t2[j], row_shr<4>(t1[j], -1e30f), row_shr<4>(t2[j], -1e30f));
#pragma unroll
  for (int j = 0; j < 4; ++j) top2_merge(t1[j], t2[j], row_shr<8>(t1[j], -1e30f), row_shr<8>(t2[j], -1e30f));
#pragma unroll
  for (int j = 0; j < 4; ++j)
    top2_merge(t1[j], t2[j], row_bcast15(t1[j], -1e30f), row_bcast15(t2[j], -1e30f));
  float gs[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    gs[2 * j] = readlane_f(t1[j], 31) + readlane_f(t2[j], 31);
    gs[2 * j + 1] = readlane_f(t1[j], 63) + readlane_f(t2[j], 63);
  }
  float mine = -1e30f;
#pragma unroll
  for (int G = 0; G < 8; ++G) mine = lane == G ? gs[G] : mine;
  int rank = 0;
#pragma unroll
  for (int h = 0; h < 8; ++h) {
    // bitwise, not short-circuit: the && / || form compiles to exec-mask branches
    const int oe = (int)(gs[h] > -1e30f);
    rank += oe & ((int)(gs[h] > mine) | ((int)(gs[h] == mine) & (int)(h < lane)));
  }
  const unsigned selmask = (unsigned)__ballot(lane < 8 && mine > -1e30f && rank < 4);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool in_sel = (selmask >> (2 * j + (lane >> 5))) & 1u;
    vk[j] = in_sel ? sort_key(choice[j]) : sort_key(-1e30f);
  }
}

// route_keys in the "four consecutive experts" layout: lane l holds the
// sigmoid scores of experts 4 l .. 4 l + 3 in score4[m] (their biases in
// bj4[m]), so a group of 32 experts is the eight lanes 8 g .. 8 g + 7.  The
// group's top-2 multiset (infer.m:933-941) is its lanes' local top-2 merged
// by three DPP row shifts inside the eight lanes (a shifted-in value from
// the group before is replaced by -1e30): one dependent chain of three
// steps instead of five steps over four registers.  The top-2 is a multiset,
// so the merge order does not change it, and each group's sum t1 + t2 is
// the same float addition as in route_keys; the group choice and the masked
// keys follow route_keys.  Keys vk4[m] belong to expert 4 l + m.
__device__ __forceinline__ void route_keys4(const float score4[4], const float bj4[4], int vk4[4]) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  float choice[4], a[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    choice[m] = score4[m] + bj4[m];
    a[m] = choice[m] > -1e30f ? choice[m] : -1e30f;
  }
  float t1 = fmaxf(a[0], a[1]), t2 = fminf(a[0], a[1]);
  top2_merge(t1, t2, fmaxf(a[2], a[3]), fminf(a[2], a[3]));
  const int gl = lane & 7;  // lane within the group
  {
    float o1 = row_shr<1>(t1, -1e30f), o2 = row_shr<1>(t2, -1e30f);
    top2_merge(t1, t2, gl >= 1 ? o1 : -1e30f, gl >= 1 ? o2 : -1e30f);
  }
  {
    float o1 = row_shr<2>(t1, -1e30f), o2 = row_shr<2>(t2, -1e30f);
    top2_merge(t1, t2, gl >= 2 ? o1 : -1e30f, gl >= 2 ? o2 : -1e30f);
  }
  {
    float o1 = row_shr<4>(t1, -1e30f), o2 = row_shr<4>(t2, -1e30f);
    top2_merge(t1, t2, gl >= 4 ? o1 : -1e30f, gl >= 4 ? o2 : -1e30f);
  }
  const float gsum = t1 + t2;  // lane 8 g + 7: group g's sum
  float gs[8];
#pragma unroll
  for (int g = 0; g < 8; ++g) gs[g] = readlane_f(gsum, 8 * g + 7);
  float mine = -1e30f;
#pragma unroll
  for (int G = 0; G < 8; ++G) mine = lane == G ? gs[G] : mine;
  int rank = 0;
#pragma unroll
  for (int h = 0; h < 8; ++h) {
    // bitwise, not short-circuit: the && / || form compiles to exec-mask branches
    const int oe = (int)(gs[h] > -1e30f);
    rank += oe & ((int)(gs[h] > mine) | ((int)(gs[h] == mine) & (int)(h < lane)));
  }
  const unsigned selmask = (unsigned)__ballot(lane < 8 && mine > -1e30f && rank < 4);
  // a bit blend, not a conditional: the compiler would branch on in_sel
  const int sel = -(int)((selmask >> (lane >> 3)) & 1u);
  const int kf = sort_key(-1e30f);
#pragma unroll
  for (int m = 0; m < 4; ++m) vk4[m] = (sort_key(choice[m]) & sel) | (kf & ~sel);
}

// route() for one token, executed by one full wave with the sigmoid scores
// in registers: exact reference selection, tie rules and slot order.  Lane
// k (k < K) receives slot k's expert id and weight.
__device__ __forceinline__ void route_exact_lane(const float score[4], const float bj[4], int K,
                                        float scale, int& id, float& wv) {
  int vk[4];
  route_keys(score, bj, vk);
  id = 0;
  wv = 0.0f;
  slot_scan(vk, score, K, scale, id, wv);
}

__device__ __forceinline__ void route_scores_wave(const float score[4], const float bj[4], int K, float scale,
                                  int* __restrict__ idx_out, float* __restrict__ w_out) {
  const int lane = threadIdx.x & 63;
  int id;
  float wv;
  route_exact_lane(score, bj, K, scale, id, wv);
  if (lane < K) {
    idx_out[lane] = id;
    w_out[lane] = wv;
  }
}

// route() reading the token's logits (and bias) from memory.
__device__ __forceinline__ void route_wave(const float* logits, const float* bias, int K, float scale,
                          int* __restrict__ idx_out, float* __restrict__ w_out) {
  const int lane = threadIdx.x & 63;
  float score[4], bj[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    score[j] = sigmoid_det(load_relaxed(logits + 64 * j + lane));
    bj[j] = bias ? bias[64 * j + lane] : 0.0f;
  }
  route_scores_wave(score, bj, K, scale, idx_out, w_out);
}

// The SET of experts route() selects.  The sequential slot scan always
// ends holding K elements that are >= everything it does not hold, so when
// the K-th largest key T is unique among the candidates the set is exactly
// {key >= T}.  T is found by a radix search over the order-preserving keys
// (as unsigned, MSB first: keep bit b when at least K keys are >= the
// prefix with it), counting with ballots; the search stops as soon as
// exactly K keys are >= the prefix, which already fixes the set.  Returns
// false (the caller then runs the exact scan) when the K-th key is tied
// with a candidate left out, or when fewer than K candidates exceed -1e30.
// On success lane k (k < K) receives the k-th expert of the set, in
// (register j, lane) order -- a provisional order.
__device__ __forceinline__ bool topk_set(const int vk[4], int K, int& id_out) {
  const int lane = threadIdx.x & 63;
  unsigned u[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) u[j] = (unsigned)vk[j] ^ 0x80000000u;
  unsigned T = 0;
  int nT = 256;
  for (int b = 31; b >= 0 && nT != K; --b) {
    const unsigned c = T | (1u << b);
    const unsigned long long m0 = __ballot(u[0] >= c), m1 = __ballot(u[1] >= c);
    const unsigned long long m2 = __ballot(u[2] >= c), m3 = __ballot(u[3] >= c);
    const int n = (__popcll(m0) + __popcll(m1)) + (__popcll(m2) + __popcll(m3));
    if (n >= K) {
      T = c;
      nT = n;
    }
  }
  const unsigned floor_u = (unsigned)sort_key(-1e30f) ^ 0x80000000u;
  if (nT != K || T <= floor_u) return false;
  // compaction: the selected lane at position p pushes its id to lane p
  int id = 0, base = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const unsigned long long sel = __ballot(u[j] >= T);
    const int cnt = __popcll(sel);
    const bool mine = (sel >> lane) & 1ull;
    const int pos = base + (int)__builtin_amdgcn_mbcnt_hi((unsigned)(sel >> 32),
                                                          __builtin_amdgcn_mbcnt_lo((unsigned)sel, 0u));
    const int got = __builtin_amdgcn_ds_permute((mine ? pos : 63) * 4, 64 * j + lane);
    id = (lane >= base && lane < base + cnt) ? got : id;
    base += cnt;
  }
  id_out = id;
  return true;
}

// ---- the expert set, largest first, published slot by slot -------------------------------
// Maximum of an int over the whole wave (uniform result): DPP row shifts
// leave each row's maximum in its lane 15, row_bcast:15 folds rows 0 and 2
// into rows 1 and 3, row_bcast:31 folds row 1 into rows 2 and 3, so lane
// 63 holds the maximum; one readlane.
__device__ __forceinline__ int wave_max_i32(int v) {
  v = max(v, __builtin_amdgcn_update_dpp(INT_MIN, v, 0x111, 0xF, 0xF, false));
  v = max(v, __builtin_amdgcn_update_dpp(INT_MIN, v, 0x112, 0xF, 0xF, false));
  v = max(v, __builtin_amdgcn_update_dpp(INT_MIN, v, 0x114, 0xF, 0xF, false));
  v = max(v, __builtin_amdgcn_update_dpp(INT_MIN, v, 0x118, 0xF, 0xF, false));
  v = max(v, __builtin_amdgcn_update_dpp(INT_MIN, v, 0x142, 0xA, 0xF, false));
  v = max(v, __builtin_amdgcn_update_dpp(INT_MIN, v, 0x143, 0xC, 0xF, false));
  return __builtin_amdgcn_readlane(v, 63);
}

// ---- the eight largest packed keys of the wave, by a merge network -------------------
// Packed keys are unique, so "largest" is a strict order.  cx keeps the
// larger of two in a, the smaller in b.
__device__ __forceinline__ void cx(int& a, int& b) {
  const int hi = max(a, b);
  b = min(a, b);
  a = hi;
}

// Sorts a bitonic sequence of eight, largest first.
__device__ __forceinline__ void bitonic8(int (&t)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) cx(t[i], t[i + 4]);
#pragma unroll
  for (int i = 0; i < 8; i += 4) {
    cx(t[i], t[i + 2]);
    cx(t[i + 1], t[i + 3]);
  }
#pragma unroll
  for (int i = 0; i < 8; i += 2) cx(t[i], t[i + 1]);
}

// The partner's list by one DPP pattern (lanes it does not reach get
// INT_MIN), merged into the lane's own: the eight largest of both lists
// (each sorted, largest first) are max(t[i], p[7 - i]), a bitonic sequence.
template <int CTRL, int ROWS>
__device__ __forceinline__ void merge8(int (&t)[8]) {
  int p[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) p[i] = __builtin_amdgcn_update_dpp(INT_MIN, t[i], CTRL, ROWS, 0xF, false);
#pragma unroll
  for (int i = 0; i < 8; ++i) t[i] = max(t[i], p[7 - i]);
  bitonic8(t);
}

// The eight largest of the wave's 256 keys (lane l holds k[0..3]), largest
// first, in t[0..7] of lanes 48-63 (INT_MIN where fewer than eight keys
// exist).  Each lane sorts its four; lanes l and l^1 merge their fours into
// one sorted eight (quad_perm [1,0,3,2]); then lists merge with l^2
// (quad_perm [2,3,0,1]), the other quad of the half row (row_half_mirror),
// the other half row (row_mirror), row 0 into 1 and row 2 into 3
// (row_bcast:15) and row 1 into 3 (row_bcast:31).  About 200 VALU
// operations and no scalar round trip: every slot is known at once.
__device__ __forceinline__ void top8_wave(const int (&k)[4], int (&t)[8]) {
  int a[4] = {k[0], k[1], k[2], k[3]};
  cx(a[0], a[1]);
  cx(a[2], a[3]);
  cx(a[0], a[2]);
  cx(a[1], a[3]);
  cx(a[1], a[2]);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    t[i] = a[i];
    // the partner's four, reversed: a bitonic sequence of eight
    t[7 - i] = __builtin_amdgcn_update_dpp(INT_MIN, a[i], 0xB1, 0xF, 0xF, false);
  }
  bitonic8(t);
  merge8<0x4E, 0xF>(t);   // quad_perm [2,3,0,1]
  merge8<0x141, 0xF>(t);  // row_half_mirror
  merge8<0x140, 0xF>(t);  // row_mirror
  merge8<0x142, 0xA>(t);  // row_bcast:15 into rows 1 and 3
  merge8<0x143, 0xC>(t);  // row_bcast:31 into rows 2 and 3
}

// The set route() selects (scores and biases in both layouts: score[j] /
// bj[j] of expert 64 j + lane, score4[m] / bj4[m] of expert 4 lane + m).
// Keys are PACKED: the order-preserving key's
// upper 24 bits, then 255 - expert id, so the keys are unique and each
// names its expert (the lowest id first among equal truncated keys).
// Truncation is monotone, so the K largest packed keys are the reference's
// set of the K largest full keys whenever the K-th and (K+1)-th TRUNCATED
// keys differ: everything selected is then strictly above everything left,
// and route()'s scan always keeps the keys strictly above its K-th.  Which
// of several equal keys the scan keeps depends on its slot order, so when
// those two truncated keys are equal (full keys tied, or within 256 units
// of the last place), or fewer than K keys exceed -1e30, the exact scan
// decides.  publish(slot, id) is called by every lane of the wave; a lane
// with slot < 0 has nothing to publish.
//  K <= 8: the eight largest by a merge network (top8_wave), every slot
//    published at once by lanes 48 .. 48 + K - 1.
//  K > 8: repeated extraction of the largest key, K + 1 times (one wave
//    maximum each); slot s (the s-th extraction) is certain, and published,
//    as soon as a strictly smaller truncated key follows it.
// In the ambiguous case the slots not yet published receive the rest of
// the reference's (multi)set from the exact scan.
template <typename Publish>
__device__ __forceinline__ void route_set_publish(const float score[4], const float bj[4], const float score4[4],
                                                  const float bj4[4], int K, Publish&& publish) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  // the set from the four-consecutive-experts layout (route_keys4); the
  // exact scan of the ambiguous case below takes the 64 j + lane layout
  int vk4[4];
  route_keys4(score4, bj4, vk4);
  const int floor = sort_key(-1e30f);
  int pk[4];
  bool near_floor = false;  // a candidate whose truncated key is the floor's
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const bool cand = vk4[m] > floor;
    near_floor = near_floor || (cand && (vk4[m] >> 8) == (floor >> 8));
    pk[m] = (cand && (vk4[m] >> 8) != (floor >> 8)) ? ((vk4[m] & ~255) | (255 - (4 * lane + m))) : INT_MIN;
  }
  bool ambiguous = __ballot(near_floor) != 0;
  int ext = 0;    // extraction: lane k holds the k-th extracted expert
  int n_pub = 0;  // slots 0 .. n_pub-1 published
  if (K <= 8) {
    if (!ambiguous) {
      int t[8];
      top8_wave(pk, t);
      int tk = t[0], tn = t[0];  // the K-th and (K+1)-th largest (lanes 48-63)
#pragma unroll
      for (int i = 1; i < 8; ++i) {
        tk = i == K - 1 ? t[i] : tk;
        tn = i == K ? t[i] : tn;
      }
      const int kth = __builtin_amdgcn_readlane(tk, 63);
      if (K < 8) {
        const int next = __builtin_amdgcn_readlane(tn, 63);
        ambiguous = kth == INT_MIN || (next != INT_MIN && (next >> 8) == (kth >> 8));
      } else {
        // no ninth key shares the eighth's truncated prefix: exactly eight
        // keys have a prefix >= it (non-candidates, INT_MIN, lie below every
        // candidate's prefix); ballots and counts instead of a wave maximum
        const int kp = kth >> 8;
        int cnt = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) cnt += __popcll(__ballot((pk[j] >> 8) >= kp));
        ambiguous = kth == INT_MIN || cnt != 8;
      }
      if (!ambiguous) {
        const int s = lane - 48;
        int v = t[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) v = s == i ? t[i] : v;
        publish((s >= 0 && s < K) ? s : -1, 255 - (v & 255));
        return;
      }
    }
  } else {
    int m = max(max(pk[0], pk[1]), max(pk[2], pk[3]));
    int prev_t = INT_MAX;
    for (int k = 0; k <= K && !ambiguous; ++k) {
      const int wm = wave_max_i32(m);
      if (wm == INT_MIN) {
        ambiguous = k < K;  // fewer than K candidates
        break;
      }
      const int wt = wm >> 8;
      if (k == K) {
        ambiguous = wt == prev_t;  // the K-th truncated key is tied with the (K+1)-th
        break;
      }
      if (k > 0 && prev_t > wt) {
        // every slot so far holds a truncated key >= prev_t > wt: all certain
        for (int s = n_pub; s < k; ++s) publish(lane == 0 ? s : -1, __builtin_amdgcn_readlane(ext, s));
        n_pub = k;
      }
      prev_t = wt;
      if (lane == k) ext = 255 - (wm & 255);
#pragma unroll
      for (int j = 0; j < 4; ++j) pk[j] = pk[j] == wm ? INT_MIN : pk[j];
      m = max(max(pk[0], pk[1]), max(pk[2], pk[3]));
    }
    if (!ambiguous) {
      for (int s = n_pub; s < K; ++s) publish(lane == 0 ? s : -1, __builtin_amdgcn_readlane(ext, s));
      return;
    }
  }
  // Ambiguous: the exact scan gives the reference's slots (lane k: slot k's
  // id; slots never filled hold expert 0, possibly several times).  The
  // published experts are strictly above the K-th key, so each is in it;
  // match each published slot to one exact slot and hand the unmatched
  // exact slots to the remaining slots.
  int vk[4];
  route_keys(score, bj, vk);
  int eid;
  float ew;
  slot_scan(vk, score, K, 2.5f, eid, ew);
  bool matched = lane >= K;
  for (int s = 0; s < n_pub; ++s) {
    const int pid = __builtin_amdgcn_readlane(ext, s);
    const unsigned long long hit = __ballot(!matched && eid == pid);
    if (hit && lane == __ffsll(hit) - 1) matched = true;
  }
  unsigned long long rest = __ballot(!matched);
  for (int s = n_pub; s < K && rest; ++s) {
    const int l = __ffsll(rest) - 1;
    publish(lane == 0 ? s : -1, __builtin_amdgcn_readlane(eid, l));
    rest &= rest - 1;
  }
}

// ---- the exact slot order without the sequential scan ---------------------------------------
// The scan of slot_scan keeps, after each expert, the top-K of the keys seen
// so far: expert e ENTERS a slot iff fewer than K earlier experts have a key
// >= its own (and its key exceeds -1e30).  Among the entering experts
// x_1, x_2, ... (index order) the first K fill slots 0 .. K-1 in order (the
// empty slots are the first minima); each later x_m replaces the current
// minimum, i.e. the earlier entry with exactly K-1 larger earlier entries,
// and takes over its slot.  A slot ends with its last entry.  With all
// entering keys distinct this reproduces the scan exactly; otherwise (or
// with more than 63 entries) the scan itself runs.
struct __attribute__((aligned(16))) RouteScratch {
  int key[256];    // order-preserving keys of the masked choices (route_keys)
  float sc[256];   // unbiased sigmoid scores
  int enter[256];  // 1: the expert enters a slot at some point
};

// Four waves (threads t < 256, expert e = t): the enter flag of every expert.
// Each wave scans the keys of experts below its last one (a uniform bound).
__device__ __forceinline__ void route_enter_flags_aux(RouteScratch& r, int K, int t) {
  const int e = t, ke = r.key[e];
  const int n4 = 16 * ((t >> 6) + 1);  // 4-key steps covering experts 0 .. 64 w + 63
  const int4* k4 = reinterpret_cast<const int4*>(r.key);
  int cnt = 0;
  for (int i = 0; i < n4; ++i) {
    const int4 v = k4[i];
    const int j = 4 * i;
    cnt += (j + 0 < e && v.x >= ke) ? 1 : 0;
    cnt += (j + 1 < e && v.y >= ke) ? 1 : 0;
    cnt += (j + 2 < e && v.z >= ke) ? 1 : 0;
    cnt += (j + 3 < e && v.w >= ke) ? 1 : 0;
  }
  r.enter[e] = (ke > sort_key(-1e30f) && cnt < K) ? 1 : 0;
}

// Wave 0, after route_enter_flags_aux: lane k (k < K) receives slot k's expert id
// and weight, as slot_scan (vk, score: the wave's registers for the fallback).
__device__ __forceinline__ void route_exact_slots(const RouteScratch& r, const int vk[4], const float score[4],
                                                  int K, float scale, int& id_out, float& w_out) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  // compaction of the entering experts, in index order: entry i in lane i
  int key = INT_MIN, id = 0, E = 0;
  float sc = 0.0f;
  bool fits = true;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const unsigned long long m = __ballot(r.enter[64 * j + lane] != 0);
    const int n = __popcll(m);
    if (E + n > 63) fits = false;  // lane 63 takes the pushes of unselected lanes
    if (fits) {
      const bool mine = (m >> lane) & 1ull;
      const int pos = E + (int)__builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u));
      const int src = 64 * j + lane;
      const int kk = __builtin_amdgcn_ds_permute((mine ? pos : 63) * 4, r.key[src]);
      const int ii = __builtin_amdgcn_ds_permute((mine ? pos : 63) * 4, src);
      const int ss = __builtin_amdgcn_ds_permute((mine ? pos : 63) * 4, __float_as_int(r.sc[src]));
      if (lane >= E && lane < E + n) {
        key = kk;
        id = ii;
        sc = __int_as_float(ss);
      }
    }
    E += n;
  }
  bool tie = !fits;
  int cnt = 0;     // entries before the current one with a larger key (lanes < m)
  int slot = -1;
  for (int m = 0; m < E && !tie; ++m) {
    const int km = __builtin_amdgcn_readlane(key, m);
    const bool before = lane < m;
    tie = __ballot(before && key == km) != 0ull;
    const int larger = __popcll(__ballot(before && key > km));
    int sm;
    if (m < K) {
      sm = m;
    } else {
      const unsigned long long ev = __ballot(before && cnt == K - 1);
      tie = tie || __popcll(ev) != 1;
      sm = __builtin_amdgcn_readlane(slot, ev ? __ffsll((unsigned long long)ev) - 1 : 0);
    }
    if (lane == m) {
      slot = sm;
      cnt = larger;
    }
    if (before && km > key) ++cnt;
  }
  if (tie) {
    slot_scan(vk, score, K, scale, id_out, w_out);
    return;
  }
  // slot k's last entry; a slot never filled keeps expert 0 (and its score)
  int sid = 0;
  float ssc = readlane_f(score[0], 0);
  for (int k = 0; k < K; ++k) {
    const unsigned long long b = __ballot(lane < E && slot == k);
    if (b) {
      const int last = 63 - __clzll(b);
      const int idk = __builtin_amdgcn_readlane(id, last);
      const float sck = readlane_f(sc, last);
      if (lane == k) {
        sid = idk;
        ssc = sck;
      }
    }
  }
  float sum = 0.0f;
  for (int k = 0; k < K; ++k) sum += readlane_f(ssc, k);
  const float f = sum > 0.0f ? __fdiv_rn(scale, sum) : 1.0f;
  id_out = sid;
  w_out = sum > 0.0f ? ssc * f : ssc;
}

}  // namespace fdm
