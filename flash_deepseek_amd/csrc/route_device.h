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

// Merge two top-2 multisets (a1 >= a2, b1 >= b2).
__device__ __forceinline__ void top2_merge(float& t1, float& t2, float o1, float o2) {
  const float n2 = fmaxf(fminf(t1, o1), fmaxf(t2, o2));
  t1 = fmaxf(t1, o1);
  t2 = n2;
}

// Order-preserving int image of a non-NaN float (-0 and +0 map together);
// NaN maps below every other key, so it never enters a slot.
__device__ __forceinline__ int sort_key(float f) {
  if (f != f) return INT_MIN;
  const int b = __float_as_int(f + 0.0f);
  return b >= 0 ? b : b ^ 0x7FFFFFFF;
}

// Maximum of an int over the whole wave (DPP within rows of 16, then the
// four row results).
__device__ __forceinline__ int wave_max_i32(int v) {
  v = max(v, __builtin_amdgcn_update_dpp(INT_MIN, v, 0x111, 0xF, 0xF, false));
  v = max(v, __builtin_amdgcn_update_dpp(INT_MIN, v, 0x112, 0xF, 0xF, false));
  v = max(v, __builtin_amdgcn_update_dpp(INT_MIN, v, 0x114, 0xF, 0xF, false));
  v = max(v, __builtin_amdgcn_update_dpp(INT_MIN, v, 0x118, 0xF, 0xF, false));
  const int a = __builtin_amdgcn_readlane(v, 15), b = __builtin_amdgcn_readlane(v, 31);
  const int c = __builtin_amdgcn_readlane(v, 47), d = __builtin_amdgcn_readlane(v, 63);
  return max(max(a, b), max(c, d));
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
// 2j + l / 32.
__device__ __forceinline__ void route_keys(const float score[4], const float bj[4], int vk[4]) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  float choice[4];
  float gs[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    choice[j] = score[j] + bj[j];
    // running top-2 of a group = top-2 of the multiset of its choices that
    // exceed -1e30 (NaN never enters), padded with -1e30: reduce each row of
    // 16 lanes by DPP, then merge the two rows of the group
    float t1 = choice[j] > -1e30f ? choice[j] : -1e30f;
    float t2 = -1e30f;
    top2_merge(t1, t2, row_shr<1>(t1, -1e30f), row_shr<1>(t2, -1e30f));
    top2_merge(t1, t2, row_shr<2>(t1, -1e30f), row_shr<2>(t2, -1e30f));
    top2_merge(t1, t2, row_shr<4>(t1, -1e30f), row_shr<4>(t2, -1e30f));
    top2_merge(t1, t2, row_shr<8>(t1, -1e30f), row_shr<8>(t2, -1e30f));
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      float a1 = readlane_f(t1, 32 * half + 15), a2 = readlane_f(t2, 32 * half + 15);
      const float b1 = readlane_f(t1, 32 * half + 31), b2 = readlane_f(t2, 32 * half + 31);
      top2_merge(a1, a2, b1, b2);
      gs[2 * j + half] = a1 + a2;
    }
  }
  unsigned selmask = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    int best = -1;
    float bs = -1e30f;
#pragma unroll
    for (int G = 0; G < 8; ++G) {
      if (!((selmask >> G) & 1u) && gs[G] > bs) {
        bs = gs[G];
        best = G;
      }
    }
    if (best >= 0) selmask |= 1u << best;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool in_sel = (selmask >> (2 * j + (lane >> 5))) & 1u;
    vk[j] = in_sel ? sort_key(choice[j]) : sort_key(-1e30f);
  }
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

// The SET of experts route() selects, found in parallel: K extractions of
// the wave maximum of the masked keys.  The sequential slot scan always
// ends holding K elements that are >= everything it does not hold, so when
// the K-th largest key is unique among the candidates the set is exactly
// the K extracted experts.  Returns false (the caller then runs the exact
// scan) when the K-th key is tied with a candidate left out, or when fewer
// than K candidates exceed -1e30.  On success lane k (k < K) receives the
// k-th extracted expert id; the order (descending key) is provisional.
__device__ __forceinline__ bool topk_set(const int vk_in[4], int K, int& id_out) {
  const int lane = threadIdx.x & 63;
  const int floor_key = sort_key(-1e30f);
  int v[4] = {vk_in[0], vk_in[1], vk_in[2], vk_in[3]};
  int id = 0, m = INT_MIN;
  for (int k = 0; k < K; ++k) {
    m = wave_max_i32(max(max(v[0], v[1]), max(v[2], v[3])));
    if (m <= floor_key) return false;
    int pick = -1;
#pragma unroll
    for (int j = 3; j >= 0; --j) {
      const unsigned long long b = __ballot(v[j] == m);
      if (b) pick = 64 * j + __ffsll(b) - 1;  // lowest expert index holding m
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)  // constant indices only: v stays in registers
      if (j == (pick >> 6) && lane == (pick & 63)) v[j] = INT_MIN;
    if (lane == k) id = pick;
  }
  const bool tie = __ballot(v[0] == m || v[1] == m || v[2] == m || v[3] == m) != 0ull;
  id_out = id;
  return !tie;
}

// Critical-path routing for the batch-1 layer: group limit and the expert
// set (topk_set) from the sigmoid scores; lane k (k < K) receives the k-th
// expert of the set.  When the set is ambiguous (a tie at the K-th key, or
// fewer than K candidates), the exact reference scan runs instead and the
// lanes hold the reference slot order.
__device__ __forceinline__ int route_set_lane(const float score[4], const float bj[4], int K) {
#pragma clang fp contract(off)
  int vk[4];
  route_keys(score, bj, vk);
  int id = 0;
  const bool ok = topk_set(vk, K, id);
  if (!ok) {
    float wv;
    slot_scan(vk, score, K, 2.5f, id, wv);
  }
  return id;
}

__device__ __forceinline__ void route_set_wave(const float score[4], const float bj[4], int K,
                                      int* __restrict__ prov_idx) {
  const int lane = threadIdx.x & 63;
  const int id = route_set_lane(score, bj, K);
  if (lane < K) prov_idx[lane] = id;
}

}  // namespace fdm
