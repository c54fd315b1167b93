// layer_kernel.hip -- the whole batch-1 MoE layer of one token in ONE
// launch: router logits (infer.m:350-353), route() (infer.m:920-991), the
// routed and shared experts' gate/up + SwiGLU and down (encode_expert,
// infer.m:1559-1575, for every slot), the combine moe += w_k * E_k
// (infer.m:1689-1695) and the residual hidden = h_in + moe + shared
// (infer.m:1922).
//
// Why one launch.  At batch 1 the layer is a chain of small dependent
// steps (logits -> route -> expert weights -> activations -> down ->
// combine).  As separate launches each step pays a dispatch ramp and a
// drain, and no weight of a later step is fetched before the earlier step
// has ended.  Here each workgroup is one item of an ordered work list:
//
//   with a norm weight: the fused rms_norm of the hidden state (1)
//   digits of h_post (28: four 64-element groups each)
//   router row e (256)
//   route: the expert set (1);  the exact route() (1)
//   shared expert: gate/up items of both column parts, then the digit
//     records of its activations (one item per part)
//   routed experts, part-major: gate/up items of part q of every slot, then
//     the down items of part q - lag of every slot, q = 0, 1, ...; a down
//     item makes its part's activation records itself from the tagged
//     activations (no digit item between: one coherent round trip less on
//     the tail)
//   final items: the shared expert's down rows and the combine of the
//     same rows (224)
//
// Every routed down matrix is split into two column parts: down part p of a
// slot needs only the slot's activations of part p, so the downs of part 0
// stream alongside the gate/up items of part 1 instead of waiting for the
// slot's last activation.  A slot's expert output is its part sums added in
// part order.  (Measured on MI355X: 2 parts, lag 1 beat 1, 4 and 8 parts and
// lags 0 and 2.)  The shared expert's down rows are the last bytes of the
// list: its activations are ready long before, so the final items contract
// them while the last routed down items finish, then combine.  (The shared
// expert's gate/up items request their weights before they wait for the
// digits: they fill the front of the launch while the router rows, the
// route and -- with the fused rms_norm -- the norm are in flight.)
//
// Items only wait for items earlier in the list, and a waiting item has
// already issued every weight load it can (down tiles load their weights
// before they wait for the activations).  Workgroups are dispatched in
// list order within each XCD, so the earliest unfinished item is always
// resident or dispatchable and never waits on anything unfinished: the
// grid drains.  Every wait is bounded as well: one that times out records
// the call's epoch in the error flag, which releases every other wait, so
// the launch always completes (the host reports the error on its next
// sync).
//
// Hand-off.  Under full HBM streaming every round trip to the coherence
// point costs microseconds, so an item must not chain store
// acknowledgements, counters and flags.  Values crossing workgroups are
// therefore TAGGED: a 64-bit word {epoch, payload} written with one
// agent-scope store and read with agent-scope loads; the reader's load is
// its own readiness check (tag == this call's epoch), the writer never
// waits, and nothing is ever cleared.  Only the 23 KB digit record of
// h_post is published untagged, behind a flag set by the last of its 28
// producers, and staged with 16-byte coherent loads.
//
// Memory ordering.  Every hand-off is a relaxed agent-scope store read by
// relaxed agent-scope loads; there is no release/acquire pair.  What makes
// a tagged word safe is that payload and tag are one 64-bit store, which
// the memory system performs as a single access: a reader that sees the
// tag sees the payload written with it.  The untagged digit record relies
// on the store counter instead: a wave's stores are complete (acknowledged
// by the coherence point) once s_waitcnt has counted them down, which every
// producer waits for before it bumps the arrival counter; the last arrival
// then sets the flag, and a reader issues its record loads only after its
// flag load has returned the epoch, so they cannot observe the record
// before its stores completed.  The agent-scope (sc1) cache policy of all
// these accesses bypasses the non-coherent per-XCD caches, so no stale line
// of an earlier launch is read.
#include "fdm_internal.h"
#include "rms_device.h"
#include "route_device.h"

namespace fdm {

namespace {

constexpr int kStride = kLayerStride;        // ints between counters / flags (256 B)
constexpr int kRows = 256;                   // router rows (R1 experts)
constexpr int kXdItems = kHidden / 64 / 4;   // 28 digit items of 4 groups
constexpr int kGuTileRows = 8;               // gate (and up) rows per gate/up tile
#ifndef FDM_LAYER_PARTS
#define FDM_LAYER_PARTS 2  // measured on MI355X: 2 parts, lag 1, one tile per item
#endif
#ifndef FDM_LAYER_LAG
#define FDM_LAYER_LAG 1
#endif
#ifndef FDM_LAYER_GUPER
#define FDM_LAYER_GUPER 1
#endif
// Column parts of every down matrix: part p of slot s needs only the slot's
// activations kPartCols p .. kPartCols (p + 1) - 1, so it runs while gate/up
// of the slot's later rows is still streaming.
constexpr int kParts = FDM_LAYER_PARTS;
static_assert(kParts == 1 || kParts == 2 || kParts == 4 || kParts == 8, "parts: 1, 2, 4 or 8");
static_assert(kParts <= kLayerMaxParts, "tagged eo holds kLayerMaxParts parts");
constexpr int kLag = FDM_LAYER_LAG;          // down parts follow gate/up parts this many parts later
static_assert(kLag >= 0 && kLag <= kParts, "lag: 0 .. parts");
constexpr int kGuPer = FDM_LAYER_GUPER;      // gate/up tiles per work item
constexpr int kPartCols = kFfn / kParts;     // activations per part
constexpr int kPartGroups = kPartCols / 64;  // digit records per part
constexpr int kGuPerPart = kPartCols / kGuTileRows / kGuPer;  // gate/up items per (slot, part)
static_assert(kGuPerPart * kGuTileRows * kGuPer == kPartCols, "gate/up items tile a part");
// Q4_K down item: one lane per 64-element group of a row's part, kDnRowsQ4L
// rows per lane.  Q6_K down item: one lane per 128-element half block.
#ifndef FDM_ACT_DIRECT
#define FDM_ACT_DIRECT 1
#endif
#ifndef FDM_LAYER_DNROWS
#define FDM_LAYER_DNROWS 7
#endif
constexpr int kDnLanesQ4 = kPartGroups;                     // lanes per row
constexpr int kDnRowsQ4L = FDM_LAYER_DNROWS;                // rows per lane
constexpr int kDnRowsQ4 = 4 * kDnRowsQ4L * (64 / kDnLanesQ4);  // rows per item (448)
constexpr int kDnLanesQ6 = kPartCols / 128;
constexpr int kDnRowsQ6L = 2;
constexpr int kDnRowsQ6 = 4 * kDnRowsQ6L * (64 / kDnLanesQ6);  // 256
static_assert(kHidden % kDnRowsQ4 == 0 && kHidden % kDnRowsQ6 == 0, "down items tile the rows");
__host__ __device__ constexpr int dn_per_part(bool q6) { return kHidden / (q6 ? kDnRowsQ6 : kDnRowsQ4); }

// flag and counter slots (units of kStride)
constexpr int kFlagXd = 0;
constexpr int kFlagErr = kLayerFlagErr;
constexpr int kCntXd = 0;

struct LayerSmem {
  union {
    XGroup xs[kHidden / 64];  // digits of h_post (gate/up) or of a part's activations (down)
    struct {
      XGroup xs[kFfn / 64];                          // the shared activations' digit records
      float v[2 * (kLayerMaxSlots - 1) * 32];        // the routed part outputs of the item's rows
      float esh[32];                                 // the shared expert's output of each row
    } fin;                                           // final items
    RmsSmem rms;              // the fused rms_norm (router rows and digit items)
    float ssc[256];           // the route item: scores handed from a polling wave to wave 0
  };
  float red[4];
  float inv;                  // the fused rms_norm's 1 / rms
  float cw[kLayerMaxSlots];   // combine: route() weights in slot order
  int cperm[kLayerMaxSlots];  // combine: the expert-set slot of each
  int eid;                  // expert of the item's slot
  int sflag;                // the route item: 0 waiting, 1 scores in ssc, 2 gave up
};

// Whole-workgroup wait: every thread runs try_once() (its share of the
// loads and checks) until all of them succeed.  Gives up after a.spin_limit
// rounds, or when another workgroup already gave up (looked at every 64th
// round: each look is one more round trip), recording the epoch in the
// error flag.  Returns false on giving up.
template <typename F>
__device__ __forceinline__ bool poll_all(const LayerArgs& a, F&& try_once) {
  unsigned* err = a.flags + kStride * kFlagErr;
  for (unsigned n = 0;; ++n) {
    if (__syncthreads_and(try_once())) return true;
    int give_up = 0;
    if (threadIdx.x == 0)
      give_up = n >= a.spin_limit || ((n & 63) == 63 && load_u32_agent(err) == a.epoch);
    if (__syncthreads_or(give_up)) {
      if (threadIdx.x == 0) store_u32_agent(err, a.epoch);
      return false;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}


__device__ __forceinline__ const uint8_t* expert_blob(const LayerArgs& a, int e) {
  if (e < 0 || e >= a.n_experts) return nullptr;  // invalid id: expert contributes 0
  return a.experts + (size_t)e * a.expert_size;
}

// Thread 0 waits for the digits of h_post and, for a routed slot, for the
// slot's expert; the expert id lands in sm.eid.  (One tagged flag per digit
// item, polled by 28 threads, measured slower: every waiting gate/up item
// then loads 28 words per round.)
__device__ __forceinline__ void wait_route_xd(const LayerArgs& a, int slot, bool routed,
                                              bool need_xd, LayerSmem& sm) {
  poll_all(a, [&] {
    if (threadIdx.x != 0) return true;
    bool ok = !need_xd || load_u32_agent(a.flags + kStride * kFlagXd) == a.epoch;
    if (routed) {
      const uint64_t v = get_tagged(a.prov + slot);
      ok = ok && tag_is(v, a.epoch);
      sm.eid = tagged_i(v);
    }
    return ok;
  });
}


// ---- the fused rms_norm --------------------------------------------------------------
// The first item of the list computes 1 / sqrt(sum h^2 / 7168 + 1e-6) of the
// hidden state, bit-exact with infer.m:369-374 (rms_sumsq_exact), and
// publishes it as one tagged word; the router rows and digit items wait for
// it (router rows after their weight loads are issued) and form
// h_post = (h * inv) * w element by element as infer.m:372.  Whole
// workgroup; h is 16-byte aligned.
__device__ __forceinline__ float layer_inv(const LayerArgs& a, LayerSmem& sm) {
  float xv[kRmsMaxPer];
  f32x4 c[kRmsMaxPer / 4];
  rms_stage_7168<false>(reinterpret_cast<const f32x4*>(a.h), 1.0f, xv, c, sm.rms);
  const float inv = rms_inv(rms_sumsq_exact(xv, kHidden, sm.rms), kHidden);
  __syncthreads();  // sm.rms is reused by the caller's next stage
  return inv;
}

// h_post_out is written before inv is published: every read of h happens
// before any item can depend on the publication (the output may alias h).
__device__ __forceinline__ void norm_item(const LayerArgs& a, LayerSmem& sm) {
#pragma clang fp contract(off)
  __builtin_amdgcn_s_setprio(3);  // first on the critical path: issue ahead of the CU's streaming waves
  const float inv = layer_inv(a, sm);
  if (a.h_post_out) {
    for (int i = threadIdx.x; i < kHidden; i += 256) a.h_post_out[i] = (a.h[i] * inv) * a.norm_w[i];
    __syncthreads();
  }
  if (threadIdx.x == 0) put_tagged(a.norm_inv, a.epoch, __float_as_uint(inv));
}

// The published 1 / rms, in every thread.
__device__ __forceinline__ float wait_inv(const LayerArgs& a, LayerSmem& sm) {
  poll_all(a, [&] {
    if (threadIdx.x != 0) return true;
    const uint64_t v = get_tagged(a.norm_inv);
    sm.inv = tagged_f(v);
    return tag_is(v, a.epoch);
  });
  return sm.inv;
}

// ---- digits of h_post: groups 4i .. 4i+3, one per wave ------------------------------
// Published untagged (16 KB read by every gate/up tile): agent-scope stores,
// then the last of the 28 items sets the digit flag.  With the fused norm,
// h_post = (h * inv) * w as infer.m:372 (and optionally written out).
__device__ __forceinline__ void xd_item(const LayerArgs& a, int i, LayerSmem& sm) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = 4 * i + wave;
  float v = a.h[64 * G + lane];
  if (a.norm_w) {
#pragma clang fp contract(off)
    const float w = a.norm_w[64 * G + lane];
    v = (v * wait_inv(a, sm)) * w;
  }
  publish_digit_group(v, a.xd + G);
  wait_stores_done();
  __syncthreads();
  if (threadIdx.x == 0) {
    int* c = a.counters + kStride * kCntXd;
    if (arrive_agent(c) == kXdItems - 1) {
      reset_agent(c);
      store_u32_agent(a.flags + kStride * kFlagXd, a.epoch);
    }
  }
}

// ---- router row e ---------------------------------------------------------------------
// Logit e in the canonical order (partial t of 256 accumulates float4 chunks
// t, t+256, ... by fma; xor butterfly per wave; (s0 + s1) + (s2 + s3)),
// published as its tagged sigmoid score.
__device__ __forceinline__ void router_row(const LayerArgs& a, int e, LayerSmem& sm) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = 64 * wave + lane;
  const float4* w4 = reinterpret_cast<const float4*>(a.Wg + (size_t)e * kHidden);
  const float4* x4 = reinterpret_cast<const float4*>(a.h);
  u32x4 wv[kHidden / 1024];
  float4 xv[kHidden / 1024];
#pragma unroll
  for (int i = 0; i < kHidden / 1024; ++i) {
    wv[i] = *reinterpret_cast<const u32x4*>(w4 + t + 256 * i);
    xv[i] = x4[t + 256 * i];
  }
  if (a.norm_w) {
    // h_post = (h * inv) * w, element by element as infer.m:372; the norm
    // weights are requested before the wait as well
    const float4* n4 = reinterpret_cast<const float4*>(a.norm_w);
    float4 nw[kHidden / 1024];
#pragma unroll
    for (int i = 0; i < kHidden / 1024; ++i) nw[i] = n4[t + 256 * i];
    const float inv = wait_inv(a, sm);
#pragma unroll
    for (int i = 0; i < kHidden / 1024; ++i) {
      xv[i].x = (xv[i].x * inv) * nw[i].x;
      xv[i].y = (xv[i].y * inv) * nw[i].y;
      xv[i].z = (xv[i].z * inv) * nw[i].z;
      xv[i].w = (xv[i].w * inv) * nw[i].w;
    }
  }
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < kHidden / 1024; ++i) {
    acc = fmaf(__uint_as_float(wv[i].x), xv[i].x, acc);
    acc = fmaf(__uint_as_float(wv[i].y), xv[i].y, acc);
    acc = fmaf(__uint_as_float(wv[i].z), xv[i].z, acc);
    acc = fmaf(__uint_as_float(wv[i].w), xv[i].w, acc);
  }
  acc = wave_sum_lane0(acc);  // the butterfly's lane-0 sum, VALU only
  if (lane == 0) sm.red[wave] = acc;
  __syncthreads();
  if (threadIdx.x == 0)
    put_tagged(a.scores + e, a.epoch,
               __float_as_uint(sigmoid_det((sm.red[0] + sm.red[1]) + (sm.red[2] + sm.red[3]))));
}

// The 256 tagged scores into wave 0's registers (lane l: expert 64 j + l in
// sc[j]); the other waves only take part in the wait.
__device__ __forceinline__ void wait_scores(const LayerArgs& a, float sc[4]) {
  const int lane = threadIdx.x & 63;
  poll_all(a, [&] {
    if (threadIdx.x >= 64) return true;
    bool ok = true;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint64_t v = get_tagged(a.scores + 64 * j + lane);
      ok = ok && tag_is(v, a.epoch);
      sc[j] = tagged_f(v);
    }
    return ok;
  });
}

// The 256 tagged scores into wave 0's registers (lane l: expert 64 j + l in
// sc[j]), polled by waves 1-3, staggered by ~0.5 us each: the first to see
// every tag of this call writes the scores to LDS and raises an LDS flag
// that wave 0 spins on.  A value is then seen within ~1/3 of a round trip
// plus one round trip of landing (one poller: 1/2 to 1), and no poll load is
// left outstanding in wave 0's registers when it starts the set.  Every
// thread calls it (one barrier).
__device__ __forceinline__ void wait_scores_staggered(const LayerArgs& a, float sc[4], LayerSmem& sm) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  volatile int* flag = &sm.sflag;
  if (threadIdx.x == 0) *flag = 0;
  __syncthreads();
  if (wave == 0) {
    while (*flag == 0) __builtin_amdgcn_s_sleep(1);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
#pragma unroll
    for (int j = 0; j < 4; ++j) sc[j] = sm.ssc[64 * j + lane];
    return;
  }
  if (wave == 2) __builtin_amdgcn_s_sleep(19);
  if (wave == 3) __builtin_amdgcn_s_sleep(38);
  unsigned* err = a.flags + kStride * kFlagErr;
  for (unsigned n = 0;; ++n) {
    float v[4];
    bool ok = true;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint64_t t = get_tagged(a.scores + 64 * j + lane);
      ok = ok && tag_is(t, a.epoch);
      v[j] = tagged_f(t);
    }
    const bool all = __ballot(!ok) == 0;
    if (*flag != 0) return;  // another poller was first
    if (all) {
#pragma unroll
      for (int j = 0; j < 4; ++j) sm.ssc[64 * j + lane] = v[j];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      if (lane == 0) *flag = 1;
      return;
    }
    if (n >= a.spin_limit || ((n & 63) == 63 && load_u32_agent(err) == a.epoch)) {
      if (lane == 0) {
        store_u32_agent(err, a.epoch);
        *flag = 2;
      }
      return;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

// ---- route: the expert set ------------------------------------------------------------
// On the critical path of every routed weight load: the bias is fetched
// before the wait, and the wave issues ahead of the SIMD's expert waves.
__device__ __forceinline__ void route_item(const LayerArgs& a, LayerSmem& sm) {
  const int lane = threadIdx.x & 63;
  __builtin_amdgcn_s_setprio(3);
  float bj[4], bj4[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) bj[j] = a.bias ? a.bias[64 * j + lane] : 0.0f;
#pragma unroll
  for (int m = 0; m < 4; ++m) bj4[m] = a.bias ? a.bias[4 * lane + m] : 0.0f;  // 4-byte aligned bias
  float sc[4], sc4[4];
  // Two passes over one copy of the set code.  Pass 0 runs it on made-up
  // scores and publishes nothing, while the router rows are still
  // streaming: every launch starts with an empty instruction cache, and the
  // set code would otherwise be fetched line by line on the critical path,
  // each fetch queued behind the weight stream (measured on MI355X: the
  // layer ~0.6 us faster).  Pass 1 waits for the scores and publishes: every
  // slot goes out as soon as it is certain (all at once for K <= 8).
#pragma nounroll
  for (int pass = 0; pass < 2; ++pass) {
    int p = pass;
    __asm__ volatile("" : "+s"(p));  // opaque: the loop keeps one copy of the code
    if (p == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sc[j] = (float)(64 * j + lane) * (1.0f / 256.0f);
        sc4[j] = (float)(4 * lane + j) * (1.0f / 256.0f);
      }
    } else {
      wait_scores_staggered(a, sc, sm);
      if (threadIdx.x < 64) {
        const f32x4 v = reinterpret_cast<const f32x4*>(sm.ssc)[lane];  // experts 4 lane .. 4 lane + 3
        sc4[0] = v.x;
        sc4[1] = v.y;
        sc4[2] = v.z;
        sc4[3] = v.w;
      }
    }
    if (threadIdx.x < 64)
      route_set_publish(sc, bj, sc4, bj4, a.K, [&](int slot, int id) {
        if (p == 1 && slot >= 0) put_tagged(a.prov + slot, a.epoch, (uint32_t)id);
      });
  }
}

// ---- the exact route() ----------------------------------------------------------------
// The reference's slot order and weights: idx and w (the caller's outputs)
// and, tagged for the combine, the weights and perm[k] = the slot of the
// expert set that runs expert idx[k].
__device__ __forceinline__ void exact_item(const LayerArgs& a) {
  const int lane = threadIdx.x & 63;
  float sc[4];
  wait_scores(a, sc);
  int pv = 0;
  poll_all(a, [&] {
    if (threadIdx.x >= a.K) return true;
    const uint64_t v = get_tagged(a.prov + threadIdx.x);
    pv = tagged_i(v);
    return tag_is(v, a.epoch);
  });
  if (threadIdx.x >= 64) return;
  float bj[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) bj[j] = a.bias ? a.bias[64 * j + lane] : 0.0f;
  int id;
  float wv;
  route_exact_lane(sc, bj, a.K, 2.5f, id, wv);
  int p = 0;
  for (int s = a.K - 1; s >= 0; --s) p = __builtin_amdgcn_readlane(pv, s) == id ? s : p;
  if (lane < a.K) {
    a.idx[lane] = id;
    a.w[lane] = wv;
    put_tagged(a.route_w + lane, a.epoch, __float_as_uint(wv));
    put_tagged(a.route_perm + lane, a.epoch, (uint32_t)p);
  }
}

// ---- gate/up run: kGuPer consecutive 8-row tiles of gate and up of one slot --------
// Wave w owns rows 2w, 2w+1 of each tile in both matrices (lanes 0-31 gate,
// 32-63 up, 16 lanes per row); SwiGLU in registers; the activations go out
// tagged.  The route and the digits of h_post are waited for and staged
// once per run, so their round trips are paid once for kGuPer tiles.
template <bool ROUTED>
__device__ __forceinline__ void gateup_run(const LayerArgs& a, int slot, int tile0, LayerSmem& sm) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane >> 4, l16 = lane & 15, g = l16 & 3;
  // The digit record (23 KB, every gate/up item reads all of it): all of a
  // thread's 16-byte loads are issued before any is written to LDS (loads
  // past the record return 0 through the buffer's range check), with the
  // coherent (sc1) cache policy.
  constexpr int kXsVec = (int)sizeof(sm.xs) / 16;
  constexpr int kXsPer = (kXsVec + 255) / 256;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.xd, 0, (int)sizeof(XGroup) * (kHidden / 64), 0x00020000);
  u32x4 xv[kXsPer];
  auto load_xd = [&] {
#pragma unroll
    for (int k = 0; k < kXsPer; ++k)
      xv[k] = __builtin_amdgcn_raw_buffer_load_b128(xr, (threadIdx.x + 256 * k) * 16, 0, 16);
  };
  auto store_xd = [&] {
#pragma unroll
    for (int k = 0; k < kXsPer; ++k)
      if (threadIdx.x + 256 * k < kXsVec) reinterpret_cast<u32x4*>(sm.xs)[threadIdx.x + 256 * k] = xv[k];
    __syncthreads();
  };
  // A routed slot waits for its expert (and the digits), requests the digit
  // record and then the weights, so the record lands first and each weight
  // group is used as soon as it arrives.  The shared expert's weights are
  // requested before the digits are waited for.  The loads are issued on
  // every path (an invalid expert id reads the layer's first expert and
  // contributes 0), so the code is straight-line and the LDS stores of the
  // record wait for the record's loads only, not for the weights behind it.
  if (ROUTED) {
    wait_route_xd(a, slot, true, true, sm);
    load_xd();
  }
  // The shared expert's items of the layer hold their weight loads back
  // ~0.85 us (2048 cycles): the router rows' 7 MB and the digits of h_post
  // then lead the memory queues and the route goes out sooner, while these
  // 16.5 MB still fill the time the route takes (measured on MI355X: 0.5,
  // 0.85 and 1.3 us all ~0.8 us faster than no hold).
  if (!ROUTED) __builtin_amdgcn_s_sleep(32);
  const uint8_t* blob = ROUTED ? expert_blob(a, sm.eid) : a.shared;
  const uint8_t* src = blob ? blob : a.experts;
  const Q4KScaleSel sel = q4k_scale_sel(g);
  for (int t = 0; t < kGuPer; ++t) {
    const int row = (tile0 + t) * kGuTileRows + 2 * wave + (q & 1);
    Q4KGroupLoad ld[7];
    // resident expert layout: each half-wave load reads one 512-byte run
    const uint8_t* mat = src + (q >= 2 ? kGateBytes : 0);
#pragma unroll
    for (int i = 0; i < 7; ++i) ld[i] = rel_load_group<false>(mat, row, 4 * i + (l16 >> 2), g);
    if (t == 0) {
      if (!ROUTED) {
        wait_route_xd(a, slot, false, true, sm);
        load_xd();
      }
      store_xd();
    }
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 7; ++i) {
      acc += q4k_group_dot_ld(ld[i], sel, &sm.xs[16 * i + l16]);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (!blob) acc = 0.0f;
    acc = sum16(acc);
    const float up = __shfl(acc, (lane + 32) & 63);
    if (lane == 0 || lane == 16) {
      const float av = silu_mul(acc, up);
      put_tagged(a.act + (size_t)slot * kFfn + row, a.epoch, __float_as_uint(av));
    }
  }
}

// ---- activation digits of one (slot, part) --------------------------------------------
// Every down item of a slot's part contracts against the digit records of the
// same 1024 activations, so they are made once, here, instead of once per
// down item: the item waits for the part's tagged activations, turns them
// into kPartGroups records in LDS and publishes the records' 32-bit words as
// tagged words (act_xd[slot][group][word]); the down items stage them with
// their own loads, whose tags are their readiness check.
constexpr int kXgWords = (int)sizeof(XGroup) / 4;            // 52 words per record
constexpr int kPartXdWords = kPartGroups * kXgWords;         // words of a part's records
__device__ __forceinline__ uint64_t* act_xd_words(const LayerArgs& a, int slot, int group) {
  return a.act_xd + ((size_t)slot * (kFfn / 64) + group) * kXgWords;
}

// A poll of a whole digit record (hundreds of tagged words per round):
// full() loads and checks every word.  When the first round finds the
// record incomplete, thread 0 polls only one or two sentinel words of it
// until they carry the epoch, then full() runs again (words land in any
// order, so it still checks every tag): an item that waits long -- down and
// final items are resident from the start of short lists -- would otherwise
// reload every word each round, kilobytes of coherent loads per item
// competing with the weight stream.  A record already complete costs one
// round, as a plain poll.
template <typename F>
__device__ __forceinline__ void poll_record(const LayerArgs& a, const uint64_t* s0, const uint64_t* s1, F&& full) {
  for (;;) {
    if (__syncthreads_and(full())) return;
    const bool ok = poll_all(a, [&] {
      if (threadIdx.x != 0) return true;
      bool got = tag_is(get_tagged(s0), a.epoch);
      if (s1) got = got && tag_is(get_tagged(s1), a.epoch);
      return got;
    });
    if (!ok) return;  // gave up: the error flag is set
  }
}

__device__ __forceinline__ void adg_item(const LayerArgs& a, int slot, int part, LayerSmem& sm) {
  const int wave = threadIdx.x >> 6;
  const uint64_t* act = a.act + (size_t)slot * kFfn + part * kPartCols;
  constexpr int kPer = kPartCols / 256;
  float v[kPer];
  poll_all(a, [&] {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const uint64_t t = get_tagged(act + threadIdx.x + 256 * i);
      ok = ok && tag_is(t, a.epoch);
      v[i] = tagged_f(t);
    }
    return ok;
  });
  // element 256 i + 64 w + lane lives in wave w's lanes: record 4 i + w
#pragma unroll
  for (int i = 0; i < kPer; ++i) digits_to_lds(v[i], sm.xs[4 * i + wave]);
  __syncthreads();
  const uint32_t* src = reinterpret_cast<const uint32_t*>(sm.xs);
  uint64_t* dst = act_xd_words(a, slot, part * kPartGroups);
  for (int i = threadIdx.x; i < kPartXdWords; i += 256) put_tagged(dst + i, a.epoch, src[i]);
}

// The records of `n_groups` consecutive groups of a slot's activations into
// sm.xs[0 ..): every thread loads its words (after the caller's weight loads,
// so the first poll returns with them) until all carry this call's tag.
template <int NG>
__device__ __forceinline__ void stage_act_digits(const LayerArgs& a, int slot, int group0, LayerSmem& sm) {
  constexpr int kW = NG * kXgWords, kPer = (kW + 255) / 256;
  const uint64_t* src = act_xd_words(a, slot, group0);
  uint32_t w[kPer];
  poll_record(a, src + kW - 1, nullptr, [&] {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int k = threadIdx.x + 256 * i;
      if (k < kW) {
        const uint64_t t = get_tagged(src + k);
        ok = ok && tag_is(t, a.epoch);
        w[i] = (uint32_t)t;
      }
    }
    return ok;
  });
  uint32_t* dst = reinterpret_cast<uint32_t*>(sm.xs);
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int k = threadIdx.x + 256 * i;
    if (k < kW) dst[k] = w[i];
  }
  __syncthreads();
}

// The records of part `part` of a slot's activations made here, from the
// part's 1024 tagged activations (four per thread), into sm.xs[0 .. 16):
// no hand-off through a digit item (a coherent round trip each way).
__device__ __forceinline__ void stage_act_direct(const LayerArgs& a, int slot, int part, LayerSmem& sm) {
  const int wave = threadIdx.x >> 6;
  const uint64_t* act = a.act + (size_t)slot * kFfn + part * kPartCols;
  constexpr int kPer = kPartCols / 256;
  float v[kPer];
  poll_record(a, act + kPartCols - 1, nullptr, [&] {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const uint64_t t = get_tagged(act + threadIdx.x + 256 * i);
      ok = ok && tag_is(t, a.epoch);
      v[i] = tagged_f(t);
    }
    return ok;
  });
  // element 256 i + 64 w + lane lives in wave w's lanes: record 4 i + w
#pragma unroll
  for (int i = 0; i < kPer; ++i) digits_to_lds(v[i], sm.xs[4 * i + wave]);
  __syncthreads();
}

// ---- down item: rows of one column part of one routed slot's down matrix --------------
// Part p covers columns kPartCols p .. kPartCols (p+1) - 1.  The weights are
// loaded before the part's digit records are waited for and staged; each
// row's partial sum goes out tagged into eo[slot][p][row] for the final items.
//  Q4_K: kDnLanesQ4 lanes per row (one 64-element group each), lane row
//        group rr = lane / kDnLanesQ4, rows rr + 4 j (j < kDnRowsQ4L).
//  Q6_K: kDnLanesQ6 lanes per row (one 128-element half block each).
template <bool Q6>
__device__ __forceinline__ void down_part(const LayerArgs& a, int slot, int part, int item, LayerSmem& sm) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  wait_route_xd(a, slot, true, false, sm);
  const uint8_t* blob = expert_blob(a, sm.eid);
  const uint8_t* dbase = blob ? blob + 2 * (size_t)kGateBytes : nullptr;
  uint64_t* eo = a.eo + ((size_t)slot * kLayerMaxParts + part) * kHidden;
  if (!Q6) {
    constexpr int LR = kDnLanesQ4, RPW = 64 / LR;
    const int gl = lane % LR;  // group of the row's part
    const int row0 = item * kDnRowsQ4 + wave * (kDnRowsQ4L * RPW) + lane / LR;  // + RPW j
    const int blk = (part * kPartGroups + gl) / 4;
    Q4KGroupLoad ld[kDnRowsQ4L];
    if (blob) {
      // resident expert layout: a wave's load (4 rows x one block quad) reads one 1 KB run
#pragma unroll
      for (int j = 0; j < kDnRowsQ4L; ++j) ld[j] = rel_load_group<true>(dbase, row0 + RPW * j, blk, gl & 3);
    }
    if (FDM_ACT_DIRECT)
      stage_act_direct(a, slot, part, sm);
    else
      stage_act_digits<kPartGroups>(a, slot, part * kPartGroups, sm);
    float acc[kDnRowsQ4L] = {};
    // the lane's rows share one digit record: each quarter of it is read
    // from LDS once for all of them
    if (blob) q4k_group_dot_rows<kDnRowsQ4L>(ld, q4k_scale_sel(gl & 3), &sm.xs[gl], acc);
#pragma unroll
    for (int j = 0; j < kDnRowsQ4L; ++j) {
      float v = acc[j];
#pragma unroll
      for (int m = LR / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m);
      if (gl == 0) put_tagged(eo + row0 + RPW * j, a.epoch, __float_as_uint(v));
    }
  } else {
    // Q6_K resident layout: lane (half h = bit 0, row r of a 4-row group =
    // bits 1-2, block b of the part = bits 3-4, 4-row group g4 = bit 5); the
    // wave's rows are one 16-row step, so its load j of a half block per lane
    // reads 64 consecutive pieces (rows 8 j .. 8 j + 7 of the step)
    static_assert(kDnLanesQ6 == 8 && kDnRowsQ6L == 2 && kDnRowsQ6 == 64, "Q6_K down item: 16 rows per wave");
    const int h = lane & 1, r = (lane >> 1) & 3, b = (lane >> 3) & 3, g4 = lane >> 5;
    const int gl = 2 * b + h;  // half block of the row's part
    const int row0 = item * kDnRowsQ6 + wave * 16 + 4 * g4 + r;  // + 8 j
    Q6KHalfW l6[kDnRowsQ6L];
    if (blob) {
#pragma unroll
      for (int j = 0; j < kDnRowsQ6L; ++j) l6[j] = q6k_rel_load_half(dbase, row0 + 8 * j, part * 4 + b, h);
    }
    if (FDM_ACT_DIRECT)
      stage_act_direct(a, slot, part, sm);
    else
      stage_act_digits<kPartGroups>(a, slot, part * kPartGroups, sm);
    float acc[kDnRowsQ6L] = {};
    if (blob) {
#pragma unroll
      for (int j = 0; j < kDnRowsQ6L; ++j) {
        int gi = 2 * gl;
        __asm__ volatile("" : "+v"(gi));
        acc[j] = q6k_half_dot_w(l6[j], &sm.xs[gi]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int j = 0; j < kDnRowsQ6L; ++j) {
      // the half blocks of a row's part, gl bits 2, 1, 0 = lane bits 4, 3, 0,
      // summed in the order of the xor butterfly over 4, 2, 1
      float v = acc[j];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 8);
      v += __shfl_xor(v, 1);
      if ((lane & 0x19) == 0) put_tagged(eo + row0 + 8 * j, a.epoch, __float_as_uint(v));
    }
  }
}

// ---- final item: the shared expert's down rows and the combine of the same rows ----------
// The last items of the list.  Each takes kFinRows rows of the output: it
// loads the shared expert's down rows (both column parts) first, stages the
// shared activations' digit records and, with the same loads, the routed
// slots' tagged part outputs of its rows and the exact route, contracts the
// shared rows (part sums by the butterflies the down items use, so the same
// bits), and writes
//   hidden[r] = (h_in[r] + sum_k w[k] (E_perm[k][r] part 0 + part 1)) + S[r]
// in the reference's slot order (infer.m:1689-1695, 1922).  Its weights are
// the last bytes of the list, and the combine needs no further hand-off: the
// routed outputs it polls were published while these weights streamed.
//  Q4_K: 32 rows; lane (bq = lane / 16, rs = lane / 4 % 4, g = lane % 4) of
//        wave w holds rows 8 w + 4 m + rs (m < 2), block quad bq of both
//        parts (blocks bq and 4 + bq), group g: a wave's load is one resident
//        layout step (4 rows x 4 blocks).
//  Q6_K: 16 rows; lane (half h = bit 0, row r = bits 1-2, block b = bits
//        3-4, part = bit 5) of wave w holds row 4 w + r, half
//        h of block 4 part + b: in the Q6_K resident layout a wave's load
//        reads 32 consecutive pieces of each part.
static_assert(kParts == 2, "final items: two column parts");
#ifndef FDM_FIN_ROWS_Q6
#define FDM_FIN_ROWS_Q6 16  // two Q6_K half-block loads per lane would not fit 128 VGPRs
#endif
#ifndef FDM_FIN_ROWS_Q4
#define FDM_FIN_ROWS_Q4 32
#endif
constexpr int kFinRowsQ4 = FDM_FIN_ROWS_Q4, kFinRowsQ6 = FDM_FIN_ROWS_Q6;
__host__ __device__ constexpr int fin_rows(bool q6) { return q6 ? kFinRowsQ6 : kFinRowsQ4; }
__host__ __device__ constexpr int fin_items(bool q6) { return kHidden / fin_rows(q6); }
constexpr int kFinMaxRouted = kLayerMaxSlots - 1;             // routed slots (FDM_MAX_K)
constexpr int kFinWordsMax = 2 * kFinMaxRouted * kFinRowsQ4;  // routed part outputs of one item
static_assert(kFinRowsQ4 >= kFinRowsQ6, "LDS of the final items sized for the Q4_K rows");

template <bool Q6>
__device__ __forceinline__ void final_item(const LayerArgs& a, int item, LayerSmem& sm) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int R = fin_rows(Q6);
  const int r0 = item * R;
  const bool has_shared = a.n_slots > a.K;
  const uint8_t* dbase = (has_shared && a.shared) ? a.shared + 2 * (size_t)kGateBytes : nullptr;
  // the residual first, so its load is not queued behind the waits
  const float hin = (threadIdx.x < R && a.h_in) ? a.h_in[r0 + threadIdx.x] : 0.0f;
  // weights of the shared rows
  constexpr int kQ4M = kFinRowsQ4 / 16;  // Q4_K rows per lane
  const int g = lane & 3, rs = (lane >> 2) & 3, bq = lane >> 4;
  const int h6 = lane & 1, r6 = (lane >> 1) & 3, b6 = (lane >> 3) & 3, p6 = lane >> 5;
  const int H = 8 * p6 + 2 * b6 + h6;  // half block of the row
  Q4KGroupLoad ld0[kQ4M], ld1[kQ4M];
  constexpr int kQ6M = kFinRowsQ6 / 16;  // Q6_K rows per lane
  Q6KHalfW l6[kQ6M];
  if (dbase) {
    if (!Q6) {
#pragma unroll
      for (int m = 0; m < kQ4M; ++m) {
        const int row = r0 + 4 * kQ4M * wave + 4 * m + rs;
        ld0[m] = rel_load_group<true>(dbase, row, bq, g);
        ld1[m] = rel_load_group<true>(dbase, row, 4 + bq, g);
      }
    } else {
#pragma unroll
      for (int j = 0; j < kQ6M; ++j) {
        const int row = r0 + 4 * kQ6M * wave + 4 * j + r6;
        l6[j] = q6k_rel_load_half(dbase, row, 4 * p6 + b6, h6);
      }
    }
  }
  // the shared activations' records (both parts) are waited for; the routed
  // part outputs of the item's rows and the exact route are loaded by the
  // same polls (the first returns with the weights) and waited for only
  // after the shared rows are contracted
  constexpr int kXW = (kFfn / 64) * kXgWords, kXPer = (kXW + 255) / 256;
  constexpr int kEPer = (kFinWordsMax + 255) / 256;
  const int nE = 2 * a.K * R;  // word e: slot e / (2 R), part e / R % 2, row e % R
  const uint64_t* xsrc = act_xd_words(a, a.K, 0);
  uint32_t xw[kXPer];
  float ev[kEPer];
  uint64_t tw = 0, tp = 0;
  bool e_ok = true;
  auto load_routed = [&] {
    e_ok = true;
#pragma unroll
    for (int i = 0; i < kEPer; ++i) {
      const int e = threadIdx.x + 256 * i;
      if (e < nE) {
        const int s = e / (2 * R), p = (e / R) & 1, r = e % R;
        const uint64_t t = get_tagged(a.eo + ((size_t)s * kLayerMaxParts + p) * kHidden + r0 + r);
        e_ok = e_ok && tag_is(t, a.epoch);
        ev[i] = tagged_f(t);
      }
    }
    if (threadIdx.x < a.K) {
      tw = get_tagged(a.route_w + threadIdx.x);
      tp = get_tagged(a.route_perm + threadIdx.x);
      e_ok = e_ok && tag_is(tw, a.epoch) && tag_is(tp, a.epoch);
    }
    return e_ok;
  };
  auto store_routed = [&] {
#pragma unroll
    for (int i = 0; i < kEPer; ++i) {
      const int e = threadIdx.x + 256 * i;
      if (e < nE) sm.fin.v[e] = ev[i];
    }
    if (threadIdx.x < a.K) {
      sm.cw[threadIdx.x] = tagged_f(tw);
      sm.cperm[threadIdx.x] = tagged_i(tp);
    }
  };
  // the last word of each part's records (activations) as sentinels
  // (without a shared expert the first round always succeeds)
  poll_record(a, xsrc + kXW / 2 - 1, xsrc + kXW - 1, [&] {
    bool ok = true;
    if (dbase) {
#pragma unroll
      for (int i = 0; i < kXPer; ++i) {
        const int k = threadIdx.x + 256 * i;
        if (k < kXW) {
          const uint64_t t = get_tagged(xsrc + k);
          ok = ok && tag_is(t, a.epoch);
          xw[i] = (uint32_t)t;
        }
      }
    }
    load_routed();
    return ok;
  });
  uint32_t* xdst = reinterpret_cast<uint32_t*>(sm.fin.xs);
#pragma unroll
  for (int i = 0; i < kXPer; ++i) {
    const int k = threadIdx.x + 256 * i;
    if (dbase && k < kXW) xdst[k] = xw[i];
  }
  store_routed();
  const bool routed_ready = __syncthreads_and(e_ok);
  // the shared rows: part sums p0, p1 by the butterflies of the down items
  if (!Q6) {
    float acc0[kQ4M] = {}, acc1[kQ4M] = {};
    if (dbase) {
      const Q4KScaleSel sel = q4k_scale_sel(g);
      q4k_group_dot_rows<kQ4M>(ld0, sel, &sm.fin.xs[4 * bq + g], acc0);
      q4k_group_dot_rows<kQ4M>(ld1, sel, &sm.fin.xs[16 + 4 * bq + g], acc1);
    }
#pragma unroll
    for (int m = 0; m < kQ4M; ++m) {
      // group index within the part = 4 bq + g: its bits 3, 2, 1, 0 are lane
      // bits 5, 4, 1, 0 (the down items' xor 8, 4, 2, 1)
      float p0 = acc0[m], p1 = acc1[m];
      p0 += __shfl_xor(p0, 32);
      p1 += __shfl_xor(p1, 32);
      p0 += __shfl_xor(p0, 16);
      p1 += __shfl_xor(p1, 16);
      p0 += __shfl_xor(p0, 2);
      p1 += __shfl_xor(p1, 2);
      p0 += __shfl_xor(p0, 1);
      p1 += __shfl_xor(p1, 1);
      if ((lane & 0x33) == 0) sm.fin.esh[4 * kQ4M * wave + 4 * m + rs] = p0 + p1;
    }
  } else {
    float acc[kQ6M] = {};
    if (dbase) {
#pragma unroll
      for (int j = 0; j < kQ6M; ++j) {
        int gi = 2 * H;
        __asm__ volatile("" : "+v"(gi));
        acc[j] = q6k_half_dot_w(l6[j], &sm.fin.xs[gi]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int j = 0; j < kQ6M; ++j) {
      // half block within the part = 2 b + h: bits 2, 1, 0 are lane bits 4,
      // 3, 0 (the down items' xor 4, 2, 1)
      float v = acc[j];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 8);
      v += __shfl_xor(v, 1);
      const float p1 = __shfl_xor(v, 32);  // lanes of part 0 receive part 1's sum
      if ((lane & 0x39) == 0) sm.fin.esh[4 * kQ6M * wave + 4 * j + r6] = v + p1;
    }
  }
  if (!routed_ready) {
    poll_all(a, load_routed);
    store_routed();
  }
  __syncthreads();
  if (threadIdx.x >= R) return;
  const int r = threadIdx.x;
  float moe = 0.0f;
  for (int k = 0; k < a.K; ++k) {
    const int s = sm.cperm[k];
    const float e = sm.fin.v[(2 * s) * R + r] + sm.fin.v[(2 * s + 1) * R + r];
    moe = fmaf(sm.cw[k], e, moe);
  }
  const float sd = has_shared ? sm.fin.esh[r] : 0.0f;
  a.out[r0 + r] = (hin + moe) + sd;
  if (a.moe_out) a.moe_out[r0 + r] = moe;
}

// First workgroup of each section of the work list:
//   (with a norm weight: the fused rms_norm) | digits | router rows
//   | route set | exact route
//   | shared expert: gate/up of parts 0..P-1, then its activation digits (P)
//   | routed experts, part-major: step q holds gate/up of part q of every
//     slot and then the activation digits of part q of every slot (q < P),
//     then down of part q - lag of every slot (q >= lag)
//   | final items (shared down + combine)
constexpr int kAdgRouted = FDM_ACT_DIRECT ? 0 : 1;  // activation digit items per routed (slot, part)
struct LayerList {
  int route, exact, router, xd, shared, shadg, routed, fin, total;
  int gup, dnp;  // gate/up and down items per (slot, part)
};

__host__ __device__ __forceinline__ LayerList layer_list(int K, int n_slots, bool q6, bool norm) {
  const int hs = n_slots - K;  // 1 with a shared expert
  LayerList l;
  l.gup = kGuPerPart;
  l.dnp = dn_per_part(q6);
  l.xd = norm ? 1 : 0;  // item 0: the fused rms_norm
  l.router = l.xd + kXdItems;
  l.route = l.router + kRows;
  l.exact = l.route + 1;
  l.shared = l.exact + 1;
  l.shadg = l.shared + hs * kParts * l.gup;
  // activation digit items: the shared expert's (at the head, off the
  // critical path); routed slots' down items make their records themselves
  l.routed = l.shadg + hs * kParts;
  l.fin = l.routed + K * kParts * (l.gup + kAdgRouted + l.dnp);
  l.total = l.fin + fin_items(q6);
  return l;
}

// Routed item `off` (0-based within the routed section): kind 0 gate/up
// (idx = gate/up item), 1 activation digits, 2 down (idx = down item) of
// (slot, part).
__device__ __forceinline__ void routed_item(const LayerList& l, int K, int off, int& kind, int& slot,
                                            int& part, int& idx) {
  const int GU = K * l.gup, G = GU + K * kAdgRouted, D = K * l.dnp;
  int q, r;
  if (off < kLag * G) {
    q = off / G;
    r = off % G;
  } else if (off < kLag * G + (kParts - kLag) * (G + D)) {
    const int o = off - kLag * G;
    q = kLag + o / (G + D);
    r = o % (G + D);
  } else {
    const int o = off - kLag * G - (kParts - kLag) * (G + D);
    q = kParts + o / D;
    r = G + o % D;  // a step past the last gate/up part holds down items only
  }
  if (r < GU) {
    kind = 0;
    part = q;
    slot = r / l.gup;
    idx = r % l.gup;
  } else if (r < G) {
    kind = 1;
    part = q;
    slot = r - GU;
    idx = 0;
  } else {
    kind = 2;
    part = q - kLag;
    slot = (r - G) / l.dnp;
    idx = (r - G) % l.dnp;
  }
}

}  // namespace

template <bool Q6>
__device__ __forceinline__ void layer_item(const LayerArgs& a, LayerSmem& sm) {
  const LayerList l = layer_list(a.K, a.n_slots, Q6, a.norm_w != nullptr);
  const int it = blockIdx.x;
  if (it < l.xd) {
    norm_item(a, sm);
  } else if (it < l.router) {
    xd_item(a, it - l.xd, sm);
  } else if (it < l.route) {
    router_row(a, it - l.router, sm);
  } else if (it == l.route) {
    route_item(a, sm);
  } else if (it == l.exact) {
    exact_item(a);
  } else if (it < l.shadg) {
    const int off = it - l.shared;
    gateup_run<false>(a, a.K, (off / l.gup) * (kPartCols / kGuTileRows) + (off % l.gup) * kGuPer, sm);
  } else if (it < l.routed) {
    adg_item(a, a.K, it - l.shadg, sm);
  } else if (it < l.fin) {
    int kind, slot, part, idx;
    routed_item(l, a.K, it - l.routed, kind, slot, part, idx);
    if (kind == 0)
      gateup_run<true>(a, slot, part * (kPartCols / kGuTileRows) + idx * kGuPer, sm);
    else if (kind == 1)
      adg_item(a, slot, part, sm);
    else
      down_part<Q6>(a, slot, part, idx, sm);
  } else {
    final_item<Q6>(a, it - l.fin, sm);
  }
}

// Every item fits 128 VGPRs, so four workgroups per CU.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void k_layer_q4k(
    LayerArgs a) {
  __shared__ LayerSmem sm;
  layer_item<false>(a, sm);
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void k_layer_q6k(LayerArgs a) {
  __shared__ LayerSmem sm;
  layer_item<true>(a, sm);
}

hipError_t launch_layer(const LayerArgs& a, hipStream_t s) {
  const LayerList l = layer_list(a.K, a.n_slots, a.down_q6 != 0, a.norm_w != nullptr);
  if (a.down_q6)
    hipLaunchKernelGGL(k_layer_q6k, dim3(l.total), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(k_layer_q4k, dim3(l.total), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace fdm
