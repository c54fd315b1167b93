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
//   digits of h_post (28: four 64-element groups each)
//   router row e (256)
//   route: the expert set (1);  the exact route() (1)
//   shared expert gate/up runs, shared expert down runs
//   routed gate/up runs, slot-major
//   routed down runs, slot-major
// (a run is kGuPer / kDnPer consecutive row tiles of one slot)
//   combine tiles (224)
//
// (Interleaving each slot's down tiles right behind its gate/up tiles was
// measured slower: down tiles dispatched early hold workgroup slots while
// they wait for activations, starving the remaining gate/up tiles.  The
// shared expert's gate/up tiles likewise wait for the digits before they
// load, so their weights do not compete with the router rows, which are on
// the route's critical path.)
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
// waits, and nothing is ever cleared.  Only the 16 KB digit record of
// h_post is published untagged, behind a flag set by the last of its 28
// producers, and staged with 16-byte coherent loads.
#include "fdm_internal.h"
#include "route_device.h"

namespace fdm {

namespace {

constexpr int kStride = kLayerStride;        // ints between counters / flags (256 B)
constexpr int kRows = 256;                   // router rows (R1 experts)
constexpr int kXdItems = kHidden / 64 / 4;   // 28 digit items of 4 groups
constexpr int kGuTileRows = 8;               // gate (and up) rows per gate/up tile
constexpr int kGuTileCount = kFfn / kGuTileRows;      // 256
// down tile: 16 rows per pass of the four waves; two passes for Q4_K rows
// (1152 B), one for the larger Q6_K rows (1680 B, more registers per row)
__host__ __device__ constexpr int dn_passes(bool q6) { return q6 ? 1 : 2; }
__host__ __device__ constexpr int dn_tiles(bool q6) { return kHidden / (16 * dn_passes(q6)); }
constexpr int kGuPer = 2;                    // gate/up tiles per work item
constexpr int kDnPer = 2;                    // down tiles per work item
constexpr int kCombRows = 32;                // rows per combine tile
constexpr int kCombTiles = kHidden / kCombRows;       // 224
constexpr unsigned kSpinLimit = 1u << 17;    // polls of one wait (each >= ~1 us)

// flag and counter slots (units of kStride)
constexpr int kFlagXd = 0;
constexpr int kFlagErr = kLayerFlagErr;
constexpr int kCntXd = 0;

__device__ __forceinline__ unsigned load_u32_agent(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_u32_agent(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- tagged words ------------------------------------------------------------------
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

struct LayerSmem {
  XGroup xs[kHidden / 64];  // digits of h_post (gate/up) or of one slot's activations (down)
  float red[4];
  int eid;                  // expert of the item's slot
};

// Whole-workgroup wait: every thread runs try_once() (its share of the
// loads and checks) until all of them succeed.  Gives up after kSpinLimit
// rounds, or when another workgroup already gave up (looked at every 64th
// round: each look is one more round trip), recording the epoch in the
// error flag.  Returns false on giving up.
template <typename F>
__device__ __forceinline__ bool poll_all(const LayerArgs& a, F&& try_once) {
  unsigned* err = a.flags + kStride * kFlagErr;
  for (unsigned n = 0;; ++n) {
    if (__syncthreads_and(try_once())) return true;
    int give_up = 0;
    if (threadIdx.x == 0 && (n & 63) == 63)
      give_up = n >= kSpinLimit || load_u32_agent(err) == a.epoch;
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
// slot's expert; the expert id lands in sm.eid.
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

// Digits of the 64 elements held by one wave (lane l: element l) into LDS
// record g (two sub-blocks of 32, one per half-wave).
__device__ __forceinline__ void digits_to_lds(float v, XGroup& g) {
  const int lane = threadIdx.x & 63;
  int8_t da, db;
  float ds, dsum;
  make_digits32(v, da, db, ds, dsum);
  g.a[lane] = da;
  g.b[lane] = db;
  if ((lane & 31) == 0) {
    g.s[lane >> 5] = ds;
    g.xsum[lane >> 5] = dsum;
  }
}

// ---- digits of h_post: groups 4i .. 4i+3, one per wave ------------------------------
// Published untagged (16 KB read by every gate/up tile): agent-scope stores,
// then the last of the 28 items sets the digit flag.
__device__ __forceinline__ void xd_item(const LayerArgs& a, int i) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = 4 * i + wave;
  int8_t da, db;
  float ds, dsum;
  make_digits32(a.h[64 * G + lane], da, db, ds, dsum);
  const unsigned ua = (uint8_t)da, ub = (uint8_t)db;
  const int l = lane & 31, sub = lane >> 5;
  const unsigned wa = ua | (__shfl_down(ua, 1, 32) << 8) | (__shfl_down(ua, 2, 32) << 16) |
                      (__shfl_down(ua, 3, 32) << 24);
  const unsigned wb = ub | (__shfl_down(ub, 1, 32) << 8) | (__shfl_down(ub, 2, 32) << 16) |
                      (__shfl_down(ub, 3, 32) << 24);
  XGroup* xg = a.xd + G;
  if ((l & 3) == 0) {
    store_u32_agent(reinterpret_cast<unsigned*>(xg->a) + 8 * sub + l / 4, wa);
    store_u32_agent(reinterpret_cast<unsigned*>(xg->b) + 8 * sub + l / 4, wb);
  }
  if (l == 0) {
    store_agent(&xg->s[sub], ds);
    store_agent(&xg->xsum[sub], dsum);
  }
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
  float4 wv[kHidden / 1024], xv[kHidden / 1024];
#pragma unroll
  for (int i = 0; i < kHidden / 1024; ++i) {
    wv[i] = w4[t + 256 * i];
    xv[i] = x4[t + 256 * i];
  }
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < kHidden / 1024; ++i) {
    acc = fmaf(wv[i].x, xv[i].x, acc);
    acc = fmaf(wv[i].y, xv[i].y, acc);
    acc = fmaf(wv[i].z, xv[i].z, acc);
    acc = fmaf(wv[i].w, xv[i].w, acc);
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) acc = acc + __shfl_xor(acc, m);
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

// ---- route: the expert set ------------------------------------------------------------
// On the critical path of every routed weight load: the bias is fetched
// before the wait, and the wave issues ahead of the SIMD's expert waves.
__device__ __forceinline__ void route_item(const LayerArgs& a) {
  const int lane = threadIdx.x & 63;
  __builtin_amdgcn_s_setprio(3);
  float bj[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) bj[j] = a.bias ? a.bias[64 * j + lane] : 0.0f;
  float sc[4];
  wait_scores(a, sc);
  if (threadIdx.x >= 64) return;
  const int id = route_set_lane(sc, bj, a.K);
  if (lane < a.K) put_tagged(a.prov + lane, a.epoch, (uint32_t)id);
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
__device__ __forceinline__ void gateup_run(const LayerArgs& a, int slot, int tile0, bool routed,
                                           LayerSmem& sm) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane >> 4, l16 = lane & 15, g = l16 & 3;
  wait_route_xd(a, slot, routed, true, sm);
  const uint8_t* blob = routed ? expert_blob(a, sm.eid) : a.shared;
  const Q4KScaleSel sel = q4k_scale_sel(g);
  for (int t = 0; t < kGuPer; ++t) {
    const int row = (tile0 + t) * kGuTileRows + 2 * wave + (q & 1);
    Q4KGroupLoad ld[7];
    if (blob) {
      const uint8_t* rowp = blob + (q >= 2 ? kGateBytes : 0) + (size_t)row * kQ4KRowHidden;
#pragma unroll
      for (int i = 0; i < 7; ++i) ld[i] = q4k_load_group(rowp + (4 * i + (l16 >> 2)) * kQ4KBlock, g);
    }
    if (t == 0) {
      // the digit record: 16-byte loads with the coherent (sc1) cache policy
      const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
          (void*)a.xd, 0, (int)sizeof(XGroup) * (kHidden / 64), 0x00020000);
      for (int i = threadIdx.x; i < (int)sizeof(sm.xs) / 16; i += 256)
        reinterpret_cast<u32x4*>(sm.xs)[i] = __builtin_amdgcn_raw_buffer_load_b128(r, i * 16, 0, 16);
      __syncthreads();
    }
    float acc = 0.0f;
    if (blob) {
#pragma unroll
      for (int i = 0; i < 7; ++i) {
        acc += q4k_group_dot_ld(ld[i], sel, &sm.xs[16 * i + l16]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    acc = sum16(acc);
    const float up = __shfl(acc, (lane + 32) & 63);
    if (lane == 0 || lane == 16)
      put_tagged(a.act + (size_t)slot * kFfn + row, a.epoch, __float_as_uint(silu_mul(acc, up)));
  }
}

// ---- down run: kDnPer consecutive tiles of 16 * P rows of one slot's down matrix ----
// Wave w owns rows 4P w .. 4P w + 4P-1 of each tile as row groups of 16
// lanes (row 4P w + 4j + lane/16 in pass j).  The first tile's weights are
// loaded before the slot's 2048 tagged activations (8 per thread) are
// waited for and turned into digits in LDS, once per run; the row outputs
// go out tagged.
template <bool Q6>
__device__ __forceinline__ void down_run(const LayerArgs& a, int slot, int tile0, bool routed,
                                         LayerSmem& sm) {
  constexpr int kDnPasses = dn_passes(Q6);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15;
  if (routed) wait_route_xd(a, slot, true, false, sm);
  const uint8_t* blob = routed ? expert_blob(a, sm.eid) : a.shared;
  const uint8_t* dbase = blob ? blob + 2 * (size_t)kGateBytes : nullptr;
  const uint64_t* act = a.act + (size_t)slot * kFfn;
  auto stage_act = [&] {
    float v[kFfn / 256];
    poll_all(a, [&] {
      bool ok = true;
#pragma unroll
      for (int i = 0; i < kFfn / 256; ++i) {
        const uint64_t t = get_tagged(act + threadIdx.x + 256 * i);
        ok = ok && tag_is(t, a.epoch);
        v[i] = tagged_f(t);
      }
      return ok;
    });
    // element 256 i + 64 w + lane lives in wave w's lanes: record 4 i + w
#pragma unroll
    for (int i = 0; i < kFfn / 256; ++i) digits_to_lds(v[i], sm.xs[4 * i + wave]);
    __syncthreads();
  };
  for (int t = 0; t < kDnPer; ++t) {
    const int row0 = (tile0 + t) * 16 * kDnPasses + wave * 4 * kDnPasses + (lane >> 4);  // + 4j
    float acc[kDnPasses] = {};
    if (!Q6) {
      Q4KGroupLoad ld[kDnPasses][2];
      if (blob) {
#pragma unroll
        for (int j = 0; j < kDnPasses; ++j) {
          const uint8_t* rowp = dbase + (size_t)(row0 + 4 * j) * kQ4KRowFfn;
#pragma unroll
          for (int i = 0; i < 2; ++i)
            ld[j][i] = q4k_load_group(rowp + (4 * i + (l16 >> 2)) * kQ4KBlock, l16 & 3);
        }
      }
      if (t == 0) stage_act();
      if (blob) {
        const Q4KScaleSel sel = q4k_scale_sel(l16 & 3);
#pragma unroll
        for (int j = 0; j < kDnPasses; ++j)
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            acc[j] += q4k_group_dot_ld(ld[j][i], sel, &sm.xs[16 * i + l16]);
            __builtin_amdgcn_sched_barrier(0);  // one group's LDS reads at a time
          }
      }
    } else {
      // 16 halves of 128 elements per 2048-column row: one per lane
      Q6KHalfLoad l6[kDnPasses];
      if (blob) {
#pragma unroll
        for (int j = 0; j < kDnPasses; ++j)
          l6[j] = q6k_load_half(dbase + (size_t)(row0 + 4 * j) * kQ6KRowFfn + (l16 >> 1) * kQ6KBlock,
                                l16 & 1);
      }
      if (t == 0) stage_act();
      if (blob) {
#pragma unroll
        for (int j = 0; j < kDnPasses; ++j) {
          acc[j] = q6k_half_dot_ld(l6[j], &sm.xs[2 * l16]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < kDnPasses; ++j) {
      const float sres = sum16(acc[j]);
      if (l16 == 0)
        put_tagged(a.eo + (size_t)slot * kHidden + row0 + 4 * j, a.epoch, __float_as_uint(sres));
    }

    // the next tile's loads are issued here, not hoisted above this tile's
    // staging and math (they would hold a second tile of registers)
    __builtin_amdgcn_sched_barrier(0);
  }
}

// ---- combine tile: rows 32*tile .. 32*tile+31 ------------------------------------------
// Waits for every slot's output of its rows and for the exact route, then
// sums the routed experts in the reference's slot order and adds the shared
// expert and the residual.
__device__ __forceinline__ void combine_tile(const LayerArgs& a, int tile) {
  const int r = tile * kCombRows + threadIdx.x;
  poll_all(a, [&] {
    if (threadIdx.x >= kCombRows) return true;
    bool ok = true;
    for (int s = 0; s < a.n_slots; ++s) ok = ok && tag_is(get_tagged(a.eo + (size_t)s * kHidden + r), a.epoch);
    return ok;
  });
  // the exact route is finished long before the last expert output
  poll_all(a, [&] {
    if (threadIdx.x >= a.K) return true;
    return tag_is(get_tagged(a.route_w + threadIdx.x), a.epoch) &&
           tag_is(get_tagged(a.route_perm + threadIdx.x), a.epoch);
  });
  if (threadIdx.x >= kCombRows) return;
  float moe = 0.0f;
  for (int k = 0; k < a.K; ++k) {
    const int sl = tagged_i(get_tagged(a.route_perm + k));
    moe = fmaf(tagged_f(get_tagged(a.route_w + k)), tagged_f(get_tagged(a.eo + (size_t)sl * kHidden + r)),
               moe);
  }
  const float sd = a.n_slots > a.K ? tagged_f(get_tagged(a.eo + (size_t)a.K * kHidden + r)) : 0.0f;
  const float hin = a.h_in ? a.h_in[r] : 0.0f;
  a.out[r] = (hin + moe) + sd;
  if (a.moe_out) a.moe_out[r] = moe;
}

// First workgroup of each section of the work list.
struct LayerList {
  int router, route, exact, sgu, sdn, gu, dn, comb, total;
  int gu_items, dn_items;  // work items per slot
};

__host__ __device__ __forceinline__ LayerList layer_list(int K, int n_slots, bool q6) {
  const int hs = n_slots - K;  // 1 with a shared expert
  LayerList l;
  l.gu_items = kGuTileCount / kGuPer;
  l.dn_items = dn_tiles(q6) / kDnPer;
  l.router = kXdItems;
  l.route = l.router + kRows;
  l.exact = l.route + 1;
  l.sgu = l.exact + 1;
  l.sdn = l.sgu + hs * l.gu_items;
  l.gu = l.sdn + hs * l.dn_items;
  l.dn = l.gu + K * l.gu_items;
  l.comb = l.dn + K * l.dn_items;
  l.total = l.comb + kCombTiles;
  return l;
}

}  // namespace

template <bool Q6>
__device__ __forceinline__ void layer_item(const LayerArgs& a, LayerSmem& sm) {
  const LayerList l = layer_list(a.K, a.n_slots, Q6);
  const int it = blockIdx.x;
  if (it < l.router) {
    xd_item(a, it);
  } else if (it < l.route) {
    router_row(a, it - l.router, sm);
  } else if (it == l.route) {
    route_item(a);
  } else if (it == l.exact) {
    exact_item(a);
  } else if (it < l.sdn) {
    gateup_run(a, a.K, (it - l.sgu) * kGuPer, false, sm);
  } else if (it < l.gu) {
    down_run<Q6>(a, a.K, (it - l.sdn) * kDnPer, false, sm);
  } else if (it < l.dn) {
    gateup_run(a, (it - l.gu) / l.gu_items, (it - l.gu) % l.gu_items * kGuPer, true, sm);
  } else if (it < l.comb) {
    down_run<Q6>(a, (it - l.dn) / l.dn_items, (it - l.dn) % l.dn_items * kDnPer, true, sm);
  } else {
    combine_tile(a, it - l.comb);
  }
}

// Q4_K down: every item fits 128 VGPRs, so four workgroups per CU.  Q6_K
// down rows need more registers (the realigned 6-bit words): three.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void k_layer_q4k(
    LayerArgs a) {
  __shared__ LayerSmem sm;
  layer_item<false>(a, sm);
}

__global__ __launch_bounds__(256) void k_layer_q6k(LayerArgs a) {
  __shared__ LayerSmem sm;
  layer_item<true>(a, sm);
}

hipError_t launch_layer(const LayerArgs& a, hipStream_t s) {
  const LayerList l = layer_list(a.K, a.n_slots, a.down_q6 != 0);
  if (a.down_q6)
    hipLaunchKernelGGL(k_layer_q6k, dim3(l.total), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(k_layer_q4k, dim3(l.total), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace fdm
