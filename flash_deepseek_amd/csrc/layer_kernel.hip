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
//   shared expert gate/up tiles (256), the exact route() (1),
//   shared expert down tiles (224)
//   routed gate/up tiles, slot-major (256 per slot)
//   routed down tiles, slot-major (224 per slot), each combined by the
//   last slot to finish its rows
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
// Hand-off.  Values crossing workgroups are written with agent-scope
// stores and read with agent-scope loads (past the per-XCD L2s), and the
// writer waits for its stores before it bumps a counter or sets a flag.
// Flags hold the call's epoch (a number the host increments per call), so
// they never need clearing; arrival counters are reset by their last
// arriver.
#include "fdm_internal.h"
#include "route_device.h"

namespace fdm {

namespace {

constexpr int kStride = kLayerStride;        // ints between counters / flags (256 B)
constexpr int kRows = 256;                   // router rows (R1 experts)
constexpr int kXdItems = kHidden / 64 / 4;   // 28 digit items of 4 groups
constexpr int kGuTileRows = 8;               // gate (and up) rows per gate/up tile
constexpr int kGuTileCount = kFfn / kGuTileRows;      // 256
constexpr int kDnTileRows = 32;              // down rows per down tile
constexpr int kDnTileCount = kHidden / kDnTileRows;   // 224
constexpr int kDnPasses = kDnTileRows / 16;           // row groups per wave
constexpr int kSubBlocks = kFfn / 32;        // activation sub-blocks per slot
constexpr int kArriveGroup = 16;             // router arrival: 16 groups of 16
constexpr unsigned kSpinLimit = 1u << 18;    // polls of one flag (each ~1 us)

// counter slots (units of kStride ints)
constexpr int kCntRouter = 0;                                  // top + 16 groups
constexpr int kCntXd = 17;                                     // digit items
constexpr int kCntSub = 18;                                    // 17 slots x 64
constexpr int kCntSlot = kCntSub + kLayerMaxSlots * kSubBlocks;  // 17
constexpr int kCntTile = kCntSlot + kLayerMaxSlots;            // 224
static_assert(kCntTile + kDnTileCount == kLayerCounters, "counter layout");
// flag slots
constexpr int kFlagRoute = 0;
constexpr int kFlagExact = 1;
constexpr int kFlagErr = 2;
constexpr int kFlagXd = 3;
constexpr int kFlagAct = 4;  // + slot
static_assert(kFlagAct + kLayerMaxSlots <= kLayerFlags, "flag layout");
static_assert(kFlagErr == kLayerFlagErr, "error flag slot");

__device__ __forceinline__ unsigned load_u32_agent(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int load_i32_agent(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_u32_agent(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_i32_agent(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct LayerSmem {
  XGroup xs[kHidden / 64];  // digits of h_post (gate/up) or of one slot's activations (down)
  float red[4];
  int flag;
};

// Thread 0 polls `flag` until it holds this call's epoch; then the whole
// workgroup proceeds.  Gives up after kSpinLimit polls, or at once when
// another workgroup already gave up, recording the epoch in the error flag.
__device__ __forceinline__ void wait_epoch(const LayerArgs& a, int which) {
  if (threadIdx.x == 0) {
    const unsigned* f = a.flags + kStride * which;
    unsigned* err = a.flags + kStride * kFlagErr;
    for (unsigned n = 0;; ++n) {
      if (load_u32_agent(f) == a.epoch) break;
      if (n >= kSpinLimit || load_u32_agent(err) == a.epoch) {
        store_u32_agent(err, a.epoch);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  __syncthreads();
}

__device__ __forceinline__ void set_flag(const LayerArgs& a, int which) {
  store_u32_agent(a.flags + kStride * which, a.epoch);
}

__device__ __forceinline__ int* counter(const LayerArgs& a, int slot) {
  return a.counters + kStride * slot;
}

__device__ __forceinline__ const uint8_t* expert_blob(const LayerArgs& a, int e) {
  if (e < 0 || e >= a.n_experts) return nullptr;  // invalid id: expert contributes 0
  return a.experts + (size_t)e * a.expert_size;
}

// Agent-scope store of the digits of one 32-element sub-block, made by
// make_digits32 in the 32 lanes of a half-wave (l = lane within the half):
// four lanes' bytes go out as one dword.  `sub` selects the record's
// sub-block (elements 32 * sub ..).
__device__ __forceinline__ void store_digits_agent(XGroup* xg, int sub, int l, int8_t da,
                                                   int8_t db, float ds, float dsum) {
  const unsigned ua = (uint8_t)da, ub = (uint8_t)db;
  const unsigned wa = ua | (__shfl_down(ua, 1, 32) << 8) | (__shfl_down(ua, 2, 32) << 16) |
                      (__shfl_down(ua, 3, 32) << 24);
  const unsigned wb = ub | (__shfl_down(ub, 1, 32) << 8) | (__shfl_down(ub, 2, 32) << 16) |
                      (__shfl_down(ub, 3, 32) << 24);
  if ((l & 3) == 0) {
    store_u32_agent(reinterpret_cast<unsigned*>(xg->a) + 8 * sub + l / 4, wa);
    store_u32_agent(reinterpret_cast<unsigned*>(xg->b) + 8 * sub + l / 4, wb);
  }
  if (l == 0) {
    store_agent(&xg->s[sub], ds);
    store_agent(&xg->xsum[sub], dsum);
  }
}

// `n` digit records published by other workgroups into LDS, once `flag` is set.
__device__ __forceinline__ void stage_digits(const LayerArgs& a, int flag, const XGroup* src,
                                             int n, XGroup* dst) {
  wait_epoch(a, flag);
  const unsigned* s = reinterpret_cast<const unsigned*>(src);
  unsigned* d = reinterpret_cast<unsigned*>(dst);
  for (int i = threadIdx.x; i < n * (int)(sizeof(XGroup) / 4); i += 256) d[i] = load_u32_agent(s + i);
  __syncthreads();
}

// ---- digits of h_post: groups 4i .. 4i+3, one per wave ------------------------------
__device__ __forceinline__ void xd_item(const LayerArgs& a, int i) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = 4 * i + wave;
  int8_t da, db;
  float ds, dsum;
  make_digits32(a.h[64 * G + lane], da, db, ds, dsum);
  store_digits_agent(a.xd + G, lane >> 5, lane & 31, da, db, ds, dsum);
  wait_stores_done();
  __syncthreads();
  if (threadIdx.x == 0) {
    int* c = counter(a, kCntXd);
    if (arrive_agent(c) == kXdItems - 1) {
      reset_agent(c);
      set_flag(a, kFlagXd);
    }
  }
}

// ---- router row e ---------------------------------------------------------------------
// Logit e in the canonical order (partial t of 256 accumulates float4 chunks
// t, t+256, ... by fma; xor butterfly per wave; (s0 + s1) + (s2 + s3)),
// stored as its sigmoid score.  The last of the 256 rows to arrive selects
// the expert set and publishes it (prov) with the route flag.
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
  if (threadIdx.x == 0) {
    store_agent(a.scores + e, sigmoid_det((sm.red[0] + sm.red[1]) + (sm.red[2] + sm.red[3])));
    wait_stores_done();
    int* grp = counter(a, kCntRouter + 1 + e / kArriveGroup);
    int last = 0;
    if (arrive_agent(grp) == kArriveGroup - 1) {
      reset_agent(grp);
      last = arrive_agent(counter(a, kCntRouter)) == kRows / kArriveGroup - 1;
    }
    sm.flag = last;
  }
  __syncthreads();
  if (sm.flag && wave == 0) {
    float sc[4], bj[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      sc[j] = load_agent(a.scores + 64 * j + lane);
      bj[j] = a.bias ? a.bias[64 * j + lane] : 0.0f;
    }
    const int id = route_set_lane(sc, bj, a.K);
    if (lane < a.K) store_i32_agent(a.prov + lane, id);
    wait_stores_done();
    if (lane == 0) {
      reset_agent(counter(a, kCntRouter));
      set_flag(a, kFlagRoute);
    }
  }
}

// ---- the exact route() ------------------------------------------------------------------
// The reference's slot order and weights (idx, w) and, for the combine,
// perm[k] = the slot of prov that runs expert idx[k].
__device__ __forceinline__ void exact_route(const LayerArgs& a) {
  wait_epoch(a, kFlagRoute);
  if (threadIdx.x >= 64) return;
  const int lane = threadIdx.x;
  float sc[4], bj[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    sc[j] = load_agent(a.scores + 64 * j + lane);
    bj[j] = a.bias ? a.bias[64 * j + lane] : 0.0f;
  }
  int id;
  float wv;
  route_exact_lane(sc, bj, a.K, 2.5f, id, wv);
  if (lane < a.K) {
    int p = 0;
    for (int s = a.K - 1; s >= 0; --s) p = load_i32_agent(a.prov + s) == id ? s : p;
    store_i32_agent(a.idx + lane, id);
    store_agent(a.w + lane, wv);
    store_i32_agent(a.perm + lane, p);
  }
  wait_stores_done();
  if (lane == 0) set_flag(a, kFlagExact);
}

// ---- gate/up tile: rows 8*tile .. 8*tile+7 of gate and up of one slot --------------
// Wave w owns rows 2w, 2w+1 in both matrices (lanes 0-31 gate, 32-63 up, 16
// lanes per row); SwiGLU in registers.  The weights are loaded before the
// digits of h_post are staged.  The last of the four tiles of a 32-row
// sub-block makes the sub-block's digits; the last sub-block of the slot
// sets the slot's activation flag.
__device__ __forceinline__ void gateup_tile(const LayerArgs& a, int slot, int tile,
                                            const uint8_t* blob, LayerSmem& sm) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane >> 4, l16 = lane & 15, g = l16 & 3;
  const int row = tile * kGuTileRows + 2 * wave + (q & 1);
  Q4KGroupLoad ld[7];
  if (blob) {
    const uint8_t* rowp = blob + (q >= 2 ? kGateBytes : 0) + (size_t)row * kQ4KRowHidden;
#pragma unroll
    for (int i = 0; i < 7; ++i) ld[i] = q4k_load_group(rowp + (4 * i + (l16 >> 2)) * kQ4KBlock, g);
  }
  stage_digits(a, kFlagXd, a.xd, kHidden / 64, sm.xs);
  float acc = 0.0f;
  if (blob) {
    const Q4KScaleSel sel = q4k_scale_sel(g);
#pragma unroll
    for (int i = 0; i < 7; ++i) {
      acc += q4k_group_dot_ld(ld[i], sel, &sm.xs[16 * i + l16]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  acc = sum16(acc);
  const float up = __shfl(acc, (lane + 32) & 63);
  float* act = a.act + (size_t)slot * kFfn;
  if (lane == 0 || lane == 16) {
    store_agent(act + row, silu_mul(acc, up));
    wait_stores_done();
  }
  __syncthreads();
  const int sub = tile >> 2;
  int* sub_cnt = counter(a, kCntSub + slot * kSubBlocks + sub);
  if (threadIdx.x == 0) sm.flag = arrive_agent(sub_cnt) == 3;
  __syncthreads();
  if (sm.flag && wave == 0) {
    // both half-waves make the same 32 digits; lanes 0-31 store them
    int8_t da, db;
    float ds, dsum;
    make_digits32(load_agent(act + sub * 32 + (lane & 31)), da, db, ds, dsum);
    if (lane < 32)
      store_digits_agent(a.act_xd + (size_t)slot * (kFfn / 64) + (sub >> 1), sub & 1, lane, da,
                         db, ds, dsum);
    wait_stores_done();
    if (lane == 0) {
      reset_agent(sub_cnt);
      int* slot_cnt = counter(a, kCntSlot + slot);
      if (arrive_agent(slot_cnt) == kSubBlocks - 1) {
        reset_agent(slot_cnt);
        set_flag(a, kFlagAct + slot);
      }
    }
  }
}

// ---- down tile: rows 32*tile .. 32*tile+31 of one slot's down matrix ----------------
// Wave w owns rows 8w .. 8w+7 of the tile as row groups of 16 lanes (row
// 8w + 4j + lane/16 in pass j).  All weights of the tile are loaded first,
// then the slot's activation digits are waited for and staged.  The last of
// the n_slots slots of a row tile to finish combines them in the
// reference's slot order and adds the shared expert and the residual.
__device__ __forceinline__ void down_tile(const LayerArgs& a, int slot, int tile,
                                          const uint8_t* blob, LayerSmem& sm) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15;
  const int row0 = tile * kDnTileRows + wave * 8 + (lane >> 4);  // + 4j
  const uint8_t* dbase = blob ? blob + 2 * (size_t)kGateBytes : nullptr;
  const XGroup* axd = a.act_xd + (size_t)slot * (kFfn / 64);
  float acc[kDnPasses] = {};
  if (!a.down_q6) {
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
    stage_digits(a, kFlagAct + slot, axd, kFfn / 64, sm.xs);
    if (blob) {
      const Q4KScaleSel sel = q4k_scale_sel(l16 & 3);
#pragma unroll
      for (int j = 0; j < kDnPasses; ++j)
#pragma unroll
        for (int i = 0; i < 2; ++i) acc[j] += q4k_group_dot_ld(ld[j][i], sel, &sm.xs[16 * i + l16]);
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
    stage_digits(a, kFlagAct + slot, axd, kFfn / 64, sm.xs);
    if (blob) {
#pragma unroll
      for (int j = 0; j < kDnPasses; ++j) acc[j] = q6k_half_dot_ld(l6[j], &sm.xs[2 * l16]);
    }
  }
#pragma unroll
  for (int j = 0; j < kDnPasses; ++j) {
    const float v = sum16(acc[j]);
    if (l16 == 0) store_agent(a.eo + (size_t)slot * kHidden + row0 + 4 * j, v);
  }
  wait_stores_done();
  __syncthreads();
  int* tile_cnt = counter(a, kCntTile + tile);
  if (threadIdx.x == 0) sm.flag = arrive_agent(tile_cnt) == a.n_slots - 1;
  __syncthreads();
  if (sm.flag) {
    wait_epoch(a, kFlagExact);
    if (threadIdx.x < kDnTileRows) {
      const int r = tile * kDnTileRows + threadIdx.x;
      float moe = 0.0f;
      for (int k = 0; k < a.K; ++k) {
        const int sl = load_i32_agent(a.perm + k);
        moe = fmaf(load_agent(a.w + k), load_agent(a.eo + (size_t)sl * kHidden + r), moe);
      }
      const float sd = a.n_slots > a.K ? load_agent(a.eo + (size_t)a.K * kHidden + r) : 0.0f;
      const float hin = a.h_in ? a.h_in[r] : 0.0f;
      a.out[r] = (hin + moe) + sd;
      if (a.moe_out) a.moe_out[r] = moe;
    }
    if (threadIdx.x == 0) reset_agent(tile_cnt);
  }
}

// First workgroup of each section of the work list.
struct LayerList {
  int router, sgu, exact, sdn, gu, dn, total;
};

__host__ __device__ __forceinline__ LayerList layer_list(int K, int n_slots) {
  const int hs = n_slots - K;  // 1 with a shared expert
  LayerList l;
  l.router = kXdItems;
  l.sgu = l.router + kRows;
  l.exact = l.sgu + hs * kGuTileCount;
  l.sdn = l.exact + 1;
  l.gu = l.sdn + hs * kDnTileCount;
  l.dn = l.gu + K * kGuTileCount;
  l.total = l.dn + K * kDnTileCount;
  return l;
}

}  // namespace

__global__ __launch_bounds__(256) void k_layer(LayerArgs a) {
  __shared__ LayerSmem sm;
  const LayerList l = layer_list(a.K, a.n_slots);
  const int it = blockIdx.x;
  if (it < l.router) {
    xd_item(a, it);
  } else if (it < l.sgu) {
    router_row(a, it - l.router, sm);
  } else if (it < l.exact) {
    gateup_tile(a, a.K, it - l.sgu, a.shared, sm);
  } else if (it == l.exact) {
    exact_route(a);
  } else if (it < l.gu) {
    down_tile(a, a.K, it - l.sdn, a.shared, sm);
  } else if (it < l.dn) {
    wait_epoch(a, kFlagRoute);
    const int slot = (it - l.gu) / kGuTileCount;
    gateup_tile(a, slot, (it - l.gu) % kGuTileCount,
                expert_blob(a, load_i32_agent(a.prov + slot)), sm);
  } else {
    wait_epoch(a, kFlagRoute);
    const int slot = (it - l.dn) / kDnTileCount;
    down_tile(a, slot, (it - l.dn) % kDnTileCount, expert_blob(a, load_i32_agent(a.prov + slot)),
              sm);
  }
}

hipError_t launch_layer(const LayerArgs& a, hipStream_t s) {
  const LayerList l = layer_list(a.K, a.n_slots);
  hipLaunchKernelGGL(k_layer, dim3(l.total), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace fdm
