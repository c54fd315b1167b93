// stream_kernel.hip -- the batch-1 MoE layer of one token as ONE launch of
// 256 resident workgroups (one per CU) that stream the layer's weights
// through LDS.  Same contract and results as the ordered-item kernel
// (layer_kernel.hip): router logits (infer.m:350-353), route()
// (infer.m:920-991), the routed and shared experts (encode_expert,
// infer.m:1559-1575), the combine in slot order (infer.m:1689-1695) and the
// residual (infer.m:1922).
//
// Ownership.  Workgroup c owns 1/256 of every matrix of the layer: router
// row c, gate and up rows 8c .. 8c+7 and down rows 28c .. 28c+27 of the
// shared expert and of each routed slot.  Its down rows are the same for
// every slot, so the combine of output rows 28c .. 28c+27 needs nothing
// from other workgroups but the route; the only cross-workgroup values are
// the 256 router scores and each slot's 2048 activations (tagged words, as
// in the item kernel: {epoch, payload} in one agent-scope store, the
// reader's load is its own readiness check).
//
// Streaming.  The workgroup's share is a fixed sequence of chunks of at
// 16 KB (the router row in two, then the shared expert's gate, up and down
// rows, each slot's gate and up rows, each slot's down rows: a gate or up
// share is two chunks of 4 rows, a Q4_K down share two of 14 rows, a Q6_K
// one four of 7).  They flow through a ring of eight 16 KB LDS slots (up to
// seven chunks in flight while one is read) filled by
// direct global -> LDS loads (global_load_lds_dwordx4, 1 KB per wave
// instruction).  The 16 waves split into three roles that synchronise
// through LDS counters only (no workgroup barrier inside the stream: a
// stalled load issue must not hold up the arithmetic, nor the reverse):
//  - producers (waves 12-15) issue the ring loads, 8 KB of every chunk
//    each, and publish a chunk once their share has landed; a slot is
//    refilled when all consumers have released it.  They make no other
//    global access: vmcnt retires in order on gfx9, so anything queued
//    behind in-flight ring loads would wait for them.
//  - consumers (waves 4-11) contract the chunks from LDS: wave 4 + r owns
//    gate/up row r (publishing its activations itself) and a share of the
//    down rows.
//  - aux (waves 0-3) compute the router row, the route, the exact route and,
//    ahead of the consumers, each down slot's activation digits.
// The ring loads are inline assembly, so the compiler neither tracks them
// nor inserts waits for them; every wait on them is an explicit s_waitcnt.
//
// Requires all 256 workgroups to be resident at once (one per CU: the LDS
// footprint allows no second one); the host runs it only when selected
// (fdm_set_layer_kernel) and only on devices with at least 256 CUs.  It
// measures slower than the item kernel on MI355X (~77 vs ~61 us per
// token), so it is not the default.  Every cross-workgroup wait is bounded like the item
// kernel's: a timeout records the call's epoch in the error flag, which
// releases every other wait, and the launch completes.
#include "fdm_internal.h"
#include "route_device.h"

namespace fdm {

namespace {

constexpr int kSWg = 256;                       // workgroups, one per CU
constexpr int kThreads = 1024;                  // 16 waves
constexpr int kAuxWaves = 4;                    // waves 0-3
constexpr int kCons0 = 4, kConsWaves = 8;       // waves 4-11
constexpr int kDmaWave0 = 12;                   // waves 12-15 issue the ring loads
constexpr int kProdWaves = 4;
constexpr int kChunk = 16384;                   // ring slot bytes
constexpr int kRingSlots = 8;
constexpr int kDmaWaveInstrs = kChunk / (kProdWaves * 1024);  // 4: ring loads per DMA wave per chunk
constexpr int kRtChunks = 2;                    // the router row: 16 KB + 12 KB
constexpr int kGuRows = kFfn / kSWg;            // 8 gate (and up) rows per workgroup
constexpr int kDnRows = kHidden / kSWg;         // 28 down rows per workgroup
constexpr int kGuHalf = kGuRows / 2;            // 4 gate (or up) rows per chunk
constexpr int kQ4Rows = kDnRows / 2;            // 14 Q4_K down rows per chunk
constexpr int kQ6Rows = kDnRows / 4;            // 7 Q6_K down rows per chunk
constexpr int kRouterBytes = kHidden * 4;       // 28672
constexpr unsigned kSpin = 1u << 17;            // polls of one cross-workgroup wait
constexpr unsigned kLdsSpin = 1u << 22;         // polls of one in-workgroup wait
constexpr int kErrFlag = kLayerFlagErr * kLayerStride;
static_assert(kGuHalf * kQ4KRowHidden <= kChunk && kQ4Rows * kQ4KRowFfn <= kChunk &&
                  kQ6Rows * kQ6KRowFfn <= kChunk && kRouterBytes <= kRtChunks * kChunk,
              "chunk sizes");

enum ChunkKind { kRouter, kGate, kUp, kDown };

struct Chunk {
  const uint8_t* src;  // global bytes (a valid address even for an empty chunk)
  int bytes;
  int kind, slot, part;  // part: gate/up half (rows 4 part ..) or down part
  bool live;           // false: an invalid expert id, the chunk's results are zero
};

// The workgroup's chunk sequence.  hs = 1 with a shared expert (slot K).
struct Plan {
  int dnc, n_sh, gu0, dn0, total;
  __device__ Plan(int K, int n_slots, bool q6) {
    dnc = q6 ? kDnRows / kQ6Rows : kDnRows / kQ4Rows;
    n_sh = n_slots > K ? 4 + dnc : 0;
    gu0 = kRtChunks + n_sh;
    dn0 = gu0 + 4 * K;
    total = dn0 + dnc * K;
  }
  // Order of a slot among the down slots (the shared one first) and its activation buffer.
  __device__ int down_ord(int slot, int K) const { return slot == K ? 0 : slot + (n_sh ? 1 : 0); }
  __device__ int act_buf(int slot, int K) const { return down_ord(slot, K) & 1; }
};

struct StreamSmem {
  XGroup xs[kHidden / 64];          // digits of h_post
  XGroup xa[2][kFfn / 64];          // digits of a down slot's activations (double-buffered)
  RouteScratch rs;                  // the exact route
  float eo[kLayerMaxSlots][kDnRows];  // down outputs of the owned rows, per slot
  float red[4];
  int eid[kLayerMaxSlots];          // expert of each slot (set order), -1: none
  float wk[16];                     // exact route: weight of slot k
  int perm[16];                     // exact route: set position of slot k
  // in-workgroup counters (monotonic within the launch)
  int land[kRingSlots];             // producer shares landed, per slot
  int rel[kRingSlots];              // consumer releases, per slot
  int xa_ready[2];                  // down-slot order index whose digits are in xa[b]
  int xa_used[2];                   // consumer waves done with xa[b]
  int route_ready;                  // eid valid
  int aux_cnt;                      // aux-wave arrivals (router row, gathers, enter flags)
};

// ---- explicit waits and barriers -----------------------------------------------------------
__device__ __forceinline__ void bar() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// One 16-byte-per-lane direct load into LDS: lane i reads sbase + voff and
// writes lds + 16 i (M0 holds the wave-uniform LDS byte address; the
// global address is a uniform base plus a 32-bit lane offset).
typedef __attribute__((address_space(3))) const uint8_t* lds_cptr;
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_cptr)(const uint8_t*)p;
}
__device__ __forceinline__ void dma16(const uint8_t* sbase, uint32_t voff, uint32_t lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
  // readfirstlane returns int: both halves go through uint32_t, or the low
  // half would sign-extend over the high one.
  const uint64_t b = (uint64_t)(uintptr_t)sbase;
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  const uint64_t sb = ((uint64_t)hi << 32) | (uint64_t)lo;
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sb), "{m0}"(m0) : "memory");
}

// A DMA wave's share of a chunk: 8 KB into the ring slot at LDS byte
// address `slot`; lanes past `bytes` re-read the chunk's first bytes (in
// bounds; their LDS bytes are never read).  The lane offset is recomputed
// per call (opaque to the optimiser), so no per-round offsets stay live.
__device__ __forceinline__ void issue_chunk(const Chunk& ch, uint32_t slot, int wave) {
  const int dw = wave - kDmaWave0;  // uniform: the round offsets stay scalar
  uint32_t l16 = 16u * (threadIdx.x & 63);
  asm volatile("" : "+v"(l16));
#pragma unroll
  for (int k = 0; k < kDmaWaveInstrs; ++k) {
    const uint32_t base = (uint32_t)(dw * kDmaWaveInstrs + k) * 1024u;
    const uint32_t off = l16 + base;
    dma16(ch.src, off + 16u <= (uint32_t)ch.bytes ? off : 0u, slot + base);
  }
}

// ---- tagged words ------------------------------------------------------------------------
__device__ __forceinline__ void put_tag(uint64_t* p, unsigned epoch, uint32_t bits) {
  __hip_atomic_store(p, ((uint64_t)epoch << 32) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t get_tag(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool tag_ok(uint64_t v, unsigned epoch) { return (unsigned)(v >> 32) == epoch; }

// Poll by the calling waves only (no barrier inside): retries try_once()
// until it succeeds on every calling lane, bounded as the item kernel's
// waits.  Returns false on giving up (the error flag then holds the epoch).
template <typename F>
__device__ __forceinline__ bool poll_waves(const LayerArgs& a, F&& try_once) {
  unsigned* err = a.flags + kErrFlag;
  for (unsigned n = 0;; ++n) {
    if (__all(try_once())) return true;
    if ((n & 63) == 63) {
      const bool give_up =
          n >= kSpin || __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == a.epoch;
      if (give_up) {
        __hip_atomic_store(err, a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
      }
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

__device__ __forceinline__ const uint8_t* blob_of(const LayerArgs& a, int e) {
  if (e < 0 || e >= a.n_experts) return nullptr;
  return a.experts + (size_t)e * a.expert_size;
}

// Chunk q of workgroup c (routed chunks read sm.eid).
__device__ __forceinline__ Chunk chunk_of(const LayerArgs& a, const Plan& P, const StreamSmem& sm, int c,
                                          int q, bool q6) {
  Chunk ch;
  ch.live = true;
  ch.part = 0;
  const uint8_t* blob;
  int j;  // 0-3: gate h0, gate h1, up h0, up h1; 4 + p: down part p
  if (q < kRtChunks) {
    ch.kind = kRouter;
    ch.slot = 0;
    ch.part = q;
    ch.src = reinterpret_cast<const uint8_t*>(a.Wg + (size_t)c * kHidden) + q * kChunk;
    ch.bytes = q ? kRouterBytes - kChunk : kChunk;
    return ch;
  } else if (q < kRtChunks + P.n_sh) {
    ch.slot = a.K;
    blob = a.shared;
    j = q - kRtChunks;
  } else if (q < P.dn0) {
    ch.slot = (q - P.gu0) >> 2;
    blob = blob_of(a, sm.eid[ch.slot]);
    j = (q - P.gu0) & 3;
  } else {
    ch.slot = (q - P.dn0) / P.dnc;
    blob = blob_of(a, sm.eid[ch.slot]);
    j = 4 + (q - P.dn0) % P.dnc;
  }
  ch.live = blob != nullptr;
  if (!blob) blob = reinterpret_cast<const uint8_t*>(a.Wg);  // any readable bytes
  if (j < 4) {
    ch.kind = j < 2 ? kGate : kUp;
    ch.part = j & 1;
    ch.src = blob + (j < 2 ? 0 : kGateBytes) + (size_t)(c * kGuRows + ch.part * kGuHalf) * kQ4KRowHidden;
    ch.bytes = kGuHalf * kQ4KRowHidden;
  } else {
    ch.kind = kDown;
    ch.part = j - 4;
    const uint8_t* dn = blob + 2 * (size_t)kGateBytes;
    if (q6) {
      ch.src = dn + (size_t)(c * kDnRows + ch.part * kQ6Rows) * kQ6KRowFfn;
      ch.bytes = kQ6Rows * kQ6KRowFfn;
    } else {
      ch.src = dn + (size_t)(c * kDnRows + ch.part * kQ4Rows) * kQ4KRowFfn;
      ch.bytes = kQ4Rows * kQ4KRowFfn;
    }
  }
  if (!ch.live) ch.bytes = 16;
  return ch;
}

// ---- reductions ----------------------------------------------------------------------------
// Inclusive row prefix by DPP row shifts: lane 15 of each row of 16 ends
// with the row's sum.
__device__ __forceinline__ float row_prefix(float v) {
  v += row_shr<1>(v, 0.0f);
  v += row_shr<2>(v, 0.0f);
  v += row_shr<4>(v, 0.0f);
  v += row_shr<8>(v, 0.0f);
  return v;
}
// Sum over the wave (uniform result).
__device__ __forceinline__ float wave_sum(float v) {
  v = row_prefix(v);
  return (readlane_f(v, 15) + readlane_f(v, 31)) + (readlane_f(v, 47) + readlane_f(v, 63));
}

// ---- in-workgroup counters (LDS) ------------------------------------------------------------
// LDS operations of one wave complete in order and the ring loads' LDS
// writes are complete when vmcnt says so, so a counter written after the
// data it announces (with the compiler kept from reordering) publishes it.
__device__ __forceinline__ int lds_load(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_add(int* p, int v) {
  asm volatile("" ::: "memory");  // the caller's earlier LDS accesses are issued first
  __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_store(int* p, int v) {
  asm volatile("" ::: "memory");
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Wait until *p >= target (or == target).  Bounded: giving up records the
// error epoch (the launch then completes with an unspecified result).
__device__ __forceinline__ void lds_wait_ge(const LayerArgs& a, const int* p, int target) {
  for (unsigned n = 0; lds_load(p) < target; ++n) {
    if (n >= kLdsSpin) {
      __hip_atomic_store(a.flags + kErrFlag, a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  asm volatile("" ::: "memory");  // data reads after the wait stay after it
}
__device__ __forceinline__ void lds_wait_eq(const LayerArgs& a, const int* p, int target) {
  for (unsigned n = 0; lds_load(p) != target; ++n) {
    if (n >= kLdsSpin) {
      __hip_atomic_store(a.flags + kErrFlag, a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  asm volatile("" ::: "memory");
}

// DMA waves: wait until at most `younger` of their chunks (4 loads each) are in flight.
__device__ __forceinline__ void wait_ring(int younger) {
  static_assert(kDmaWaveInstrs == 4 && kRingSlots == 8, "vmcnt immediates below");
  switch (younger) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(16)" ::: "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(20)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(24)" ::: "memory"); break;
  }
}

// ---- consumers (weights from the ring slot, digits from registers or LDS) -----------------
// Gate or up row `row`: lane l takes groups l (digits resident in x1) and
// l + 64 (lanes < 48; digits from LDS).  Returns the row total (uniform).
__device__ __forceinline__ float gu_row(const uint8_t* slot, int row, int lane, const XDig& x1,
                                        const StreamSmem& sm) {
  const int g = lane & 3;
  const Q4KScaleSel sel = q4k_scale_sel(g);
  const uint8_t* rp = slot + row * kQ4KRowHidden;
  const Q4KGroupLoad l1 = q4k_load_group(rp + (lane >> 2) * kQ4KBlock, g);
  float acc = q4k_group_dot_ld(l1, sel, x1);
  const bool ok2 = lane < kHidden / 64 - 64;
  const int g2 = ok2 ? lane + 64 : 4 * (kHidden / 256 - 1) + g;  // stand-in: the quad stays converged
  const Q4KGroupLoad l2 = q4k_load_group(rp + (g2 >> 2) * kQ4KBlock, g);
  const float v2 = q4k_group_dot_ld(l2, sel, &sm.xs[g2]);
  acc += ok2 ? v2 : 0.0f;
  return wave_sum(acc);
}

// Q4_K down rows 28c + 14 part .. +13 (consumer wave cw): group grp = lane & 31
// of row rr = 2 cw + (lane >> 5) (rows 14-15 of wave 7 compute and drop).
__device__ __forceinline__ void dn_rows_q4k(const uint8_t* slot, const XGroup* xa, StreamSmem& sm, int s, int part,
                                            int cw, int lane, bool live) {
  const int grp = lane & 31, hi = lane >> 5, g = lane & 3;
  const int rr = 2 * cw + hi, row = min(rr, kQ4Rows - 1);
  const XDig xd = load_xdig(&xa[grp]);
  const Q4KGroupLoad ld = q4k_load_group(slot + row * kQ4KRowFfn + (grp >> 2) * kQ4KBlock, g);
  const float p = row_prefix(q4k_group_dot_ld(ld, q4k_scale_sel(g), xd));
  const float sum = hi ? readlane_f(p, 47) + readlane_f(p, 63) : readlane_f(p, 15) + readlane_f(p, 31);
  if (grp == 0 && rr < kQ4Rows) sm.eo[s][kQ4Rows * part + rr] = live ? sum : 0.0f;
}

// Q6_K down rows 28c + 7 part .. +6: item 64 cw + lane < 112, row item >> 4,
// one 128-element half per lane (consumer waves 0-1).
__device__ __forceinline__ void dn_rows_q6k(const uint8_t* slot, const XGroup* xa, StreamSmem& sm, int s, int part,
                                            int cw, int lane, bool live) {
  if (cw >= 2) return;
  const int item = 64 * cw + lane, l16 = item & 15;
  const int rr = min(item >> 4, kQ6Rows - 1);
  const Q6KHalfLoad l6 = q6k_load_half(slot + rr * kQ6KRowFfn + (l16 >> 1) * kQ6KBlock, l16 & 1);
  const float v = sum16(q6k_half_dot_ld(l6, &xa[2 * l16]));
  if (l16 == 0 && (item >> 4) < kQ6Rows) sm.eo[s][kQ6Rows * part + rr] = live ? v : 0.0f;
}

// Digits of 64 consecutive values held by one wave (lane l: element l) into a record.
__device__ __forceinline__ void digits_to(float v, XGroup& xg, int lane) {
  int8_t da, db;
  float ds, dsum;
  make_digits32(v, da, db, ds, dsum);
  xg.a[lane] = da;
  xg.b[lane] = db;
  if ((lane & 31) == 0) {
    xg.s[lane >> 5] = ds;
    xg.xsum[lane >> 5] = dsum;
  }
}

// Aux waves: a slot's 2048 activations (thread t < 256: elements t + 256 i)
// -> digits in xa (group g = 4 i + wave).
__device__ __forceinline__ void gather_act(const LayerArgs& a, int slot, int t, XGroup* xa) {
  const int lane = t & 63, wave = t >> 6;
  const uint64_t* act = a.act + (size_t)slot * kFfn;
  uint64_t raw[8];
  poll_waves(a, [&] {
    bool o = true;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      raw[i] = get_tag(act + t + 256 * i);
      o = o && tag_ok(raw[i], a.epoch);
    }
    return o;
  });
#pragma unroll
  for (int i = 0; i < 8; ++i) digits_to(__uint_as_float((uint32_t)raw[i]), xa[4 * i + wave], lane);
}

// ---- roles -----------------------------------------------------------------------------------
// Producers: chunk q is announced once this wave's share has landed; chunk
// q + 7 then goes into the slot of chunk q - 1 as soon as every consumer
// has released that (and, for a routed chunk, the route is known).  Chunks
// 0 and 1 (the router row) belong to the aux waves.
template <bool Q6>
__device__ __forceinline__ void producer(const LayerArgs& a, const Plan& P, StreamSmem& sm, uint8_t* ring, int c,
                                         int wave) {
  int issued = min(P.total, kRingSlots);  // chunks 2-7 were issued before
  for (int q = 1; q < P.total; ++q) {
    if (q >= kRtChunks) {
      wait_ring(issued - 1 - q);
      if ((threadIdx.x & 63) == 0) lds_add(&sm.land[q & (kRingSlots - 1)], 1);
    }
    const int nq = q + kRingSlots - 1;
    if (nq < P.total) {
      lds_wait_ge(a, &sm.rel[(q - 1) & (kRingSlots - 1)], kConsWaves * (((q - 1) / kRingSlots) + 1));
      if (nq >= P.gu0) lds_wait_ge(a, &sm.route_ready, 1);
      issue_chunk(chunk_of(a, P, sm, c, nq, Q6), lds_addr(ring) + (nq & (kRingSlots - 1)) * kChunk, wave);
      issued = nq + 1;
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Consumers: wave 4 + cw owns gate/up row cw of every slot (in the chunk of
// half cw >> 2) and its share of every down chunk.  Chunk q is read once its
// producer shares have landed; every consumer releases every chunk (one it
// does not read at once).
template <bool Q6>
__device__ __forceinline__ void consumer(const LayerArgs& a, const Plan& P, StreamSmem& sm, const uint8_t* ring,
                                         int c, int cw, int lane) {
  XDig x1 = load_xdig(&sm.xs[lane]);  // gate/up group `lane`: resident through the gate/up chunks
  float gate = 0.0f;
  for (int q = kRtChunks; q < P.total; ++q) {
    const Chunk ch = chunk_of(a, P, sm, c, q, Q6);
    int ln = lane;  // opaque per chunk: lane-dependent addresses are formed here, not hoisted
    asm volatile("" : "+v"(ln));
    const uint8_t* slot = ring + (q & (kRingSlots - 1)) * kChunk;
    const bool gu = ch.kind == kGate || ch.kind == kUp;
    if (!gu || ch.part == (cw >> 2)) {
      lds_wait_ge(a, &sm.land[q & (kRingSlots - 1)], kProdWaves * ((q / kRingSlots) + 1));
      if (ch.kind == kGate) {
        gate = gu_row(slot, cw & 3, ln, x1, sm);
      } else if (ch.kind == kUp) {
        const float up = gu_row(slot, cw & 3, ln, x1, sm);
        if (ln == 0) {
          const float act = ch.live ? silu_mul(gate, up) : 0.0f;
          put_tag(a.act + (size_t)ch.slot * kFfn + c * kGuRows + cw, a.epoch, __float_as_uint(act));
        }
      } else {
        const int b = P.act_buf(ch.slot, a.K);
        if (ch.part == 0) lds_wait_eq(a, &sm.xa_ready[b], P.down_ord(ch.slot, a.K));
        if (Q6)
          dn_rows_q6k(slot, sm.xa[b], sm, ch.slot, ch.part, cw, ln, ch.live);
        else
          dn_rows_q4k(slot, sm.xa[b], sm, ch.slot, ch.part, cw, ln, ch.live);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (ch.part == P.dnc - 1 && ln == 0) lds_add(&sm.xa_used[b], 1);
        if (q + 1 < P.dn0)
          x1 = load_xdig(&sm.xs[lane]);
        else
          x1 = XDig{};  // no gate/up chunk follows
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's reads of the slot are done
    }
    if (ln == 0) lds_add(&sm.rel[q & (kRingSlots - 1)], 1);
  }
}

// Aux: after the route, the shared slot's activation digits (its down chunk
// follows its up rows directly), the exact route, then the routed slots'
// digits, each one buffer ahead of the consumers.
template <bool Q6>
__device__ __forceinline__ void aux(const LayerArgs& a, const Plan& P, StreamSmem& sm, int c, int t, int wave,
                                    int lane, const float (&sc)[4], const int (&vk)[4]) {
  int arrivals = 2 * kAuxWaves;  // router-row arrivals so far
  auto publish = [&](int b, int ord) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (lane == 0) lds_add(&sm.aux_cnt, 1);
    arrivals += kAuxWaves;
    if (wave == 0) {
      lds_wait_ge(a, &sm.aux_cnt, arrivals);
      if (lane == 0) lds_store(&sm.xa_ready[b], ord);
    }
  };
  if (P.n_sh) {
    gather_act(a, a.K, t, sm.xa[0]);
    publish(0, 0);
  }
  route_enter_flags_aux(sm.rs, a.K, t);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  if (lane == 0) lds_add(&sm.aux_cnt, 1);
  arrivals += kAuxWaves;
  if (wave == 0) {
    lds_wait_ge(a, &sm.aux_cnt, arrivals);
    int id;
    float wv;
    route_exact_slots(sm.rs, vk, sc, a.K, 2.5f, id, wv);
    int p = 0;
    for (int s = a.K - 1; s >= 0; --s) p = sm.eid[s] == id ? s : p;
    if (lane < a.K) {
      sm.wk[lane] = wv;
      sm.perm[lane] = p;
      if (c == 0) {
        a.idx[lane] = id;
        a.w[lane] = wv;
      }
    }
  }
  for (int s = 0; s < a.K; ++s) {
    const int ord = P.down_ord(s, a.K), b = ord & 1;
    if (ord >= 2) lds_wait_ge(a, &sm.xa_used[b], kConsWaves * (ord >> 1));
    gather_act(a, s, t, sm.xa[b]);
    publish(b, ord);
  }
}

template <bool Q6>
__device__ __forceinline__ void stream_layer(const LayerArgs& a) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) uint8_t ring[kRingSlots][kChunk];
  __shared__ StreamSmem sm;
  const int c = blockIdx.x, t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // uniform: role branches are scalar
  const bool aux_w = wave < kAuxWaves, cons_w = wave >= kCons0 && wave < kDmaWave0, prod_w = wave >= kDmaWave0;
  const Plan P(a.K, a.n_slots, Q6);

  // ---- prologue: the router row (aux waves), h_post in registers ----
  if (aux_w) {
    const uint8_t* src = reinterpret_cast<const uint8_t*>(a.Wg + (size_t)c * kHidden);
#pragma unroll
    for (int k = 0; k < kRouterBytes / 4096; ++k) {
      const int base = (wave * (kRouterBytes / 4096) + k) * 1024;
      dma16(src, (uint32_t)(base + 16 * lane), lds_addr(ring[0]) + base);
    }
  }
  if (t == 0) {
    for (int s = 0; s < kLayerMaxSlots; ++s) sm.eid[s] = -1;
    for (int i = 0; i < kRingSlots; ++i) {
      sm.land[i] = 0;
      sm.rel[i] = 0;
    }
    sm.xa_ready[0] = sm.xa_ready[1] = -1;
    sm.xa_used[0] = sm.xa_used[1] = 0;
    sm.route_ready = 0;
    sm.aux_cnt = 0;
  }
  const float4* h4 = reinterpret_cast<const float4*>(a.h);
  float4 hv[kHidden / 1024];  // router layout: float4 t + 256 i (aux waves)
#pragma unroll
  for (int i = 0; i < kHidden / 1024; ++i) hv[i] = aux_w ? h4[t + 256 * i] : float4{0.0f, 0.0f, 0.0f, 0.0f};
  // digit layout: element 64 (7 w + i) + lane; wave 0 (the route) leaves its
  // groups to wave 15
  float hd[kHidden / 64 / 16], hd0[kHidden / 64 / 16];
#pragma unroll
  for (int i = 0; i < kHidden / 64 / 16; ++i) {
    hd[i] = wave ? a.h[64 * (7 * wave + i) + lane] : 0.0f;
    hd0[i] = wave == 15 ? a.h[64 * i + lane] : 0.0f;
  }
  // h_post arrives here in every wave, so no later use of it waits on ring loads
#pragma unroll
  for (int i = 0; i < kHidden / 1024; ++i) asm volatile("" ::"v"(hv[i].x), "v"(hv[i].y), "v"(hv[i].z), "v"(hv[i].w));
#pragma unroll
  for (int i = 0; i < kHidden / 64 / 16; ++i) asm volatile("" ::"v"(hd[i]), "v"(hd0[i]));
  bar();  // counters initialised
  if (prod_w)  // the shared expert's chunks (route-independent) into slots 2-7
    for (int q = kRtChunks; q < min(P.total, kRingSlots); ++q)
      if (q < P.gu0) issue_chunk(chunk_of(a, P, sm, c, q, Q6), lds_addr(ring[0]) + q * kChunk, wave);

  // ---- router row c -> tagged sigmoid score (canonical order of router_row) ----
  if (aux_w) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's router loads
    if (lane == 0) lds_add(&sm.aux_cnt, 1);
    lds_wait_ge(a, &sm.aux_cnt, kAuxWaves);  // every aux wave's share of the row landed
    const float4* w4 = reinterpret_cast<const float4*>(ring[0]);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < kHidden / 1024; ++i) {
      const float4 wv = w4[t + 256 * i];
      acc = fmaf(wv.x, hv[i].x, acc);
      acc = fmaf(wv.y, hv[i].y, acc);
      acc = fmaf(wv.z, hv[i].z, acc);
      acc = fmaf(wv.w, hv[i].w, acc);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc = acc + __shfl_xor(acc, m);
    if (lane == 0) sm.red[wave] = acc;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (lane == 0) lds_add(&sm.aux_cnt, 1);
    if (wave == 0) {
      lds_wait_ge(a, &sm.aux_cnt, 2 * kAuxWaves);
      if (lane == 0) {
        put_tag(a.scores + c, a.epoch,
                __float_as_uint(sigmoid_det((sm.red[0] + sm.red[1]) + (sm.red[2] + sm.red[3]))));
        // the router's ring slots are free: counted as if delivered by the
        // producers and read by the consumers
        for (int i = 0; i < kRtChunks; ++i) {
          lds_add(&sm.land[i], kProdWaves);
          lds_add(&sm.rel[i], kConsWaves);
        }
      }
    }
  }

  // ---- digits of h_post (7 groups per wave; wave 15 also wave 0's) ----
  if (wave) {
#pragma unroll
    for (int i = 0; i < kHidden / 64 / 16; ++i) digits_to(hd[i], sm.xs[7 * wave + i], lane);
  }
  if (wave == 15) {
#pragma unroll
    for (int i = 0; i < kHidden / 64 / 16; ++i) digits_to(hd0[i], sm.xs[i], lane);
  }

  // ---- scores -> the expert set (aux wave 0) ----
  float sc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, bj[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  int vk[4] = {0, 0, 0, 0};
  if (wave == 0) {
    poll_waves(a, [&] {
      bool ok = true;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint64_t v = get_tag(a.scores + 64 * j + lane);
        ok = ok && tag_ok(v, a.epoch);
        sc[j] = __uint_as_float((uint32_t)v);
      }
      return ok;
    });
#pragma unroll
    for (int j = 0; j < 4; ++j) bj[j] = a.bias ? a.bias[64 * j + lane] : 0.0f;
    route_keys(sc, bj, vk);
    int id = 0;
    if (!topk_set(vk, a.K, id)) {
      float wv;
      slot_scan(vk, sc, a.K, 2.5f, id, wv);
    }
    if (lane < a.K) sm.eid[lane] = id;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      sm.rs.key[64 * j + lane] = vk[j];
      sm.rs.sc[64 * j + lane] = sc[j];
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (lane == 0) lds_store(&sm.route_ready, 1);
  }
  bar();  // h_post digits complete (and the route known)

  // ---- the stream ----
  if (prod_w) {
    // routed chunks the prologue could not issue (slots 1-3 without a shared expert)
    for (int q = kRtChunks; q < min(P.total, kRingSlots); ++q)
      if (q >= P.gu0) issue_chunk(chunk_of(a, P, sm, c, q, Q6), lds_addr(ring[0]) + q * kChunk, wave);
    producer<Q6>(a, P, sm, ring[0], c, wave);
  } else if (cons_w) {
    consumer<Q6>(a, P, sm, ring[0], c, wave - kCons0, lane);
  } else {
    aux<Q6>(a, P, sm, c, t, wave, lane, sc, vk);
  }
  bar();

  // ---- combine rows 28c .. 28c+27 (the reference's slot order) ----
  if (t < kDnRows) {
    const int r = c * kDnRows + t;
    float moe = 0.0f;
    for (int k = 0; k < a.K; ++k) moe = fmaf(sm.wk[k], sm.eo[sm.perm[k]][t], moe);
    const float sd = a.n_slots > a.K ? sm.eo[a.K][t] : 0.0f;
    const float hin = a.h_in ? a.h_in[r] : 0.0f;
    a.out[r] = (hin + moe) + sd;
    if (a.moe_out) a.moe_out[r] = moe;
  }
}

__global__ __launch_bounds__(kThreads) void k_stream_q4k(LayerArgs a) { stream_layer<false>(a); }
__global__ __launch_bounds__(kThreads) void k_stream_q6k(LayerArgs a) { stream_layer<true>(a); }

}  // namespace

int stream_layer_workgroups() { return kSWg; }

hipError_t launch_stream_layer(const LayerArgs& a, hipStream_t s) {
  if (a.down_q6)
    hipLaunchKernelGGL(k_stream_q6k, dim3(kSWg), dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL(k_stream_q4k, dim3(kSWg), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace fdm
