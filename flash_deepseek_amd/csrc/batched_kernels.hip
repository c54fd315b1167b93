// batched_kernels.hip -- batched decode through one MoE layer: T tokens per
// step with token -> expert dispatch, so each selected expert's weights are
// read from HBM once per step however many tokens chose it.
//
// The reference decodes one token at a time (infer.m:2219-2229); per token
// the result is the MoE branch of layer_forward (infer.m:1878-1922), and
// routing (route(), infer.m:920-991) is exactly the per-token one.
//
//   k_router_logits / k_route   per token (router_kernels.hip)
//   k_dispatch                  group the T*K (token, slot) pairs by expert
//   k_xdigits                   digits of the T tokens
// Experts are read in the resident expert layout (rel_load_group).
//
//   k_bgateup                   per (distinct expert or shared, 8-row tile): the
//                               weight tile stays in registers while the
//                               expert's tokens stream through LDS
//   k_xdigits                   digits of every pair's activations
//   k_bdown                     per (expert, 16-row tile), as k_bgateup
//   k_bcombine                  per token: h_in + sum_k w_k E_k + shared
#include "fdm_internal.h"

namespace fdm {

namespace {

constexpr int kExperts = 256;                 // R1 routed experts
constexpr int kBGuRows = 8;                   // gate (and up) rows per tile
constexpr int kBGuTiles = kFfn / kBGuRows;    // 256
constexpr int kBDnRows = 16;                  // down rows per tile
constexpr int kBDnTiles = kHidden / kBDnRows; // 448
constexpr int kBShChunk = 16;                 // shared-expert tokens per work item

// Token t's row list of one work item: a distinct routed expert (its
// (token, slot) pairs, rows = pair positions) or one chunk of kBShChunk
// tokens of the shared expert (rows = P + t).
struct ItemRows {
  int first, count;  // pair positions [first, first + count) or tokens [0, count)
  bool shared;
};

__device__ __forceinline__ ItemRows item_rows(const BatchArgs& b, int d, int D, int* expert) {
  ItemRows r;
  if (d < D) {
    const int e = b.distinct[d];
    *expert = e;
    r.first = b.seg_start[e];
    r.count = b.seg_start[e + 1] - r.first;
    r.shared = false;
  } else {
    *expert = -1;
    r.first = (d - D) * kBShChunk;
    r.count = min(kBShChunk, b.T - r.first);
    r.shared = true;
  }
  return r;
}

__device__ __forceinline__ int n_items_of(const BatchArgs& b, int D) {
  return D + (b.shared ? (b.T + kBShChunk - 1) / kBShChunk : 0);
}

// One token's digit records (N records of 13 x 16 bytes) held in registers,
// 16 bytes per thread per step: loaded while the previous token is being
// contracted, stored to LDS after it.
template <int N>
struct Records {
  static constexpr int kSteps = (N * kXGroupVec + 255) / 256;
  u32x4 v[kSteps];
  __device__ __forceinline__ void load(const XGroup* __restrict__ src) {
    const u32x4* s = reinterpret_cast<const u32x4*>(src);
#pragma unroll
    for (int k = 0; k < kSteps; ++k) {
      const int i = threadIdx.x + 256 * k;
      if (i < N * kXGroupVec) v[k] = s[i];
    }
  }
  __device__ __forceinline__ void store(XGroup* __restrict__ dst) const {
    u32x4* d = reinterpret_cast<u32x4*>(dst);
#pragma unroll
    for (int k = 0; k < kSteps; ++k) {
      const int i = threadIdx.x + 256 * k;
      if (i < N * kXGroupVec) d[i] = v[k];
    }
  }
};

}  // namespace

// ---- dispatch -------------------------------------------------------------------------
// Exclusive prefix sum of v over the 256 threads of the workgroup; tot
// receives the total in every thread.
__device__ __forceinline__ int block_scan_excl(int v, int* wsum, int& tot) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) wsum[wave] = x;
  __syncthreads();
  int base = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) base += w < wave ? wsum[w] : 0;
  tot = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
  __syncthreads();  // wsum may be reused
  return base + x - v;
}

// One workgroup, thread e = expert e: pair counts per expert, segment
// starts, the ascending list of distinct experts, each pair's position in
// its expert's segment and, with b.ch > 0, the grouped GEMMs' chunk list
// (every distinct expert's segment in chunks of b.ch pairs, ascending, then
// the shared expert's tokens in chunks of b.ch), all by block-wide scans.
// The order of pairs inside a segment (LDS atomics) does not affect any
// result: every pair's activations and output come from its own token only.
// The first 256 kDispHeld pairs are loaded once, all at a time, and held in
// registers for both passes (their loads no longer wait one by one).
constexpr int kDispHeld = 16;
__global__ __launch_bounds__(256) void k_dispatch(BatchArgs b) {
  __shared__ int cnt[kExperts];
  __shared__ int fill[kExperts];
  __shared__ int start[kExperts];
  __shared__ int wsum[4];
  const int P = b.T * b.K;
  const int e = threadIdx.x;
  cnt[e] = 0;
  fill[e] = 0;
  int held[kDispHeld];
#pragma unroll
  for (int i = 0; i < kDispHeld; ++i) {
    const int p = threadIdx.x + 256 * i;
    held[i] = p < P ? b.idx[p] : -1;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kDispHeld; ++i)
    if (held[i] >= 0 && held[i] < kExperts) atomicAdd(&cnt[held[i]], 1);
  for (int p = threadIdx.x + 256 * kDispHeld; p < P; p += 256) {
    const int x = b.idx[p];
    if (x >= 0 && x < kExperts) atomicAdd(&cnt[x], 1);
  }
  __syncthreads();
  const int c = cnt[e];
  int tot, nd;
  const int st = block_scan_excl(c, wsum, tot);
  const int dpos = block_scan_excl(c > 0 ? 1 : 0, wsum, nd);
  start[e] = st;
  b.seg_start[e] = st;
  if (c > 0) b.distinct[dpos] = e;
  if (e == 0) {
    b.seg_start[kExperts] = tot;
    *b.n_distinct = nd;
  }
  if (b.ch > 0) {
    const int ch = b.ch;
    const int nch = (c + ch - 1) / ch;
    int nr;
    const int cpos = block_scan_excl(nch, wsum, nr);
    for (int q = 0; q < nch; ++q)
      b.chunks[cpos + q] = make_int4(e, st + q * ch, min(ch, c - q * ch), cpos | (nch << 16));
    const int ns = b.shared ? (b.T + ch - 1) / ch : 0;
    for (int q = threadIdx.x; q < ns; q += 256)
      b.chunks[nr + q] = make_int4(-1, q * ch, min(ch, b.T - q * ch), nr | (ns << 16));
    if (e == 0) *b.n_chunks = nr + ns;
  }
  __syncthreads();
  auto place = [&](int p, int x) {
    int pos = -1;
    if (x >= 0 && x < kExperts) {
      pos = start[x] + atomicAdd(&fill[x], 1);
      b.pair_tok[pos] = p / b.K;
    }
    b.pair_of[p] = pos;  // -1: invalid expert id, contributes 0
  };
#pragma unroll
  for (int i = 0; i < kDispHeld; ++i) {
    const int p = threadIdx.x + 256 * i;
    if (p < P) place(p, held[i]);
  }
  for (int p = threadIdx.x + 256 * kDispHeld; p < P; p += 256) place(p, b.idx[p]);
}

// ---- grouped gate/up ----------------------------------------------------------------------
// Work item (tile, d): d < D is the d-th distinct expert, d == D the shared
// expert; workgroups stride over d.  Wave w owns rows 2w, 2w+1 of the tile
// in gate (lanes 0-31) and up (lanes 32-63), 16 lanes per row; the tile's
// weights are loaded once and every token of the item is applied to them.
__global__ __launch_bounds__(256) void k_bgateup(BatchArgs b) {
  __shared__ XGroup xs[2][kHidden / 64];
  const int tile = blockIdx.x;
  const int D = *b.n_distinct;
  const int n_items = n_items_of(b, D);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane >> 4, l16 = lane & 15, g = l16 & 3;
  const int row = tile * kBGuRows + 2 * wave + (q & 1);
  const Q4KScaleSel sel = q4k_scale_sel(g);
  const int P = b.T * b.K;
  for (int d = blockIdx.y; d < n_items; d += gridDim.y) {
    int e;
    const ItemRows r = item_rows(b, d, D, &e);
    const uint8_t* blob = r.shared ? b.shared : b.experts + (size_t)e * b.expert_size;
    Q4KGroupLoad ld[7];
    const uint8_t* mat = blob + (q >= 2 ? kGateBytes : 0);
#pragma unroll
    for (int i = 0; i < 7; ++i) ld[i] = rel_load_group<false>(mat, row, 4 * i + (l16 >> 2), g);
    auto tok_of = [&](int i) { return r.shared ? r.first + i : b.pair_tok[r.first + i]; };
    Records<kHidden / 64> rec;
    rec.load(b.xd + (size_t)tok_of(0) * (kHidden / 64));
    __syncthreads();  // the previous item's last records are no longer read
    rec.store(xs[0]);
    __syncthreads();
    for (int i = 0; i < r.count; ++i) {
      const int out_row = r.shared ? P + r.first + i : r.first + i;
      const XGroup* cur = xs[i & 1];
      if (i + 1 < r.count) rec.load(b.xd + (size_t)tok_of(i + 1) * (kHidden / 64));
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < 7; ++k) {
        // the weights look changed to the compiler on every token, so their
        // unpacking stays inside this loop instead of being hoisted out of
        // it (seven unpacked groups would take 112 more registers)
        __asm__ volatile("" : "+v"(ld[k].q0), "+v"(ld[k].q1), "+v"(ld[k].hdr_part));
        acc += q4k_group_dot_ld(ld[k], sel, &cur[16 * k + l16]);
        __builtin_amdgcn_sched_barrier(0);
      }
      acc = sum16(acc);
      const float up = __shfl(acc, (lane + 32) & 63);
      if (lane == 0 || lane == 16) b.act[(size_t)out_row * kFfn + row] = silu_mul(acc, up);
      // the other buffer was last read before the barrier that ended token i - 1
      if (i + 1 < r.count) rec.store(xs[(i + 1) & 1]);
      __syncthreads();
    }
  }
}

// ---- grouped down -------------------------------------------------------------------------
// Work item (tile, d) as k_bgateup: 16 down rows (wave w: rows 4w..4w+3, 16
// lanes per row) of one expert, applied to the activation digits of every
// row of the item.
template <bool Q6>
__global__ __launch_bounds__(256) void k_bdown(BatchArgs b) {
  __shared__ XGroup xs[2][kFfn / 64];
  const int tile = blockIdx.x;
  const int D = *b.n_distinct;
  const int n_items = n_items_of(b, D);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15;
  // Q4_K: 16 lanes per row (lane / 16); Q6_K resident layout: lane (half h =
  // bit 0, row r = bits 1-2, block b = bits 3-4 of column part pt = bit 5),
  // so a wave's load reads 32 consecutive pieces of each part
  const int h6 = lane & 1, r6 = (lane >> 1) & 3, b6 = (lane >> 3) & 3, p6 = lane >> 5;
  const int H6 = 8 * p6 + 2 * b6 + h6;
  const int row = tile * kBDnRows + wave * 4 + (Q6 ? r6 : lane >> 4);
  const bool writer = Q6 ? (lane & 0x39) == 0 : l16 == 0;
  const int P = b.T * b.K;
  for (int d = blockIdx.y; d < n_items; d += gridDim.y) {
    int e;
    const ItemRows r = item_rows(b, d, D, &e);
    const uint8_t* blob = r.shared ? b.shared : b.experts + (size_t)e * b.expert_size;
    const uint8_t* dbase = blob + 2 * (size_t)kGateBytes;
    Q4KGroupLoad ld[2];
    Q6KHalfW l6;
    if (!Q6) {
#pragma unroll
      for (int i = 0; i < 2; ++i) ld[i] = rel_load_group<true>(dbase, row, 4 * i + (l16 >> 2), l16 & 3);
    } else {
      l6 = q6k_rel_load_half(dbase, row, 4 * p6 + b6, h6);
    }
    auto row_of = [&](int i) { return r.shared ? P + r.first + i : r.first + i; };
    Records<kFfn / 64> rec;
    rec.load(b.act_xd + (size_t)row_of(0) * (kFfn / 64));
    __syncthreads();
    rec.store(xs[0]);
    __syncthreads();
    for (int i = 0; i < r.count; ++i) {
      const int arow = row_of(i);
      const XGroup* cur = xs[i & 1];
      if (i + 1 < r.count) rec.load(b.act_xd + (size_t)row_of(i + 1) * (kFfn / 64));
      float acc = 0.0f;
      if (!Q6) {
        const Q4KScaleSel sel = q4k_scale_sel(l16 & 3);
#pragma unroll
        for (int k = 0; k < 2; ++k) acc += q4k_group_dot_ld(ld[k], sel, &cur[16 * k + l16]);
      } else {
        acc = q6k_half_dot_w(l6, &cur[2 * H6]);
      }
      if (!Q6) {
        acc = sum16(acc);
      } else {
        // H6 bits 3, 2, 1, 0 are lane bits 5, 4, 3, 0: the xor butterfly over
        // 8, 4, 2, 1, which gives lane H6 = 0 what sum16 gives its first lane
        acc += __shfl_xor(acc, 32);
        acc += __shfl_xor(acc, 16);
        acc += __shfl_xor(acc, 8);
        acc += __shfl_xor(acc, 1);
      }
      if (writer) b.eo[(size_t)arow * kHidden + row] = acc;
      if (i + 1 < r.count) rec.store(xs[(i + 1) & 1]);
      __syncthreads();
    }
  }
}

// ---- combine ------------------------------------------------------------------------------
// hidden[t] = (h_in[t] + sum_k w[t][k] E_{idx[t][k]}) + S[t], slots in route()
// order (infer.m:1689-1695, 1922).  out may alias h_in (each element is read
// before it is written, by the same thread).
// V consecutive outputs per thread (V = 4 when h_in and out are 16-byte
// aligned: every load and store a 16-byte vector), each the same chain
// (h_in + sum_k w_k E_k) + S in slot order.
template <int V>
__global__ __launch_bounds__(256) void k_bcombine(BatchArgs b) {
  typedef float vf __attribute__((ext_vector_type(V)));
  const int t = blockIdx.y;
  const int r = (blockIdx.x * 256 + threadIdx.x) * V;
  if (r >= kHidden) return;
  const int P = b.T * b.K;
  vf moe = (vf)0.0f;
  for (int k = 0; k < b.K; ++k) {
    const int pos = b.pair_of[t * b.K + k];
    const vf ev = pos >= 0 ? *reinterpret_cast<const vf*>(b.eo + (size_t)pos * kHidden + r) : (vf)0.0f;
    const float wk = b.w[t * b.K + k];
#pragma unroll
    for (int i = 0; i < V; ++i) moe[i] = fmaf(wk, ev[i], moe[i]);
  }
  const vf sd = b.shared ? *reinterpret_cast<const vf*>(b.eo + (size_t)(P + t) * kHidden + r) : (vf)0.0f;
  const vf hin = b.h_in ? *reinterpret_cast<const vf*>(b.h_in + (size_t)t * kHidden + r) : (vf)0.0f;
  vf o;
#pragma unroll
  for (int i = 0; i < V; ++i) o[i] = (hin[i] + moe[i]) + sd[i];
  *reinterpret_cast<vf*>(b.out + (size_t)t * kHidden + r) = o;
}

hipError_t launch_dispatch(const BatchArgs& b, hipStream_t s) {
  hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(256), 0, s, b);
  return hipGetLastError();
}

hipError_t launch_combine(const BatchArgs& b, hipStream_t s) {
  const bool vec = (reinterpret_cast<uintptr_t>(b.out) & 15) == 0 && (reinterpret_cast<uintptr_t>(b.h_in) & 15) == 0;
  if (vec)
    hipLaunchKernelGGL(k_bcombine<4>, dim3(kHidden / 1024, b.T), dim3(256), 0, s, b);
  else
    hipLaunchKernelGGL(k_bcombine<1>, dim3(kHidden / 256, b.T), dim3(256), 0, s, b);
  return hipGetLastError();
}

hipError_t launch_batched_down(const BatchArgs& b, bool down_q6, hipStream_t s) {
  const int P = b.T * b.K;
  const int rows = P + (b.shared ? b.T : 0);
  const int max_items = (P < kExperts ? P : kExperts) + (b.shared ? (b.T + kBShChunk - 1) / kBShChunk : 0);
  const int gy = max_items < 16 ? max_items : 16;
  if (hipError_t e = launch_xdigits(b.act, (size_t)rows * (kFfn / 64), b.act_xd, s)) return e;
  if (down_q6)
    hipLaunchKernelGGL(k_bdown<true>, dim3(kBDnTiles, gy), dim3(256), 0, s, b);
  else
    hipLaunchKernelGGL(k_bdown<false>, dim3(kBDnTiles, gy), dim3(256), 0, s, b);
  return hipGetLastError();
}

hipError_t launch_batched_experts(const BatchArgs& b, bool down_q6, hipStream_t s) {
  const int P = b.T * b.K;
  const int rows = P + (b.shared ? b.T : 0);
  const int max_items = (P < kExperts ? P : kExperts) + (b.shared ? (b.T + kBShChunk - 1) / kBShChunk : 0);
  // workgroups per tile: enough items in flight to fill the chip
  const int gy = max_items < 16 ? max_items : 16;
  hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(256), 0, s, b);
  if (hipError_t e = hipGetLastError()) return e;
  if (hipError_t e = launch_xdigits(b.x, (size_t)b.T * (kHidden / 64), b.xd, s)) return e;
  hipLaunchKernelGGL(k_bgateup, dim3(kBGuTiles, gy), dim3(256), 0, s, b);
  if (hipError_t e = hipGetLastError()) return e;
  if (hipError_t e = launch_xdigits(b.act, (size_t)rows * (kFfn / 64), b.act_xd, s)) return e;
  if (down_q6)
    hipLaunchKernelGGL(k_bdown<true>, dim3(kBDnTiles, gy), dim3(256), 0, s, b);
  else
    hipLaunchKernelGGL(k_bdown<false>, dim3(kBDnTiles, gy), dim3(256), 0, s, b);
  if (hipError_t e = hipGetLastError()) return e;
  return launch_combine(b, s);
}

}  // namespace fdm
