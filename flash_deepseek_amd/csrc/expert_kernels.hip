// expert_kernels.hip -- one SwiGLU expert at batch 1 with a Q4_K down matrix
// (fdm_expert_ffn): encode_expert (infer.m:1559-1575) on the caller's packed
// blob, out = down . (silu(gate . x) * (up . x)), in ONE launch and in fp32.
//
// Work list of 256-thread workgroups:
//   gate/up items (512): gate rows 4i .. 4i+3 and up rows 4i .. 4i+3; each
//     stages x in LDS (padded, with its sub-block sums), contracts its eight
//     rows (32 lanes per row, one wave per two rows), applies SwiGLU to the
//     four row pairs and publishes the four activations as tagged words
//   final items (224): down rows 32f .. 32f+31; each requests its weights at
//     dispatch, waits for the 2048 tagged activations, stages them in LDS and
//     contracts its rows (32 lanes per row)
// At batch 1 the expert is latency-bound (25 MB stream in ~4 us): fp32 needs
// no digit records of x or of the activations, so the chain is x and
// weights -> gate/up -> one hand-off -> down.  Every dot is the fp32 group
// dot of q4k_group_dot_f32 (dequant_matvec_q4k's arithmetic,
// shaders.metal:43-99).
//
// Final items only wait for gate/up items, which come first in the list and
// never wait: the grid drains whatever the dispatch order.  The wait is
// bounded: one that gives up records the call's epoch in the error flag
// (fdm_stream_sync reports it) and releases every other wait.
#include "fdm_internal.h"

namespace fdm {

namespace {

constexpr int kExGuRows = 4;                    // gate rows (and up rows) per gate/up item
constexpr int kExGuItems = kFfn / kExGuRows;    // 512
constexpr int kExFinRows = 32;                  // down rows per final item
constexpr int kExFinItems = kHidden / kExFinRows;  // 224
constexpr int kExXGroups = kHidden / 64;        // 112

struct ExpertSmem {
  float x[kExXGroups * kXPad];  // x (gate/up items) or the activations (final items), padded
  float xs[2 * kExXGroups];     // their 32-element sub-block sums
  float row[2 * kExGuRows];     // gate/up item: gate row sums, then up row sums
};

// Sum of v over each 32-lane half of the wave into its first lane (lanes 0
// and 32): rows 1 and 3 of 16 lanes into rows 0 and 2 by permlane16_swap,
// then the DPP row sum.
__device__ __forceinline__ float sum32_first(float v) {
  v = v + __uint_as_float(__builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false)[1]);
  return sum16(v);
}

// Whole-workgroup bounded wait: every thread runs try_once() until all of
// them succeed; gives up after spin_limit rounds, or when another
// workgroup already gave up (looked at every 64th round), recording the
// epoch in the error flag.
template <typename F>
__device__ __forceinline__ bool ex_poll(const LayerArgs& a, F&& try_once) {
  unsigned* err = a.flags + kLayerStride * kLayerFlagErr;
  for (unsigned n = 0;; ++n) {
    if (__syncthreads_and(try_once())) return true;
    int give_up = 0;
    if (threadIdx.x == 0) give_up = n >= a.spin_limit || ((n & 63) == 63 && load_u32_agent(err) == a.epoch);
    if (__syncthreads_or(give_up)) {
      if (threadIdx.x == 0) store_u32_agent(err, a.epoch);
      return false;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

__device__ __forceinline__ void ex_gateup_item(const LayerArgs& a, int item, ExpertSmem& sm) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 31;                    // lane of the row: groups li, li + 32, ...
  const int rw = 2 * (wave & 1) + (lane >> 5);  // row of the item (0-3)
  const int row = kExGuRows * item + rw;
  const uint8_t* mat = a.shared + (wave >= 2 ? kGateBytes : 0);
  // x first (its LDS copy waits for these loads only), then the weights
  constexpr int kNv = kHidden / 4 / 256;  // float4s of x per thread (7)
  f32x4 xv[kNv];
#pragma unroll
  for (int i = 0; i < kNv; ++i) xv[i] = reinterpret_cast<const f32x4*>(a.h)[threadIdx.x + 256 * i];
  Q4KGroupLoad ld[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int G = min(li + 32 * k, kExXGroups - 1);  // groups past the row: a valid one, contributing 0
    ld[k] = q4k_load_group(mat + ((size_t)row * (kHidden / kQK) + (G >> 2)) * kQ4KBlock, li & 3);
  }
  // x into LDS; each sub-block's sum by the eight threads that hold it
#pragma unroll
  for (int i = 0; i < kNv; ++i) {
    const int v = threadIdx.x + 256 * i;
    *reinterpret_cast<f32x4*>(sm.x + kXPad * (v >> 4) + 4 * (v & 15)) = xv[i];
    float sb = (xv[i].x + xv[i].y) + (xv[i].z + xv[i].w);
    sb = sb + dpp_row_shl<1>(sb);
    sb = sb + dpp_row_shl<2>(sb);
    sb = sb + dpp_row_shl<4>(sb);
    if ((v & 7) == 0) sm.xs[v >> 3] = sb;
  }
  __syncthreads();
  const float qscale = q4k_fp8_qscale();
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int G = li + 32 * k, Gc = min(G, kExXGroups - 1);
    const float part = q4k_group_dot_f32(ld[k], q4k_quad_hdr(ld[k]), li & 3, sm.x + kXPad * Gc, sm.xs[2 * Gc],
                                         sm.xs[2 * Gc + 1], qscale);
    acc += G < kExXGroups ? part : 0.0f;
  }
  acc = sum32_first(acc);
  if (li == 0) sm.row[(wave >= 2 ? kExGuRows : 0) + rw] = acc;
  __syncthreads();
  if (threadIdx.x < kExGuRows) {
    const float av = silu_mul(sm.row[threadIdx.x], sm.row[kExGuRows + threadIdx.x]);
    const int r = kExGuRows * item + threadIdx.x;
    put_tagged(a.act + r, a.epoch, __float_as_uint(av));
    if (a.act_out) a.act_out[r] = av;
  }
}

__device__ __forceinline__ void ex_final_item(const LayerArgs& a, int item, ExpertSmem& sm) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = lane & 31;  // the lane's group of its rows
  const uint8_t* down = a.shared + 2 * (size_t)kGateBytes;
  // the weights of the lane's four rows (8 k + 2 wave + lane / 32), at dispatch
  Q4KGroupLoad ld[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int row = kExFinRows * item + 8 * k + 2 * wave + (lane >> 5);
    ld[k] = q4k_load_group(down + ((size_t)row * (kFfn / kQK) + (G >> 2)) * kQ4KBlock, G & 3);
  }
  // the 2048 activations (eight per thread): after the first round finds
  // them incomplete, thread 0 watches the last one before every thread
  // loads all again (a waiting item does not reload 16 KB per round)
  constexpr int kPer = kFfn / 256;
  float v[kPer];
  auto full = [&] {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const uint64_t t = get_tagged(a.act + threadIdx.x + 256 * j);
      ok = ok && tag_is(t, a.epoch);
      v[j] = tagged_f(t);
    }
    return ok;
  };
  for (;;) {
    if (__syncthreads_and(full())) break;
    const bool ok = ex_poll(a, [&] {
      return threadIdx.x != 0 || tag_is(get_tagged(a.act + kFfn - 1), a.epoch);
    });
    if (!ok) break;  // gave up: the error flag is set
  }
  // element 256 j + 64 w + lane: group 4 j + w; each half wave one sub-block
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = threadIdx.x + 256 * j;
    sm.x[kXPad * (e >> 6) + (e & 63)] = v[j];
    const float hs = half_reduce<false>(v[j]);
    if ((lane & 31) == 0) sm.xs[e >> 5] = hs;
  }
  __syncthreads();
  const float qscale = q4k_fp8_qscale();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float acc = q4k_group_dot_f32(ld[k], q4k_quad_hdr(ld[k]), G & 3, sm.x + kXPad * G, sm.xs[2 * G],
                                  sm.xs[2 * G + 1], qscale);
    acc = sum32_first(acc);
    if (G == 0) a.out[kExFinRows * item + 8 * k + 2 * wave + (lane >> 5)] = acc;
  }
}

}  // namespace

__global__ __launch_bounds__(256) void k_expert_f32_q4k(LayerArgs a) {
  __shared__ ExpertSmem sm;
  if ((int)blockIdx.x < kExGuItems)
    ex_gateup_item(a, blockIdx.x, sm);
  else
    ex_final_item(a, blockIdx.x - kExGuItems, sm);
}

hipError_t launch_expert_f32(const LayerArgs& a, hipStream_t s) {
  if (a.down_q6) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_expert_f32_q4k, dim3(kExGuItems + kExFinItems), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace fdm
