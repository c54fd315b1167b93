// moe_kernels.hip -- the expert FFN of the MoE layer for all selected
// experts at once (infer.m:1559-1575 encode_expert, run for every slot, and
// the combine of infer.m:1689-1695 / 1922).
//
// Both kernels are shaped for memory-level parallelism: many small
// workgroups, each issuing every weight load it needs before any math, so
// that the HBM queue stays full (one 16-byte load per lane per step; the
// four lanes of a Q4_K block share its header through DPP).
//
// k_gateup  one workgroup per (slot, 8-row tile).  Wave w owns rows 2w and
//   2w+1 of the tile in BOTH gate and up (lanes 0-31 gate, 32-63 up, 16
//   lanes per row), so SwiGLU (swiglu_fused, shaders.metal:210-220) is
//   applied in registers.  The last of the four tiles of a 32-row sub-block
//   to finish turns the sub-block's activations into the digits the down
//   matvec reads (a per-sub-block arrival counter).
// k_down    one workgroup per (slot, 16-row tile): the slot's down rows.
//   The last of the slots of a row tile to finish (in this launch or an
//   earlier one of the same call: streamed layers launch slot by slot)
//   combines them in slot order, then adds the shared expert and the residual
//   (moe_out += w_k * E_k, infer.m:1690-1695; hidden = h_in + moe_out + sd,
//   infer.m:1922).
#include "fdm_internal.h"

namespace fdm {

__device__ __forceinline__ const uint8_t* slot_blob(const SlotTable& t, int slot) {
  if (slot < t.K) {
    const int e = t.idx[slot];
    if (e < 0 || e >= t.n_experts) return nullptr;  // invalid id: expert contributes 0
    return t.experts + (size_t)e * t.expert_size;
  }
  return t.shared;
}

constexpr int kGuRows = 8;                 // rows of gate (and up) per workgroup
constexpr int kGuTiles = kFfn / kGuRows;   // 256 tiles per slot

__global__ __launch_bounds__(256) void k_gateup(SlotTable t, const XGroup* __restrict__ xd,
                                                float* __restrict__ act,
                                                XGroup* __restrict__ act_xd,
                                                int* __restrict__ counters) {
  __shared__ XGroup xs[kHidden / 64];
  __shared__ int last;
  const int slot = t.slot0 + blockIdx.x / kGuTiles, tile = blockIdx.x % kGuTiles;
  if ((t.skip >> slot) & 1u) return;  // another launch of the call runs this slot
  const uint8_t* blob = slot_blob(t, slot);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane >> 4, l16 = lane & 15, g = l16 & 3;
  const int row = tile * kGuRows + 2 * wave + (q & 1);
  // the digit records first, then the weights: the records land first and
  // each weight group is used as soon as it arrives
  XStage<kHidden / 64> st;
  st.load(xd, kHidden / 64);
  Q4KGroupLoad ld[7];
  if (blob) {
    const uint8_t* mat = blob + (q >= 2 ? kGateBytes : 0);
    const uint8_t* rowp = mat + (size_t)row * kQ4KRowHidden;
#pragma unroll
    for (int i = 0; i < 7; ++i)
      ld[i] = t.rel ? rel_load_group<false>(mat, row, 4 * i + (l16 >> 2), g)
                    : q4k_load_group(rowp + (4 * i + (l16 >> 2)) * kQ4KBlock, g);
  }
  st.store(xs, kHidden / 64);
  __syncthreads();
  float acc = 0.0f;
  if (blob) {
    const Q4KScaleSel sel = q4k_scale_sel(g);
#pragma unroll
    for (int i = 0; i < 7; ++i) {
      acc += q4k_group_dot_ld(ld[i], sel, &xs[16 * i + l16]);
      __builtin_amdgcn_sched_barrier(0);  // one group's LDS reads at a time
    }
  }
  acc = sum16(acc);
  const float up = __shfl(acc, (lane + 32) & 63);
  if (lane == 0 || lane == 16) {
    store_agent(act + (size_t)slot * kFfn + row, silu_mul(acc, up));
    wait_stores_done();
  }
  __syncthreads();
  int* cnt = counters + slot * (kFfn / 32) + (tile >> 2);
  if (threadIdx.x == 0) last = (arrive_agent(cnt) == 3);
  __syncthreads();
  if (last) {
    if (threadIdx.x < 32) {
      const int base = (tile >> 2) * 32;
      const float v = load_agent(act + (size_t)slot * kFfn + base + threadIdx.x);
      int8_t a, b, c;
      float s, sum;
      make_digits3(v, a, b, c, s, sum);
      XGroup* xg = act_xd + (size_t)slot * (kFfn / 64) + (tile >> 3);
      const int half = (tile >> 2) & 1;
      xg->a[32 * half + threadIdx.x] = a;
      xg->b[32 * half + threadIdx.x] = b;
      xg->c[32 * half + threadIdx.x] = c;
      if (threadIdx.x == 0) {
        xg->s[half] = s;
        xg->xsum[half] = sum;
        reset_agent(cnt);
      }
    }
  }
}

constexpr int kDnRows = 16;                   // down rows per workgroup
constexpr int kDnTiles = kHidden / kDnRows;   // 448

template <bool Q6>
__global__ __launch_bounds__(256) void k_down(SlotTable t, const XGroup* __restrict__ act_xd,
                                              const float* __restrict__ h_in,
                                              float* __restrict__ out,
                                              float* __restrict__ moe_out,
                                              float* __restrict__ eo,
                                              int* __restrict__ counters) {
  __shared__ XGroup xs[kFfn / 64];
  __shared__ int last;
  const int slot = t.slot0 + (int)blockIdx.y, tile = blockIdx.x;
  if ((t.skip >> slot) & 1u) return;  // another launch of the call runs this slot
  const uint8_t* blob = slot_blob(t, slot);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15;
  // Q4_K: 16 lanes per row (lane / 16); Q6_K: lane (half h = bit 0, row r =
  // bits 1-2, block b = bits 3-4 of column part pt = bit 5), the mapping of
  // the Q6_K resident layout (a wave's load reads 32 consecutive pieces of
  // each part), also used on packed blobs
  const int h6 = lane & 1, r6 = (lane >> 1) & 3, b6 = (lane >> 3) & 3, p6 = lane >> 5;
  const int H6 = 8 * p6 + 2 * b6 + h6;
  const int row = tile * kDnRows + wave * 4 + (Q6 ? r6 : lane >> 4);
  const bool writer = Q6 ? (lane & 0x39) == 0 : l16 == 0;
  float acc = 0.0f;
  XStage<kFfn / 64> st;
  st.load(act_xd + (size_t)slot * (kFfn / 64), kFfn / 64);
  if (!Q6) {
    Q4KGroupLoad ld[2];
    if (blob) {
      const uint8_t* mat = blob + 2 * (size_t)kGateBytes;
      const uint8_t* rowp = mat + (size_t)row * kQ4KRowFfn;
#pragma unroll
      for (int i = 0; i < 2; ++i)
        ld[i] = t.rel ? rel_load_group<true>(mat, row, 4 * i + (l16 >> 2), l16 & 3)
                      : q4k_load_group(rowp + (4 * i + (l16 >> 2)) * kQ4KBlock, l16 & 3);
    }
    st.store(xs, kFfn / 64);
    __syncthreads();
    if (blob) {
      const Q4KScaleSel sel = q4k_scale_sel(l16 & 3);
#pragma unroll
      for (int i = 0; i < 2; ++i) acc += q4k_group_dot_ld(ld[i], sel, &xs[16 * i + l16]);
    }
  } else {
    // 16 halves of 128 elements per 2048-column row: one per lane
    const uint8_t* mat = blob ? blob + 2 * (size_t)kGateBytes : nullptr;
    Q6KHalfW lw;
    Q6KHalfLoad lp;
    if (blob) {
      if (t.rel)
        lw = q6k_rel_load_half(mat, row, 4 * p6 + b6, h6);
      else
        lp = q6k_load_half(mat + (size_t)row * kQ6KRowFfn + (H6 >> 1) * kQ6KBlock, h6);
    }
    st.store(xs, kFfn / 64);
    __syncthreads();
    if (blob) acc = t.rel ? q6k_half_dot_w(lw, &xs[2 * H6]) : q6k_half_dot_ld(lp, &xs[2 * H6]);
  }
  if (!Q6) {
    acc = sum16(acc);
  } else {
    // H6 bits 3, 2, 1, 0 are lane bits 5, 4, 3, 0: the xor butterfly over 8,
    // 4, 2, 1, which gives lane H6 = 0 what sum16 gives its first lane
    acc += __shfl_xor(acc, 32);
    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 8);
    acc += __shfl_xor(acc, 1);
  }
  if (writer) {
    store_agent(eo + (size_t)slot * kHidden + row, acc);
    wait_stores_done();
  }
  __syncthreads();
  if (threadIdx.x == 0) last = (arrive_agent(counters + tile) == t.n_slots - 1);
  __syncthreads();
  if (last) {
    if (threadIdx.x < kDnRows) {
      const int r = tile * kDnRows + threadIdx.x;
      float moe = 0.0f;
      for (int k = 0; k < t.K; ++k) moe = fmaf(t.w[k], load_agent(eo + (size_t)k * kHidden + r), moe);
      const float sd = t.n_slots > t.K ? load_agent(eo + (size_t)t.K * kHidden + r) : 0.0f;
      const float hin = h_in ? h_in[r] : 0.0f;
      out[r] = (hin + moe) + sd;
      if (moe_out) moe_out[r] = moe;
    }
    if (threadIdx.x == 0) reset_agent(counters + tile);
  }
}

hipError_t launch_gateup(const SlotTable& t, const XGroup* xd, float* act, XGroup* act_xd,
                         int* counters, hipStream_t s, int slot0, int n_run) {
  SlotTable r = t;
  r.slot0 = slot0;
  const int n = n_run < 0 ? t.n_slots - slot0 : n_run;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_gateup, dim3(kGuTiles * n), dim3(256), 0, s, r, xd, act, act_xd, counters);
  return hipGetLastError();
}

hipError_t launch_down_combine(const SlotTable& t, bool down_q6, const XGroup* act_xd,
                               const float* h_in, float* out, float* moe_out, float* eo,
                               int* counters, hipStream_t s, int slot0, int n_run) {
  SlotTable r = t;
  r.slot0 = slot0;
  const int n = n_run < 0 ? t.n_slots - slot0 : n_run;
  if (n <= 0) return hipSuccess;
  const dim3 grid(kDnTiles, n), block(256);
  if (down_q6)
    hipLaunchKernelGGL(k_down<true>, grid, block, 0, s, r, act_xd, h_in, out, moe_out, eo,
                       counters);
  else
    hipLaunchKernelGGL(k_down<false>, grid, block, 0, s, r, act_xd, h_in, out, moe_out, eo,
                       counters);
  return hipGetLastError();
}

}  // namespace fdm
