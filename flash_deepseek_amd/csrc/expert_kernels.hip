// expert_kernels.hip -- one SwiGLU expert at batch 1 (fdm_expert_ffn):
// encode_expert (infer.m:1559-1575) on the caller's packed blob,
// out = down . (silu(gate . x) * (up . x)), in ONE launch and in fp32.
//
// Work list of 256-thread workgroups:
//   gate/up items (512): gate rows 4i .. 4i+3 and up rows 4i .. 4i+3; each
//     stages x in LDS (padded, with its sub-block sums), contracts its eight
//     rows (32 lanes per row, one wave per two rows), applies SwiGLU to the
//     four row pairs and publishes the four activations as tagged words
//   final items: each requests its down rows' weights at dispatch, waits for
//     the 2048 tagged activations, stages them in LDS and contracts its rows
//     Q4_K down (224): rows 32f .. 32f+31, 32 lanes per row
//     Q6_K down (448): rows 16f .. 16f+15, 16 lanes per row (one 128-element
//       half block per lane)
// At batch 1 the expert is latency-bound (25-29 MB stream in ~4 us): fp32
// needs no digit records of x or of the activations, so the chain is x and
// weights -> gate/up -> one hand-off -> down.  The Q4_K dots are the fp32
// group dot of q4k_group_dot_f32 (dequant_matvec_q4k's arithmetic,
// shaders.metal:43-99); the Q6_K dots take d * sc * (q - 32) * x in fp32 as
// dequant_matvec_q6k (shaders.metal:123-179): per 16-element sub-block the
// products (4 (q - 32)) x summed, then scaled by d sc / 4.
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
constexpr int kExFinRows = 32;                  // down rows per final item (Q4_K)
constexpr int kExFinItems = kHidden / kExFinRows;  // 224
constexpr int kEx6Rows = 16;                    // down rows per final item (Q6_K)
constexpr int kEx6Items = kHidden / kEx6Rows;   // 448
constexpr int kExXGroups = kHidden / 64;        // 112
constexpr int kEx6Pad = 132;                    // LDS floats per 128-element half block (bank padding)

struct ExpertSmem {
  float x[kExXGroups * kXPad];  // x (gate/up items) or the activations (final items), padded
  float xs[2 * kExXGroups];     // their 32-element sub-block sums
  float row[2 * kExGuRows];     // gate/up item: gate row sums, then up row sums
};
static_assert(kFfn / 128 * kEx6Pad <= kExXGroups * kXPad, "the Q6_K items' activations fit the x buffer");

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

// The 2048 tagged activations, eight per thread (element threadIdx.x +
// 256 j in v[j]): after the first round finds them incomplete, thread 0
// watches the last one before every thread loads all again (a waiting item
// does not reload 16 KB per round).  A wait that gives up leaves the error
// flag set (ex_poll) and v as last read.
constexpr int kExActPer = kFfn / 256;
__device__ __forceinline__ void ex_wait_acts(const LayerArgs& a, float (&v)[kExActPer]) {
  auto full = [&] {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < kExActPer; ++j) {
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
  float v[kExActPer];
  ex_wait_acts(a, v);
  // element 256 j + 64 w + lane: group 4 j + w; each half wave one sub-block
#pragma unroll
  for (int j = 0; j < kExActPer; ++j) {
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


// Final item of a Q6_K down matrix: rows 16 f + 4 w + lane / 16 of wave w;
// lane h = lane % 16 holds half block h of its row (block h / 2, half h % 2).
// A half block's bytes give, for l < 32, the elements l, l + 32, l + 64,
// l + 96 of the half (dequantize_row_q6_K, quant.c:63-92):
//   q = (ql[l or l + 32] nibble) | (2 bits of qh[l]) << 4, value q - 32.
// Four bytes at a time: with every second bit of qh flipped, q ^ 32 -- the
// 6-bit two's complement of q - 32 -- is assembled shifted left by two, so
// each byte is the signed int8 4 (q - 32), widened by a signed byte
// conversion; the products with the activations are summed per 16-element
// sub-block, then scaled by d sc / 4.
__device__ __forceinline__ void ex_final_item_q6(const LayerArgs& a, int item, ExpertSmem& sm) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = lane & 15;
  const int row = kEx6Rows * item + 4 * wave + (lane >> 4);
  const uint8_t* down = a.shared + 2 * (size_t)kGateBytes;
  const Q6KHalfLoad ld = q6k_load_half(down + (size_t)row * kQ6KRowFfn + (h >> 1) * kQ6KBlock, h & 1);
  float v[kExActPer];
  ex_wait_acts(a, v);
  // element e into the padded half-block rows of LDS
#pragma unroll
  for (int j = 0; j < kExActPer; ++j) {
    const int e = threadIdx.x + 256 * j;
    sm.x[kEx6Pad * (e >> 7) + (e & 127)] = v[j];
  }
  __syncthreads();
  const float* xh = sm.x + kEx6Pad * h;
  uint32_t ql[16], qh[8];
#pragma unroll
  for (int i = 0; i < 16; ++i) ql[i] = funnel(ld.ql[i], ld.ql[i + 1], ld.shift);
#pragma unroll
  for (int i = 0; i < 8; ++i) qh[i] = funnel(ld.qh[i], ld.qh[i + 1], ld.shift) ^ 0xAAAAAAAAu;
  // S[k][sb]: element quarter k (elements 32 k .. 32 k + 31), sub-block sb of it
  float S[4][2] = {};
#pragma unroll
  for (int i = 0; i < 8; ++i) {  // bytes l = 4 i .. 4 i + 3
    const uint32_t A = ql[i], B = ql[i + 8], H = qh[i];
    uint32_t w4[4];
    w4[0] = ((A << 2) & 0x3C3C3C3Cu) | ((H << 6) & 0xC0C0C0C0u);  // l:      low nibble, qh bits 0-1
    w4[1] = ((B << 2) & 0x3C3C3C3Cu) | ((H << 4) & 0xC0C0C0C0u);  // l + 32: low nibble, qh bits 2-3
    w4[2] = ((A >> 2) & 0x3C3C3C3Cu) | ((H << 2) & 0xC0C0C0C0u);  // l + 64: high nibble, qh bits 4-5
    w4[3] = ((B >> 2) & 0x3C3C3C3Cu) | (H & 0xC0C0C0C0u);         // l + 96: high nibble, qh bits 6-7
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const f32x4 x4 = *reinterpret_cast<const f32x4*>(xh + 32 * k + 4 * i);
      float s = S[k][i >> 2];
      s = fmaf((float)(int8_t)(w4[k]), x4.x, s);
      s = fmaf((float)(int8_t)(w4[k] >> 8), x4.y, s);
      s = fmaf((float)(int8_t)(w4[k] >> 16), x4.z, s);
      s = fmaf((float)(int8_t)(w4[k] >> 24), x4.w, s);
      S[k][i >> 2] = s;
    }
  }
  const float d4 = half_to_float(ld.d) * 0.25f;
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const int si = 2 * k + sb;  // scale index within the half
      const float sc = (float)(int8_t)(ld.sc[si >> 2] >> (8 * (si & 3)));
      acc = fmaf(d4 * sc, S[k][sb], acc);
    }
  acc = group_sum_first<16>(acc);
  if (h == 0) a.out[row] = acc;
}

}  // namespace

__global__ __launch_bounds__(256) void k_expert_f32_q4k(LayerArgs a) {
  __shared__ ExpertSmem sm;
  if ((int)blockIdx.x < kExGuItems)
    ex_gateup_item(a, blockIdx.x, sm);
  else
    ex_final_item(a, blockIdx.x - kExGuItems, sm);
}

__global__ __launch_bounds__(256) void k_expert_f32_q6k(LayerArgs a) {
  __shared__ ExpertSmem sm;
  if ((int)blockIdx.x < kExGuItems)
    ex_gateup_item(a, blockIdx.x, sm);
  else
    ex_final_item_q6(a, blockIdx.x - kExGuItems, sm);
}

hipError_t launch_expert_f32(const LayerArgs& a, hipStream_t s) {
  if (a.down_q6)
    hipLaunchKernelGGL(k_expert_f32_q6k, dim3(kExGuItems + kEx6Items), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(k_expert_f32_q4k, dim3(kExGuItems + kExFinItems), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace fdm
