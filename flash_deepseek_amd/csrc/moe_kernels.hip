// moe_kernels.hip -- the expert FFN of the MoE layer for all selected
// experts at once (infer.m:1559-1575 encode_expert, run for every slot, and
// the combine of infer.m:1689-1695 / 1922).
//
// k_gateup:  one workgroup per (slot, 32-row tile).  Each wave computes a
//   pair of rows of gate AND the same pair of rows of up (lanes 0-31 gate,
//   32-63 up, 16 lanes per row), so SwiGLU is applied in registers
//   (swiglu_fused, shaders.metal:210-220, needs no launch of its own).  The
//   tile's 32 activations form one sub-block of the down matvec's input:
//   the workgroup writes their digits directly.
// k_down_combine:  one workgroup per 16 output rows, looping over the
//   slots: down row of each slot, weighted by the routing weight in slot
//   order, then the shared expert and the residual are added
//   (hidden = h_in + moe_out + shared, infer.m:1922).
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

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void k_gateup(SlotTable t, const XGroup* __restrict__ xd,
                                                float* __restrict__ act,
                                                XGroup* __restrict__ act_xd) {
  __shared__ XGroup xs[kHidden / 64];
  __shared__ float act_tile[32];
  const int slot = blockIdx.y, tile = blockIdx.x;
  const uint8_t* blob = slot_blob(t, slot);
  {
    const u32x4* s = reinterpret_cast<const u32x4*>(xd);
    u32x4* d = reinterpret_cast<u32x4*>(xs);
    for (int i = threadIdx.x; i < (kHidden / 64) * 9; i += 256) d[i] = s[i];
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane >> 4, l16 = lane & 15, g = l16 & 3;
  const Q4KScaleSel sel = q4k_scale_sel(g);
#pragma unroll 1
  for (int it = 0; it < 4; ++it) {
    const int rp = 8 * it + 2 * wave + (q & 1);  // row within the tile
    const int row = tile * 32 + rp;
    float acc = 0.0f;
    if (blob) {
      const uint8_t* rowp = blob + (q >= 2 ? kGateBytes : 0) + (size_t)row * kQ4KRowHidden;
      // issue every weight load of the row first (7 groups x 48 bytes per
      // lane), then consume the groups one by one against the LDS digits
      u32x4 hdr[7], q0[7], q1[7];
#pragma unroll
      for (int i = 0; i < 7; ++i) {
        const uint8_t* bp = rowp + (4 * i + (l16 >> 2)) * kQ4KBlock;
        hdr[i] = *reinterpret_cast<const u32x4_a4*>(bp);
        q0[i] = *reinterpret_cast<const u32x4_a4*>(bp + 16 + 32 * g);
        q1[i] = *reinterpret_cast<const u32x4_a4*>(bp + 32 + 32 * g);
      }
#pragma unroll
      for (int i = 0; i < 7; ++i) {
        acc += q4k_group_dot(hdr[i], q0[i], q1[i], sel, &xs[16 * i + l16]);
        // keep each group's LDS reads next to its math (bounds live registers)
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    acc = sum16(acc);
    const float up = __shfl(acc, (lane + 32) & 63);
    if (lane == 0 || lane == 16) act_tile[rp] = silu_mul(acc, up);
  }
  __syncthreads();
  if (threadIdx.x < 32) {
    const float v = act_tile[threadIdx.x];
    act[(size_t)slot * kFfn + tile * 32 + threadIdx.x] = v;
    int8_t a, b;
    float s, sum;
    make_digits32(v, a, b, s, sum);
    XGroup* xg = act_xd + (size_t)slot * (kFfn / 64) + (tile >> 1);
    const int half = tile & 1;
    xg->a[32 * half + threadIdx.x] = a;
    xg->b[32 * half + threadIdx.x] = b;
    if (threadIdx.x == 0) {
      xg->s[half] = s;
      xg->xsum[half] = sum;
    }
  }
}

template <bool Q6>
__global__ __launch_bounds__(256) void k_down_combine(SlotTable t,
                                                      const XGroup* __restrict__ act_xd,
                                                      const float* __restrict__ h_in,
                                                      float* __restrict__ out,
                                                      float* __restrict__ moe_out) {
  extern __shared__ XGroup xs[];  // n_slots * 32 records
  {
    const u32x4* s = reinterpret_cast<const u32x4*>(act_xd);
    u32x4* d = reinterpret_cast<u32x4*>(xs);
    const int n = t.n_slots * (kFfn / 64) * 9;
    for (int i = threadIdx.x; i < n; i += 256) d[i] = s[i];
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15;
  const int row = blockIdx.x * 16 + wave * 4 + (lane >> 4);
  float moe = 0.0f, sd = 0.0f;
#pragma unroll 1
  for (int k = 0; k < t.n_slots; ++k) {
    const uint8_t* blob = slot_blob(t, k);
    float acc = 0.0f;
    if (blob) {
      const uint8_t* dp = blob + 2 * (size_t)kGateBytes;
      const XGroup* xk = xs + k * (kFfn / 64);
      if (!Q6) {
        const uint8_t* rowp = dp + (size_t)row * kQ4KRowFfn;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int G = 16 * i + l16;
          const int g = G & 3;
          const Q4KScaleSel sel = q4k_scale_sel(g);
          const uint8_t* bp = rowp + (G >> 2) * kQ4KBlock;
          const u32x4 hdr = *reinterpret_cast<const u32x4_a4*>(bp);
          const u32x4 q0 = *reinterpret_cast<const u32x4_a4*>(bp + 16 + 32 * g);
          const u32x4 q1 = *reinterpret_cast<const u32x4_a4*>(bp + 32 + 32 * g);
          acc += q4k_group_dot(hdr, q0, q1, sel, &xk[G]);
        }
      } else {
        // 16 halves of 128 elements per 2048-column row: one per lane
        const uint8_t* blk = dp + (size_t)row * kQ6KRowFfn + (l16 >> 1) * kQ6KBlock;
        const int h = l16 & 1;
        uint32_t ql[16], qh[8], sc[2];
        {
          const uintptr_t a0 = reinterpret_cast<uintptr_t>(blk + 64 * h);
          const uint32_t sh = a0 & 3u;
          const uint32_t* p = reinterpret_cast<const uint32_t*>(a0 - sh);
          uint32_t wv[17];
#pragma unroll
          for (int i = 0; i < 16; ++i) wv[i] = p[i];
          wv[16] = sh ? p[16] : 0u;
#pragma unroll
          for (int i = 0; i < 16; ++i) ql[i] = funnel(wv[i], wv[i + 1], sh);
          const uint32_t* ph = reinterpret_cast<const uint32_t*>(
              reinterpret_cast<uintptr_t>(blk + 128 + 32 * h) - sh);
          uint32_t wh[9];
#pragma unroll
          for (int i = 0; i < 8; ++i) wh[i] = ph[i];
          wh[8] = sh ? ph[8] : 0u;
#pragma unroll
          for (int i = 0; i < 8; ++i) qh[i] = funnel(wh[i], wh[i + 1], sh);
        }
        const uint16_t* s16 = reinterpret_cast<const uint16_t*>(blk + 192 + 8 * h);
        sc[0] = (uint32_t)s16[0] | ((uint32_t)s16[1] << 16);
        sc[1] = (uint32_t)s16[2] | ((uint32_t)s16[3] << 16);
        const float d = half_to_float(*reinterpret_cast<const uint16_t*>(blk + 208));
        acc = d * q6k_half_dot(ql, qh, sc, &xk[2 * l16], &xk[2 * l16 + 1]);
      }
    }
    acc = sum16(acc);
    if (k < t.K)
      moe = fmaf(t.w[k], acc, moe);
    else
      sd = acc;
  }
  if (l16 == 0) {
    const float hin = h_in ? h_in[row] : 0.0f;
    out[row] = (hin + moe) + sd;
    if (moe_out) moe_out[row] = moe;
  }
}

hipError_t launch_gateup(const SlotTable& t, const XGroup* xd, float* act, XGroup* act_xd,
                         hipStream_t s) {
  hipLaunchKernelGGL(k_gateup, dim3(kFfn / 32, t.n_slots), dim3(256), 0, s, t, xd, act, act_xd);
  return hipGetLastError();
}

hipError_t launch_down_combine(const SlotTable& t, bool down_q6, const XGroup* act_xd,
                               const float* h_in, float* out, float* moe_out, hipStream_t s) {
  const size_t lds = (size_t)t.n_slots * (kFfn / 64) * sizeof(XGroup);
  const dim3 grid(kHidden / 16), block(256);
  if (lds > 65536) {
    // more than 13 slots: ask for the LDS beyond the 64 KiB default
    const void* fn = down_q6 ? reinterpret_cast<const void*>(&k_down_combine<true>)
                             : reinterpret_cast<const void*>(&k_down_combine<false>);
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  if (down_q6)
    hipLaunchKernelGGL(k_down_combine<true>, grid, block, lds, s, t, act_xd, h_in, out, moe_out);
  else
    hipLaunchKernelGGL(k_down_combine<false>, grid, block, lds, s, t, act_xd, h_in, out,
                       moe_out);
  return hipGetLastError();
}

}  // namespace fdm
