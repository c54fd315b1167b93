// dense_kernels.hip -- the dense FFN of the first layers (L < 3) and the F16
// conversion used to make its weights.
//
// The reference runs hidden = h_in + W_down . (silu(W_gate . h_post) *
// (W_up . h_post)) with F16 weights and fp32 activations (infer.m:1852-1868;
// mv_f16 / sgemv_f16_serial at infer.m:459-513; silu_mul at infer.m:378-383).
// The weights are what dequant_tensor_f16 (infer.m:530-538) leaves: the GGUF
// tensor widened to fp32 (infer.m:314-355), then cast to __fp16
// (f32_to_f16_alloc, infer.m:521-528).
//
// Both matvecs stream 2-byte weights once (792 MB per R1 layer), so they
// are bound by HBM.  Every wave reads whole rows in 1 KB instructions (64
// lanes x 8 halves, nontemporal), and multiplies them with the activation
// vector held in LDS in fp32; each lane keeps an fp32 partial sum, reduced
// across the wave at the end of the row.  The grid is one wave of resident
// workgroups whose rows divide evenly at R1 sizes (3 gate/up rows and 2
// down rows per wave on 256 CUs), so no CU finishes a row later than the
// others.
#include "fdm_internal.h"

namespace fdm {

namespace {

constexpr int kDnChunk = 512;  // halves per wave load: 64 lanes x 8
constexpr int kGuChunks = kHidden / kDnChunk;  // 14 per gate/up row
constexpr int kGuBatch = 7;                    // loads per matrix in flight per wave
constexpr int kGuWaves = 6;                    // gate/up: 6 waves, 4 workgroups per CU
constexpr int kDnWaves = 7;                    // down: 7 waves, 2 workgroups per CU
constexpr int kDnBatch = 12;                   // down loads in flight per wave
static_assert(kGuChunks % kGuBatch == 0, "gate/up batches tile a row");

// IEEE binary32 -> binary16, round to nearest even, by integer construction:
// subnormal results kept, overflow to infinity, NaN quieted with the top
// payload bits kept (what a (__fp16) cast gives on the reference's host).
__device__ __forceinline__ uint16_t f32_bits_to_f16(uint32_t x) {
  const uint32_t sign = (x >> 16) & 0x8000u, e = (x >> 23) & 0xFFu, m = x & 0x7FFFFFu;
  if (e == 0xFFu) return (uint16_t)(sign | (m ? 0x7E00u | ((m >> 13) & 0x1FFu) : 0x7C00u));
  if (e >= 143u) return (uint16_t)(sign | 0x7C00u);  // >= 2^16: beyond the largest half
  if (e >= 113u) {                                    // a normal half (or rounds up to 2^16)
    uint32_t h = ((e - 112u) << 10) | (m >> 13);
    const uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // may carry into inf: correct
    return (uint16_t)(sign | h);
  }
  const uint32_t shift = 126u - e;  // subnormal half: M x 2^(e-150) in units of 2^-24
  if (shift > 24u) return (uint16_t)sign;
  const uint32_t M = m | 0x800000u;
  uint32_t h = M >> shift;
  const uint32_t rem = M & ((1u << shift) - 1u), half = 1u << (shift - 1u);
  if (rem > half || (rem == half && (h & 1u))) ++h;
  return (uint16_t)(sign | h);
}

// acc + sum of 8 halves (one u32x4) times 8 floats, in element order.
__device__ __forceinline__ float dot8(u32x4 w, f32x4 x0, f32x4 x1, float acc) {
  const auto h = [](uint32_t v, int hi) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(hi ? v >> 16 : v & 0xFFFFu));
  };
  acc = fmaf(h(w.x, 0), x0.x, acc);
  acc = fmaf(h(w.x, 1), x0.y, acc);
  acc = fmaf(h(w.y, 0), x0.z, acc);
  acc = fmaf(h(w.y, 1), x0.w, acc);
  acc = fmaf(h(w.z, 0), x1.x, acc);
  acc = fmaf(h(w.z, 1), x1.y, acc);
  acc = fmaf(h(w.w, 0), x1.z, acc);
  acc = fmaf(h(w.w, 1), x1.w, acc);
  return acc;
}

// The xor butterfly's lane-0 sum (the same bits), through lane permutes and
// DPP shifts; only lane 0 reads it.
__device__ __forceinline__ float wave_sum(float v) { return wave_sum_lane0(v); }

}  // namespace

// dst[i] = (__fp16) of element i of src (F32, BF16 or F16 elements).
__global__ __launch_bounds__(256) void k_to_f16(const void* __restrict__ src, int type,
                                                uint16_t* __restrict__ dst, size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    uint32_t x;
    if (type == kGgmlF16) {
      dst[i] = static_cast<const uint16_t*>(src)[i];
      continue;
    }
    if (type == kGgmlBF16)
      x = (uint32_t)static_cast<const uint16_t*>(src)[i] << 16;
    else
      x = static_cast<const uint32_t*>(src)[i];
    dst[i] = f32_bits_to_f16(x);
  }
}

// act[r] = silu(gate[r] . x) * (up[r] . x) for rows r of [0, inter).
__global__ __launch_bounds__(kGuWaves * 64) __attribute__((amdgpu_waves_per_eu(6))) void k_dense_gateup(const uint16_t* __restrict__ gate,
                                                                const uint16_t* __restrict__ up,
                                                                const float* __restrict__ x,
                                                                float* __restrict__ act, int inter) {
  __shared__ float xs[kHidden];  // 28 KB
  for (int i = threadIdx.x; i < kHidden / 4; i += blockDim.x)
    reinterpret_cast<f32x4*>(xs)[i] = reinterpret_cast<const f32x4*>(x)[i];
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_waves = gridDim.x * kGuWaves;
  for (int r = blockIdx.x * kGuWaves + wave; r < inter; r += n_waves) {
    const uint16_t* gr = gate + (size_t)r * kHidden + 8 * lane;
    const uint16_t* ur = up + (size_t)r * kHidden + 8 * lane;
    float g = 0.0f, u = 0.0f;
#pragma unroll 1
    for (int b = 0; b < kGuChunks; b += kGuBatch) {
      u32x4 gw[kGuBatch], uw[kGuBatch];
#pragma unroll
      for (int i = 0; i < kGuBatch; ++i) {
        gw[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(gr + (b + i) * kDnChunk));
        uw[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ur + (b + i) * kDnChunk));
      }
      __builtin_amdgcn_sched_barrier(0);  // all 14 loads in flight before the first product
#pragma unroll
      for (int i = 0; i < kGuBatch; ++i) {
        const float* xp = xs + (b + i) * kDnChunk + 8 * lane;
        const f32x4 x0 = *reinterpret_cast<const f32x4*>(xp), x1 = *reinterpret_cast<const f32x4*>(xp + 4);
        g = dot8(gw[i], x0, x1, g);
        u = dot8(uw[i], x0, x1, u);
      }
    }
    g = wave_sum(g);
    u = wave_sum(u);
    if (lane == 0) act[r] = silu_mul(g, u);
  }
}

// out[r] = h_in[r] + down[r] . act for the kHidden rows (h_in may be null).
__global__ __launch_bounds__(kDnWaves * 64) void k_dense_down(const uint16_t* __restrict__ down,
                                                              const float* __restrict__ act,
                                                              const float* __restrict__ h_in,
                                                              float* __restrict__ out, int inter) {
  __shared__ float as[kDenseMaxFfn];  // 72 KB
  for (int i = threadIdx.x; i < inter / 4; i += blockDim.x)
    reinterpret_cast<f32x4*>(as)[i] = reinterpret_cast<const f32x4*>(act)[i];
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_waves = gridDim.x * kDnWaves, chunks = inter / kDnChunk;
  for (int r = blockIdx.x * kDnWaves + wave; r < kHidden; r += n_waves) {
    const uint16_t* dr = down + (size_t)r * inter + 8 * lane;
    float d = 0.0f;
    for (int b = 0; b < chunks; b += kDnBatch) {
      u32x4 w[kDnBatch];
#pragma unroll
      for (int i = 0; i < kDnBatch; ++i)
        if (b + i < chunks) w[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(dr + (b + i) * kDnChunk));
#pragma unroll
      for (int i = 0; i < kDnBatch; ++i) {
        if (b + i < chunks) {
          const float* ap = as + (b + i) * kDnChunk + 8 * lane;
          d = dot8(w[i], *reinterpret_cast<const f32x4*>(ap), *reinterpret_cast<const f32x4*>(ap + 4), d);
        }
      }
    }
    d = wave_sum(d);
    if (lane == 0) out[r] = (h_in ? h_in[r] : 0.0f) + d;
  }
}

// dst[h][c][r] = src[h * head_stride + r * cols + c] for r < rows, c < cols
// (the per-head transpose of k_b at load, infer.m:1707-1721).
__global__ __launch_bounds__(256) void k_transpose_heads(const uint16_t* __restrict__ src, size_t head_stride,
                                                         uint16_t* __restrict__ dst, int heads, int rows, int cols) {
  const size_t n = (size_t)heads * rows * cols, stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const int r = (int)(i % rows);
    const size_t hc = i / rows;
    const int c = (int)(hc % cols), h = (int)(hc / cols);
    dst[i] = src[(size_t)h * head_stride + (size_t)r * cols + c];
  }
}

hipError_t launch_transpose_heads(const uint16_t* src, size_t head_stride, uint16_t* dst, int heads, int rows,
                                  int cols, hipStream_t s) {
  k_transpose_heads<<<4096, 256, 0, s>>>(src, head_stride, dst, heads, rows, cols);
  return hipGetLastError();
}

hipError_t launch_to_f16(const void* src, int type, uint16_t* dst, size_t n, hipStream_t s) {
  const size_t blocks = (n + 255) / 256;
  k_to_f16<<<(unsigned)(blocks < 16384 ? (blocks ? blocks : 1) : 16384), 256, 0, s>>>(src, type, dst, n);
  return hipGetLastError();
}

hipError_t launch_dense_ffn(const DenseArgs& a, hipStream_t s) {
  k_dense_gateup<<<4 * a.n_cus, kGuWaves * 64, 0, s>>>(a.gate, a.up, a.x, a.act, a.inter);
  if (hipError_t e = hipGetLastError()) return e;
  k_dense_down<<<2 * a.n_cus, kDnWaves * 64, 0, s>>>(a.down, a.act, a.h_in, a.out, a.inter);
  return hipGetLastError();
}

}  // namespace fdm
