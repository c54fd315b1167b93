// attn_kernels.hip -- MLA attention of one decode token (mla_forward,
// infer.m:766-903) on the device, with the weights in the layout the
// reference holds them (LayerAttnDense, infer.m:687-706: F16 row-major;
// k_b per head (KV_LORA, NOPE), v_b per head (V_HEAD, KV_LORA)) and the
// latent KV cache in fp32 (MLACache, infer.m:663-669).
//
// Launch sequence of one token (fdm_attn_forward):
//   rms_norm(hidden, attn_norm)                        (bit-exact, shared kernel)
//   q_a = W_qa . normed; rms_norm(q_a, q_a_norm)       k_mv_f16, rms_norm
//   q = W_qb . q_a_n  [128][192]                        k_mv_f16
//   kv_a = W_kva . normed [576]; rms_norm(kv_a[:512])   k_mv_f16, rms_norm
//   YaRN RoPE of q_rope and k_rope at pos, cache append k_mla_rope_append
//   Q_abs[h] = k_b[h] . q_nope[h]  [128][512]           k_mv_f16_heads
//   scores[h][s] = scale (Q_abs[h].c_kv[s] + q_rope[h].k_rope[s])   k_mla_scores
//   p = softmax(scores[h]) in place                                  k_mla_softmax
//   wc[h] = sum_s p[h][s] c_kv[s] (per 64-position chunk, then summed) k_mla_wsum_part/_reduce
//   attn[h] = v_b[h] . wc[h]  [128][128]                k_mv_f16_heads
//   hidden = residual + W_o . attn                      k_mv_f16 (+ residual)
// The matvecs stream F16 weights (375 MB per R1 layer) once and bound the
// token: each wave reads a row in 1 KB instructions against the input
// vector in LDS, as the dense FFN kernels do.
#include "fdm_internal.h"

namespace fdm {

namespace {

constexpr int kMvChunk = 512;   // halves per wave load
constexpr int kMvBatch = 8;     // loads in flight per wave
constexpr int kMvWaves = 4;
constexpr int kMvMaxCols = 16384;  // o_proj input: 128 heads x 128

__device__ __forceinline__ float mv_dot8(u32x4 w, const float* x, float acc) {
  const f32x4 x0 = *reinterpret_cast<const f32x4*>(x), x1 = *reinterpret_cast<const f32x4*>(x + 4);
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

__device__ __forceinline__ float lane_sum(float v, int width) {
  for (int m = width / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

}  // namespace

// y[r] = (res ? res[r] : 0) + W[r] . x for rows r < rows; cols % 512 == 0,
// cols <= 16384.  One wave per row (grid-stride), x staged in LDS.
__global__ __launch_bounds__(kMvWaves * 64) void k_mv_f16(const uint16_t* __restrict__ W,
                                                          const float* __restrict__ x,
                                                          const float* __restrict__ res,
                                                          float* __restrict__ y, int rows, int cols) {
  __shared__ float xs[kMvMaxCols];  // 64 KB
  for (int i = threadIdx.x; i < cols / 4; i += blockDim.x)
    reinterpret_cast<f32x4*>(xs)[i] = reinterpret_cast<const f32x4*>(x)[i];
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_waves = gridDim.x * kMvWaves, chunks = cols / kMvChunk;
  for (int r = blockIdx.x * kMvWaves + wave; r < rows; r += n_waves) {
    const uint16_t* wr = W + (size_t)r * cols + 8 * lane;
    float acc = 0.0f;
    for (int b = 0; b < chunks; b += kMvBatch) {
      u32x4 w[kMvBatch];
#pragma unroll
      for (int i = 0; i < kMvBatch; ++i)
        if (b + i < chunks) w[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + (b + i) * kMvChunk));
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < kMvBatch; ++i)
        if (b + i < chunks) acc = mv_dot8(w[i], xs + (b + i) * kMvChunk + 8 * lane, acc);
    }
    acc = lane_sum(acc, 64);
    if (lane == 0) y[r] = (res ? res[r] : 0.0f) + acc;
  }
}

// Per-head matvec: y[h * rows_h + r] = W[h][r] . x[h * x_stride .. + cols]
// for h < heads, r < rows_h; cols is 128 or 512 (cols / 8 lanes per row,
// 64 / (cols / 8) rows per wave step).
__global__ __launch_bounds__(256) void k_mv_f16_heads(const uint16_t* __restrict__ W,
                                                      const float* __restrict__ x, int x_stride,
                                                      float* __restrict__ y, int heads, int rows_h, int cols) {
  const int lane = threadIdx.x & 63;
  const int lpr = cols / 8, rpw = 64 / lpr;  // lanes per row, rows per wave step
  const int sub = lane / lpr, l = lane % lpr;
  const int total = heads * rows_h;
  const int wave_g = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int n_waves = (gridDim.x * blockDim.x) >> 6;
  for (int r0 = wave_g * rpw; r0 < total; r0 += n_waves * rpw) {
    const int r = r0 + sub;
    float acc = 0.0f;
    if (r < total) {
      const int h = r / rows_h;
      const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(W + (size_t)r * cols + 8 * l));
      acc = mv_dot8(w, x + (size_t)h * x_stride + 8 * l, 0.0f);
    }
    acc = lane_sum(acc, lpr);
    if (l == 0 && r < total) y[r] = acc;
  }
}

// YaRN RoPE (interleaved pairs, infer.m:626-655) of the 128 heads' q_rope
// (q[h][128 .. 191]) and of k_rope = kv_a[512 .. 575] at position pos, with
// freq[i] the layer's table of yarn_freq(i); then the token's cache row:
// c_kv[len] = c_kv_n, k_rope[len] = rotated k_rope.
__global__ __launch_bounds__(256) void k_mla_rope_append(float* __restrict__ q, const float* __restrict__ kv_a,
                                                         const float* __restrict__ c_kv_n,
                                                         const float* __restrict__ freq, int pos,
                                                         float* __restrict__ cache_c, float* __restrict__ cache_k,
                                                         int len) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;  // pair index
  if (t < 128 * 32 + 32) {
    const int i = t & 31;
    const float ang = (float)pos * freq[i];
    const float c = cosf(ang), s = sinf(ang);
    if (t < 128 * 32) {
      float* p = q + (t >> 5) * 192 + 128 + 2 * i;
      const float a = p[0], b = p[1];
      p[0] = a * c - b * s;
      p[1] = a * s + b * c;
    } else {
      const float a = kv_a[512 + 2 * i], b = kv_a[512 + 2 * i + 1];
      cache_k[(size_t)len * 64 + 2 * i] = a * c - b * s;
      cache_k[(size_t)len * 64 + 2 * i + 1] = a * s + b * c;
    }
  }
  if (t < 512) cache_c[(size_t)len * 512 + t] = c_kv_n[t];
}

// scores[h][s] = scale * (Q_abs[h] . c_kv[s]) + scale * (q_rope[h] . k_rope[s])
// for s < S (the reference's two sgemm calls, infer.m:829-838), as a tiled
// product: workgroup (position block of 64, head block of 8); the 576 dims
// go through LDS in 9 tiles of 64 (8 latent, 1 rope), the cache tile
// transposed so the 64 lanes of a wave read 64 consecutive positions.
// Thread (wave w, lane p): position p of the block, heads 2 w, 2 w + 1.
__global__ __launch_bounds__(256) void k_mla_scores(const float* __restrict__ q_abs, const float* __restrict__ q,
                                                    const float* __restrict__ cache_c,
                                                    const float* __restrict__ cache_k, int S, float scale,
                                                    float* __restrict__ scores) {
  __shared__ float ct[64][65];  // [dim][position], padded
  __shared__ float qt[8][64];  // [head][dim]
  const int s0 = blockIdx.x * 64, h0 = blockIdx.y * 8;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float a[2] = {}, b[2] = {};
  for (int tile = 0; tile < 9; ++tile) {
    const bool rope = tile == 8;
    __syncthreads();
    // cache tile: positions s0 .. s0 + 63, dims 64 tile .. + 63 (coalesced
    // rows); every load of the tile is issued before the first LDS store
    float cv[16], qv[2];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int i = threadIdx.x + 256 * k, sp = i >> 6, d = i & 63, s = s0 + sp;
      cv[k] = s < S ? (rope ? cache_k[(size_t)s * 64 + d] : cache_c[(size_t)s * 512 + 64 * tile + d]) : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int i = threadIdx.x + 256 * k, h = h0 + (i >> 6), d = i & 63;
      qv[k] = rope ? q[(size_t)h * 192 + 128 + d] : q_abs[(size_t)h * 512 + 64 * tile + d];
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int i = threadIdx.x + 256 * k;
      ct[i & 63][i >> 6] = cv[k];
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int i = threadIdx.x + 256 * k;
      qt[i >> 6][i & 63] = qv[k];
    }
    __syncthreads();
#pragma unroll 8
    for (int d = 0; d < 64; ++d) {
      const float c = ct[d][lane];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (rope)
          b[j] = fmaf(qt[2 * wave + j][d], c, b[j]);
        else
          a[j] = fmaf(qt[2 * wave + j][d], c, a[j]);
      }
    }
  }
  const int s = s0 + lane;
  if (s < S) {
#pragma unroll
    for (int j = 0; j < 2; ++j) scores[(size_t)(h0 + 2 * wave + j) * S + s] = scale * a[j] + scale * b[j];
  }
}

// Per head (one workgroup each): scores[h][0..S) <- softmax (infer.m:385-389),
// in place.
__global__ __launch_bounds__(256) void k_mla_softmax(float* __restrict__ scores, int S) {
  __shared__ float red[4];
  __shared__ float stat;
  const int h = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float* sc = scores + (size_t)h * S;
  float m = -__builtin_inff();
  for (int s = threadIdx.x; s < S; s += 256) m = fmaxf(m, sc[s]);
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  if (lane == 0) red[wave] = m;
  __syncthreads();
  if (threadIdx.x == 0) stat = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  m = stat;
  float sum = 0.0f;
  for (int s = threadIdx.x; s < S; s += 256) {
    const float e = expf(sc[s] - m);
    sc[s] = e;
    sum += e;
  }
  sum = lane_sum(sum, 64);
  __syncthreads();
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  if (threadIdx.x == 0) stat = 1.0f / ((red[0] + red[1]) + (red[2] + red[3]));
  __syncthreads();
  const float inv = stat;
  for (int s = threadIdx.x; s < S; s += 256) sc[s] *= inv;
}

// Partial latent sums (infer.m:862-867 as a tiled product): workgroup
// (chunk c of 64 positions, block of 64 latent dims) reads its cache tile
// and the 128 heads' probabilities once; thread t: dim 64 b + (t & 63),
// heads (t >> 6) + 4 j, j < 32.  part[c][h][d] = sum over the chunk.
__global__ __launch_bounds__(256) void k_mla_wsum_part(const float* __restrict__ p, int S,
                                                       const float* __restrict__ cache_c,
                                                       float* __restrict__ part) {
  __shared__ float ct[64][64];    // [position][dim]
  __shared__ float pt[128][65];   // [head][position], padded
  const int c = blockIdx.x, d0 = blockIdx.y * 64, s0 = c * 64, ns = min(64, S - s0);
  const int lane = threadIdx.x & 63, hq = threadIdx.x >> 6;
  float cv[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int i = threadIdx.x + 256 * k, sp = i >> 6;
    cv[k] = sp < ns ? cache_c[(size_t)(s0 + sp) * 512 + d0 + (i & 63)] : 0.0f;
  }
  float pv[32];
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    const int i = threadIdx.x + 256 * k, h = i >> 6, sp = i & 63;
    pv[k] = sp < ns ? p[(size_t)h * S + s0 + sp] : 0.0f;
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int i = threadIdx.x + 256 * k;
    ct[i >> 6][i & 63] = cv[k];
  }
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    const int i = threadIdx.x + 256 * k;
    pt[i >> 6][i & 63] = pv[k];
  }
  __syncthreads();
  float acc[32] = {};
  for (int sp = 0; sp < 64; ++sp) {
    const float cval = ct[sp][lane];
#pragma unroll
    for (int j = 0; j < 32; ++j) acc[j] = fmaf(pt[hq + 4 * j][sp], cval, acc[j]);
  }
#pragma unroll
  for (int j = 0; j < 32; ++j) part[((size_t)c * 128 + hq + 4 * j) * 512 + d0 + lane] = acc[j];
}

// wc[h][d] = sum over chunks c = 0, 1, ... of part[c][h][d] (fixed order).
__global__ __launch_bounds__(256) void k_mla_wsum_reduce(const float* __restrict__ part, int n_chunks,
                                                         float* __restrict__ wc) {
  const int i = blockIdx.x * 256 + threadIdx.x;  // < 128 * 512
  float a = 0.0f;
  for (int c = 0; c < n_chunks; ++c) a += part[(size_t)c * 128 * 512 + i];
  wc[i] = a;
}

hipError_t launch_mv_f16(const uint16_t* W, const float* x, const float* res, float* y, int rows, int cols,
                         hipStream_t s) {
  const int wgs = min((rows + kMvWaves - 1) / kMvWaves, 2 * g_num_cus);
  k_mv_f16<<<wgs, kMvWaves * 64, 0, s>>>(W, x, res, y, rows, cols);
  return hipGetLastError();
}

hipError_t launch_mv_f16_heads(const uint16_t* W, const float* x, int x_stride, float* y, int heads, int rows_h,
                               int cols, hipStream_t s) {
  const int rows = heads * rows_h, rpw = 64 / (cols / 8);
  const int waves = (rows + rpw - 1) / rpw;
  const int wgs = min((waves + 3) / 4, 4 * g_num_cus);
  k_mv_f16_heads<<<wgs, 256, 0, s>>>(W, x, x_stride, y, heads, rows_h, cols);
  return hipGetLastError();
}

hipError_t launch_mla_attend(const MlaArgs& a, hipStream_t s) {
  k_mla_rope_append<<<(128 * 32 + 32 + 255) / 256, 256, 0, s>>>(a.q, a.kv_a, a.c_kv_n, a.freq, a.pos, a.cache_c,
                                                                  a.cache_k, a.len);
  if (hipError_t e = hipGetLastError()) return e;
  // Q_abs[h] = k_b[h] (512 x 128) . q_nope[h]
  if (hipError_t e = launch_mv_f16_heads(a.k_b, a.q, 192, a.q_abs, 128, 512, 128, s)) return e;
  const int S = a.len + 1;
  k_mla_scores<<<dim3((S + 63) / 64, 128 / 8), 256, 0, s>>>(a.q_abs, a.q, a.cache_c, a.cache_k, S, a.scale,
                                                             a.scores);
  if (hipError_t e = hipGetLastError()) return e;
  k_mla_softmax<<<128, 256, 0, s>>>(a.scores, S);
  if (hipError_t e = hipGetLastError()) return e;
  const int n_chunks = (S + 63) / 64;
  k_mla_wsum_part<<<dim3(n_chunks, 512 / 64), 256, 0, s>>>(a.scores, S, a.cache_c, a.part);
  if (hipError_t e = hipGetLastError()) return e;
  k_mla_wsum_reduce<<<128 * 512 / 256, 256, 0, s>>>(a.part, n_chunks, a.wc);
  if (hipError_t e = hipGetLastError()) return e;
  // attn[h] = v_b[h] (128 x 512) . wc[h]
  return launch_mv_f16_heads(a.v_b, a.wc, 512, a.attn, 128, 128, 512, s);
}

}  // namespace fdm
