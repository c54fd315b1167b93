// attn_kernels.hip -- MLA attention of one decode token (mla_forward,
// infer.m:766-903) on the device, with the weights in the layout the
// reference holds them (LayerAttnDense, infer.m:687-706: F16 row-major;
// k_b per head (KV_LORA, NOPE), v_b per head (V_HEAD, KV_LORA)) and the
// latent KV cache in fp32 (MLACache, infer.m:663-669).
//
// Launch sequence of one token (fdm_attn_forward):
//   rms_norm(hidden, attn_norm)                        (bit-exact, shared kernel)
//   [q_a; kv_a] = [W_qa; W_kva] . normed  [1536 + 576]  k_mv_f16 (the two stacked)
//   rms_norm(q_a, q_a_norm), rms_norm(kv_a[:512])        k_rms_norm_pair
//   q = W_qb . q_a_n  [128][192]                        k_mv_f16
//   YaRN RoPE of q_rope and k_rope at pos, cache append k_mla_rope_append
//   Q_abs[h] = k_b[h] . q_nope[h]  [128][512]           k_mv_f16_heads
//   scores[h][s] = scale (Q_abs[h].c_kv[s] + q_rope[h].k_rope[s])   k_mla_scores_mfma
//   p = softmax(scores[h]) in place                                  k_mla_softmax
//   wc[h] = sum_s p[h][s] c_kv[s] (per 256-position chunk, summed)  k_mla_wsum_mfma/_reduce
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
// cols <= 16384.  One wave per row (grid-stride), x staged in LDS (cols
// floats of dynamic LDS: the narrow projections keep more workgroups per CU
// than a fixed 64 KB would allow).
__global__ __launch_bounds__(kMvWaves * 64) void k_mv_f16(const uint16_t* __restrict__ W,
                                                          const float* __restrict__ x,
                                                          const float* __restrict__ res,
                                                          float* __restrict__ y, int rows, int cols) {
  extern __shared__ float xs[];  // cols floats
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
    acc = wave_sum_lane0(acc);  // the butterfly's lane-0 sum, VALU only
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
    // the group's butterfly sum into its first lane (the same bits), VALU only
    acc = lpr == 64 ? wave_sum_lane0(acc) : group_sum_first<16>(acc);
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
// for s < S (the reference's two sgemm calls, infer.m:829-838) on fp32 MFMA
// (v_mfma_f32_16x16x4f32: fp32 products, fp32 accumulation, as the sgemm): one wave per tile of 16 heads x 16
// positions, heads as rows and positions as columns.  MFMA step e of a group
// of 16 dims takes from lane l the dim 16 m + 4 (l / 16) + e of its row, so
// both operands are read as float4 along the dims (the contraction order is
// the same permutation on both sides); four accumulators (one per step)
// keep four independent chains.  Workgroup: 4 position tiles of one head tile.
__device__ __forceinline__ f32x4 mfma_f32x4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__global__ __launch_bounds__(256) void k_mla_scores_mfma(const float* __restrict__ q_abs, const float* __restrict__ q,
                                                         const float* __restrict__ cache_c,
                                                         const float* __restrict__ cache_k, int S, float scale,
                                                         float* __restrict__ scores) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q4 = lane >> 4;
  const int h0 = 16 * blockIdx.y, s0 = 64 * blockIdx.x + 16 * wave;
  const int sp = min(s0 + r, S - 1);  // past the cache: a valid row, result not written
  const float* qa = q_abs + (size_t)(h0 + r) * 512 + 4 * q4;
  const float* cc = cache_c + (size_t)sp * 512 + 4 * q4;
  f32x4 a[4], b[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) a[e] = b[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
  for (int m = 0; m < 32; ++m) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(qa + 16 * m);
    const f32x4 y = *reinterpret_cast<const f32x4*>(cc + 16 * m);
#pragma unroll
    for (int e = 0; e < 4; ++e) a[e] = mfma_f32x4(x[e], y[e], a[e]);
  }
  const float* qr = q + (size_t)(h0 + r) * 192 + 128 + 4 * q4;
  const float* kr = cache_k + (size_t)sp * 64 + 4 * q4;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(qr + 16 * m);
    const f32x4 y = *reinterpret_cast<const f32x4*>(kr + 16 * m);
#pragma unroll
    for (int e = 0; e < 4; ++e) b[e] = mfma_f32x4(x[e], y[e], b[e]);
  }
  // D: lane l holds heads h0 + 4 (l / 16) + v, position s0 + l % 16
  const int s = s0 + r;
  if (s < S) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float av = (a[0][v] + a[1][v]) + (a[2][v] + a[3][v]);
      const float bv = (b[0][v] + b[1][v]) + (b[2][v] + b[3][v]);
      scores[(size_t)(h0 + 4 * q4 + v) * S + s] = scale * av + scale * bv;
    }
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

// Partial latent sums on fp32 MFMA: part[c][h][d] = sum over the positions
// of chunk c (kMlaChunk of them) of p[h][s] c_kv[s][d] (infer.m:862-867).  One
// wave per tile of 16 heads (rows) x 16 latent dims (columns); step e of a
// group of 16 positions takes from lane l the position 16 m + 4 (l / 16) + e.
// Workgroup: 4 dim tiles of one head tile and one chunk.
constexpr int kMlaChunk = 256;

__global__ __launch_bounds__(256) void k_mla_wsum_mfma(const float* __restrict__ p, int S,
                                                       const float* __restrict__ cache_c,
                                                       float* __restrict__ part) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q4 = lane >> 4;
  const int c = blockIdx.x, h0 = 16 * (blockIdx.y >> 3), d0 = 64 * (blockIdx.y & 7) + 16 * wave;
  const int base = c * kMlaChunk, end = min(S, base + kMlaChunk);
  const float* pr = p + (size_t)(h0 + r) * S;
  f32x4 acc[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int g = base; g < end; g += 16) {
    const int s = g + 4 * q4;
    float x[4], y[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool in = s + e < end;
      x[e] = in ? pr[s + e] : 0.0f;
      y[e] = in ? cache_c[(size_t)(s + e) * 512 + d0 + r] : 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] = mfma_f32x4(x[e], y[e], acc[e]);
  }
#pragma unroll
  for (int v = 0; v < 4; ++v)
    part[((size_t)c * 128 + h0 + 4 * q4 + v) * 512 + d0 + r] = (acc[0][v] + acc[1][v]) + (acc[2][v] + acc[3][v]);
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
  if (cols < 512 || cols % 512 != 0 || cols > kMvMaxCols) return hipErrorInvalidValue;
  const size_t lds = (size_t)cols * sizeof(float);
  const int per_cu = max(1, min(8, (int)((160u << 10) / lds)));  // workgroups per CU the LDS allows
  const int wgs = min((rows + kMvWaves - 1) / kMvWaves, per_cu * g_num_cus);
  k_mv_f16<<<wgs, kMvWaves * 64, lds, s>>>(W, x, res, y, rows, cols);
  return hipGetLastError();
}

hipError_t launch_mv_f16_heads(const uint16_t* W, const float* x, int x_stride, float* y, int heads, int rows_h,
                               int cols, hipStream_t s) {
  if (cols != 128 && cols != 512) return hipErrorInvalidValue;  // 16 or 64 lanes per row
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
  k_mla_scores_mfma<<<dim3((S + 63) / 64, 128 / 16), 256, 0, s>>>(a.q_abs, a.q, a.cache_c, a.cache_k, S, a.scale,
                                                                  a.scores);
  if (hipError_t e = hipGetLastError()) return e;
  k_mla_softmax<<<128, 256, 0, s>>>(a.scores, S);
  if (hipError_t e = hipGetLastError()) return e;
  const int n_chunks = (S + kMlaChunk - 1) / kMlaChunk;
  k_mla_wsum_mfma<<<dim3(n_chunks, (128 / 16) * 8), 256, 0, s>>>(a.scores, S, a.cache_c, a.part);
  if (hipError_t e = hipGetLastError()) return e;
  k_mla_wsum_reduce<<<128 * 512 / 256, 256, 0, s>>>(a.part, n_chunks, a.wc);
  if (hipError_t e = hipGetLastError()) return e;
  // attn[h] = v_b[h] (128 x 512) . wc[h]
  return launch_mv_f16_heads(a.v_b, a.wc, 512, a.attn, 128, 128, 512, s);
}

}  // namespace fdm
