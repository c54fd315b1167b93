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
//   YaRN RoPE of q_rope and k_rope at pos, cache append, and
//   Q_abs[h] = k_b[h] . q_nope[h]  [128][512]           k_mla_prep (one launch)
//   per 64-position chunk c and 16 heads: scores = scale (Q_abs[h].c_kv[s]
//     + q_rope[h].k_rope[s]), the chunk's max m_c, p = exp(score - m_c),
//     l_c = sum p, part_c[h] = sum_s p c_kv[s]       k_mla_attn_part
//   wc[h] = sum_c e^(m_c - M) part_c[h] / sum_c e^(m_c - M) l_c (the softmax
//     weighted latent sum), attn[h] = v_b[h] . wc[h]  k_mla_combine_vb
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
__device__ __forceinline__ void mv_f16_heads(const uint16_t* __restrict__ W, const float* __restrict__ x,
                                             int x_stride, float* __restrict__ y, int heads, int rows_h, int cols,
                                             int block, int n_blocks) {
  const int lane = threadIdx.x & 63;
  const int lpr = cols / 8, rpw = 64 / lpr;  // lanes per row, rows per wave step
  const int sub = lane / lpr, l = lane % lpr;
  const int total = heads * rows_h;
  const int wave_g = (block * 256 + (int)threadIdx.x) >> 6;
  const int n_waves = (n_blocks * 256) >> 6;
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
constexpr int kRopeBlocks = (128 * 32 + 32 + 255) / 256;

__device__ __forceinline__ void mla_rope_append(float* __restrict__ q, const float* __restrict__ kv_a,
                                                const float* __restrict__ c_kv_n, const float* __restrict__ freq,
                                                int pos, float* __restrict__ cache_c, float* __restrict__ cache_k,
                                                int len, int block) {
  const int t = block * 256 + (int)threadIdx.x;  // pair index
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

// The first kRopeBlocks workgroups: RoPE and the cache append; the rest:
// Q_abs[h] = k_b[h] (512 x 128) . q_nope[h] (q_nope is not rotated, so the two
// are independent and share one launch).
__global__ __launch_bounds__(256) void k_mla_prep(float* __restrict__ q, const float* __restrict__ kv_a,
                                                  const float* __restrict__ c_kv_n, const float* __restrict__ freq,
                                                  int pos, float* __restrict__ cache_c, float* __restrict__ cache_k,
                                                  int len, const uint16_t* __restrict__ k_b,
                                                  float* __restrict__ q_abs) {
  if ((int)blockIdx.x < kRopeBlocks)
    mla_rope_append(q, kv_a, c_kv_n, freq, pos, cache_c, cache_k, len, blockIdx.x);
  else
    mv_f16_heads(k_b, q, 192, q_abs, 128, 512, 128, (int)blockIdx.x - kRopeBlocks, (int)gridDim.x - kRopeBlocks);
}

// fp32 MFMA step (v_mfma_f32_16x16x4f32: fp32 products, fp32 accumulation, as
// the reference's sgemm calls).
__device__ __forceinline__ f32x4 mfma_f32x4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ---- scores, softmax and the weighted latent sum in one pass ----------------------------
// Flash-decoding over chunks of 64 cache positions (infer.m:829-867, the
// softmax of 385-389 taken apart per chunk and put back together exactly as
// a rescaled sum).  One workgroup per (chunk c, 16 heads):
//   1. scores of its 16 heads x 64 positions on fp32 MFMA (one 16 x 16 tile
//      per wave, as the scores of the two sgemm calls: scale (Q_abs . c_kv)
//      + scale (q_rope . k_rope)) into LDS;
//   2. per head: the chunk's max m_c, p = exp(score - m_c), l_c = sum p;
//   3. part[c][h][d] = sum_s p[h][s] c_kv[s][d] over the chunk on fp32 MFMA
//      (heads as rows, 16 latent dims per tile, 8 tiles per wave),
// and writes (m_c, l_c) for each head.  k_mla_combine_vb then merges the
// chunks: wc = sum_c exp(m_c - M) part_c / sum_c exp(m_c - M) l_c.  (Splitting
// the 512 dims over four workgroups, each recomputing the chunk's scores,
// measured slower: the scores' latent reads quadruple.)
constexpr int kMlaPos = 64;  // cache positions per chunk

__global__ __launch_bounds__(256) void k_mla_attn_part(const float* __restrict__ q_abs, const float* __restrict__ q,
                                                       const float* __restrict__ cache_c,
                                                       const float* __restrict__ cache_k, int S, float scale,
                                                       float* __restrict__ part, float* __restrict__ stat) {
  __shared__ float ps[16][kMlaPos + 1];  // scores, then p (row = head)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q4 = lane >> 4;
  const int c = blockIdx.x, h0 = 16 * blockIdx.y;
  const int base = c * kMlaPos;
  // 1. scores of positions base + 16 wave .. + 15
  {
    const int s0 = base + 16 * wave;
    const int sp = min(s0 + r, S - 1);  // past the cache: a valid row, result not kept
    const float* qa = q_abs + (size_t)(h0 + r) * 512 + 4 * q4;
    const float* cc = cache_c + (size_t)sp * 512 + 4 * q4;
    const float* qr = q + (size_t)(h0 + r) * 192 + 128 + 4 * q4;
    const float* kr = cache_k + (size_t)sp * 64 + 4 * q4;
    f32x4 a[4], b[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) a[e] = b[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // two stages of 16 steps, each stage's 32 loads issued before its MFMAs
    // (the latency of a load is paid per stage, not per step); the rope
    // part's loads go out with the first stage
    f32x4 kx[4], ky[4];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      f32x4 x[16], y[16];
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        x[m] = *reinterpret_cast<const f32x4*>(qa + 16 * (16 * half + m));
        y[m] = *reinterpret_cast<const f32x4*>(cc + 16 * (16 * half + m));
      }
      if (half == 0) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          kx[m] = *reinterpret_cast<const f32x4*>(qr + 16 * m);
          ky[m] = *reinterpret_cast<const f32x4*>(kr + 16 * m);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int m = 0; m < 16; ++m)
#pragma unroll
        for (int e = 0; e < 4; ++e) a[e] = mfma_f32x4(x[m][e], y[m][e], a[e]);
    }
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int e = 0; e < 4; ++e) b[e] = mfma_f32x4(kx[m][e], ky[m][e], b[e]);
    // D: lane l holds heads h0 + 4 (l / 16) + v, position s0 + l % 16
    const bool in = s0 + r < S;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float av = (a[0][v] + a[1][v]) + (a[2][v] + a[3][v]);
      const float bv = (b[0][v] + b[1][v]) + (b[2][v] + b[3][v]);
      ps[4 * q4 + v][16 * wave + r] = in ? scale * av + scale * bv : -__builtin_inff();
    }
  }
  __syncthreads();
  // 2. per head (16 threads each, 4 positions per thread): max, exp, sum
  {
    const int h = threadIdx.x >> 4, j = threadIdx.x & 15;
    float m = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < 4; ++k) m = fmaxf(m, ps[h][4 * j + k]);
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    float l = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float e = expf(ps[h][4 * j + k] - m);  // positions past the cache: exp(-inf) = 0
      ps[h][4 * j + k] = e;
      l += e;
    }
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) l += __shfl_xor(l, o);
    if (j == 0) {
      stat[((size_t)c * 128 + h0 + h) * 2] = m;
      stat[((size_t)c * 128 + h0 + h) * 2 + 1] = l;
    }
  }
  __syncthreads();
  // 3. the chunk's weighted latent sums: wave w takes dim tiles w, w + 4, ...
  //    (step e of a group of 16 positions takes from lane l the position
  //    16 g + 4 (l / 16) + e), in two stages of four tiles whose 64 loads
  //    are issued before their MFMAs.  Positions past the cache read the
  //    last row (finite) against p = 0.
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    float y[4][kMlaPos / 16][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d0 = 16 * (wave + 4 * (4 * st + i));
#pragma unroll
      for (int g = 0; g < kMlaPos / 16; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int sidx = min(base + 16 * g + 4 * q4 + e, S - 1);
          y[i][g][e] = cache_c[(size_t)sidx * 512 + d0 + r];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d0 = 16 * (wave + 4 * (4 * st + i));
      f32x4 acc[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int g = 0; g < kMlaPos / 16; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = mfma_f32x4(ps[r][16 * g + 4 * q4 + e], y[i][g][e], acc[e]);
#pragma unroll
      for (int v = 0; v < 4; ++v)
        part[((size_t)c * 128 + h0 + 4 * q4 + v) * 512 + d0 + r] = (acc[0][v] + acc[1][v]) + (acc[2][v] + acc[3][v]);
    }
  }
}

// Per (head h, quarter of its v_b rows): the chunks merged,
//   M = max_c m_c,  L = sum_c exp(m_c - M) l_c,
//   wc[d] = (sum_c exp(m_c - M) part[c][h][d]) / L   (512 dims in LDS),
// then attn[h][r] = v_b[h][r] . wc for the quarter's 32 rows (infer.m:868-873).
__global__ __launch_bounds__(256) void k_mla_combine_vb(const float* __restrict__ part, const float* __restrict__ stat,
                                                        int n_chunks, const uint16_t* __restrict__ v_b,
                                                        float* __restrict__ wc_out, float* __restrict__ attn) {
  __shared__ float al[1024];  // exp(m_c - M) per chunk (n_chunks <= 1024)
  __shared__ float wcs[512];
  __shared__ float red[4];
  __shared__ float stat_m, stat_l;
  const int h = blockIdx.x >> 2, quarter = blockIdx.x & 3;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // the quarter's 32 rows of v_b[h] first (independent of the merge): wave w
  // takes rows 8 w .. 8 w + 7, one 16-byte load per lane per row
  const int r0 = 32 * quarter + 8 * wave;
  u32x4 w[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    w[i] = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4*>(v_b + ((size_t)h * 128 + r0 + i) * 512 + 8 * lane));
  float m = -__builtin_inff();
  for (int c = threadIdx.x; c < n_chunks; c += 256) m = fmaxf(m, stat[((size_t)c * 128 + h) * 2]);
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  if (lane == 0) red[wave] = m;
  __syncthreads();
  if (threadIdx.x == 0) stat_m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  m = stat_m;
  float l = 0.0f;
  for (int c = threadIdx.x; c < n_chunks; c += 256) {
    const float a = expf(stat[((size_t)c * 128 + h) * 2] - m);
    al[c] = a;
    l += a * stat[((size_t)c * 128 + h) * 2 + 1];
  }
  l = lane_sum(l, 64);
  __syncthreads();
  if (lane == 0) red[wave] = l;
  __syncthreads();
  if (threadIdx.x == 0) stat_l = 1.0f / ((red[0] + red[1]) + (red[2] + red[3]));
  __syncthreads();
  const float inv = stat_l;
  for (int d = threadIdx.x; d < 512; d += 256) {
    float a = 0.0f;
    int c = 0;
    for (; c + 8 <= n_chunks; c += 8) {  // eight loads in flight, then the fma chain in chunk order
      float pv[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) pv[k] = part[((size_t)(c + k) * 128 + h) * 512 + d];
#pragma unroll
      for (int k = 0; k < 8; ++k) a = fmaf(al[c + k], pv[k], a);
    }
    for (; c < n_chunks; ++c) a = fmaf(al[c], part[((size_t)c * 128 + h) * 512 + d], a);
    const float v = a * inv;
    wcs[d] = v;
    if (quarter == 0 && wc_out) wc_out[(size_t)h * 512 + d] = v;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float acc = wave_sum_lane0(mv_dot8(w[i], wcs + 8 * lane, 0.0f));
    if (lane == 0) attn[(size_t)h * 128 + r0 + i] = acc;
  }
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

hipError_t launch_mla_attend(const MlaArgs& a, hipStream_t s) {
  // RoPE + append, and Q_abs[h] = k_b[h] (512 x 128) . q_nope[h]: 16 lanes
  // per row, 4 rows per wave step, up to 4 workgroups per CU
  {
    const int waves = 128 * 512 / 4;
    const int wgs = min((waves + 3) / 4, 4 * g_num_cus);
    k_mla_prep<<<kRopeBlocks + wgs, 256, 0, s>>>(a.q, a.kv_a, a.c_kv_n, a.freq, a.pos, a.cache_c, a.cache_k, a.len,
                                                a.k_b, a.q_abs);
    if (hipError_t e = hipGetLastError()) return e;
  }
  const int S = a.len + 1;
  const int n_chunks = (S + kMlaPos - 1) / kMlaPos;
  if (n_chunks > 1024) return hipErrorInvalidValue;  // k_mla_combine_vb holds <= 1024 chunk weights
  k_mla_attn_part<<<dim3(n_chunks, 128 / 16), 256, 0, s>>>(a.q_abs, a.q, a.cache_c, a.cache_k, S, a.scale, a.part,
                                                           a.stat);
  if (hipError_t e = hipGetLastError()) return e;
  k_mla_combine_vb<<<128 * 4, 256, 0, s>>>(a.part, a.stat, n_chunks, a.v_b, a.wc, a.attn);
  return hipGetLastError();
}

}  // namespace fdm
