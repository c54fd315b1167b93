// attn_kernels.hip -- MLA attention of one decode token (mla_forward,
// infer.m:766-903) on the device, with the weights in the layout the
// reference holds them (LayerAttnDense, infer.m:687-706: F16 row-major;
// k_b per head (KV_LORA, NOPE), v_b per head (V_HEAD, KV_LORA)) and the
// latent KV cache in fp32 (MLACache, infer.m:663-669).
//
// Launch sequence of one token (fdm_attn_forward):
//   [q_a; kv_a] = [W_qa; W_kva] . (hidden * attn_norm)  [1536 + 576], and the
//     attention norm's exact 1 / rms beside it             k_mv_f16_xw
//   q = W_qb . rms_norm(q_a * inv, q_a_norm)  [128][192]  k_mv_f16_rn
//     (the q_a norm bit-exact, computed in every workgroup)
//   c_kv[len] = rms_norm(kv_a[:512] * inv, kv_a_norm); YaRN RoPE of q_rope
//     and k_rope at pos into k_rope[len]; Q_abs[h] = k_b[h] . q_nope[h]
//     [128][512]                                            k_mla_prep (one launch)
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
#include "rms_device.h"

namespace fdm {

namespace {

constexpr int kMvChunk = 512;   // halves per wave load
constexpr int kMvBatch = 8;     // loads in flight per wave
constexpr int kMvWaves = 4;
constexpr int kMvMaxCols = 16384;  // o_proj input: 128 heads x 128
constexpr int kMvWideWaves = 6;    // waves per workgroup for rows wider than 8192 (o_proj)

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
// cols <= 16384.  One wave per row (grid-stride), WV waves per workgroup
// sharing x staged in LDS (cols floats of dynamic LDS: the narrow
// projections keep more workgroups per CU than a fixed 64 KB would allow),
// NB 1 KB loads in flight per wave.
template <int WV, int NB>
__global__ __launch_bounds__(WV * 64) void k_mv_f16(const uint16_t* __restrict__ W, const float* __restrict__ x,
                                                    const float* __restrict__ res, float* __restrict__ y, int rows,
                                                    int cols) {
  extern __shared__ float xs[];  // cols floats
  for (int i = threadIdx.x; i < cols / 4; i += blockDim.x)
    reinterpret_cast<f32x4*>(xs)[i] = reinterpret_cast<const f32x4*>(x)[i];
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_waves = gridDim.x * WV, chunks = cols / kMvChunk;
  for (int r = blockIdx.x * WV + wave; r < rows; r += n_waves) {
    const uint16_t* wr = W + (size_t)r * cols + 8 * lane;
    float acc = 0.0f;
    for (int b = 0; b < chunks; b += NB) {
      u32x4 w[NB];
#pragma unroll
      for (int i = 0; i < NB; ++i)
        if (b + i < chunks) w[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + (b + i) * kMvChunk));
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < NB; ++i)
        if (b + i < chunks) acc = mv_dot8(w[i], xs + (b + i) * kMvChunk + 8 * lane, acc);
    }
    acc = wave_sum_lane0(acc);  // the butterfly's lane-0 sum, VALU only
    if (lane == 0) y[r] = (res ? res[r] : 0.0f) + acc;
  }
}

// The projections whose input is an rms_norm, without a launch of their own
// for the norm:
//   [q_a; kv_a] (k_mv_f16_xw): y[r] = W[r] . (x * nw), the attention norm's
//     weights applied and its 1 / rms not yet: workgroup 0 computes it
//     (rms_norm_inv, the reference's float chain bit for bit) into *inv
//     while the others contract the rows, one row per wave with its 14
//     loads issued at once; nothing waits;
//   q_b (k_mv_f16_rn): y[r] = W[r] . rms_norm(x * xmul, nw), xmul = *inv of
//     the launch before (the raw q_a times the scale it owes): every
//     workgroup requests its waves' first PF rows, computes the exact q_a
//     norm itself while they land, stages ((x * xmul) * inv) * nw in LDS
//     and contracts the rows as k_mv_f16 does, each consumed row's slot
//     refilled with the wave's row PF ahead.
// q_a = inv * (W . (x nw)) differs from the reference's W . ((x inv) nw)
// by the rounding of the scale's place (a few ulps of q_a).
__global__ __launch_bounds__(kMvWaves * 64) void k_mv_f16_xw(const uint16_t* __restrict__ W,
                                                             const float* __restrict__ x,
                                                             const float* __restrict__ nw,
                                                             float* __restrict__ y, int rows,
                                                             float* __restrict__ inv) {
  constexpr int NT = kHidden / kMvChunk;
  __shared__ RmsSmem sm;
  if (blockIdx.x == 0) {
    const float v = rms_norm_inv(x, kHidden, sm);
    if (threadIdx.x == 0) *inv = v;
    return;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_waves = (gridDim.x - 1) * kMvWaves;
  const int r0 = (blockIdx.x - 1) * kMvWaves + wave;
  u32x4 w[NT];
  auto load_row = [&](int r) {
    const uint16_t* wr = W + (size_t)min(r, rows - 1) * kHidden + 8 * lane;  // past the last row: not kept
#pragma unroll
    for (int i = 0; i < NT; ++i) w[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + i * kMvChunk));
  };
  // x and nw (28 KB each, L2 hits after the first workgroups) are requested
  // before the row, so they return first and are staged while the row's
  // loads are in flight (the registers are free: workgroup 0's norm sets
  // the kernel's VGPR count)
  constexpr int kXv = kHidden / 4 / (kMvWaves * 64);  // 7 float4s per thread
  f32x4 xv[kXv], nv[kXv];
#pragma unroll
  for (int k = 0; k < kXv; ++k) {
    xv[k] = reinterpret_cast<const f32x4*>(x)[threadIdx.x + kMvWaves * 64 * k];
    nv[k] = reinterpret_cast<const f32x4*>(nw)[threadIdx.x + kMvWaves * 64 * k];
  }
  load_row(r0);
  f32x4* xs = reinterpret_cast<f32x4*>(sm.k);
#pragma unroll
  for (int k = 0; k < kXv; ++k) xs[threadIdx.x + kMvWaves * 64 * k] = xv[k] * nv[k];
  __syncthreads();
  for (int r = r0; r < rows; r += n_waves) {
    if (r != r0) load_row(r);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < NT; ++i) acc = mv_dot8(w[i], reinterpret_cast<const float*>(sm.k) + i * kMvChunk + 8 * lane, acc);
    acc = wave_sum_lane0(acc);
    if (lane == 0) y[r] = acc;
  }
}

template <int D, int PF>
__global__ __launch_bounds__(kMvWaves * 64) void k_mv_f16_rn(const uint16_t* __restrict__ W,
                                                             const float* __restrict__ x,
                                                             const float* __restrict__ xmul,
                                                             const float* __restrict__ nw,
                                                             float* __restrict__ y, int rows) {
  constexpr int NT = D / kMvChunk;
  __shared__ RmsSmem sm;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_waves = gridDim.x * kMvWaves;
  const int r0 = blockIdx.x * kMvWaves + wave;
  auto load_row = [&](u32x4 (&w)[NT], int r) {
    const uint16_t* wr = W + (size_t)min(r, rows - 1) * D + 8 * lane;  // past the last row: a valid one, not kept
#pragma unroll
    for (int i = 0; i < NT; ++i) w[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + i * kMvChunk));
  };
  u32x4 w[PF][NT];
#pragma unroll
  for (int k = 0; k < PF; ++k) load_row(w[k], r0 + k * n_waves);
  const float mul = *xmul;
  const float inv = rms_norm_inv(x, D, sm, mul);
  __syncthreads();  // the norm's LDS is free
  float* xs = reinterpret_cast<float*>(sm.k);
  for (int i = threadIdx.x; i < D; i += kMvWaves * 64) xs[i] = ((x[i] * mul) * inv) * nw[i];
  __syncthreads();
  for (int r = r0; r < rows; r += PF * n_waves) {
#pragma unroll
    for (int k = 0; k < PF; ++k) {
      const int rk = r + k * n_waves;
      if (rk < rows) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < NT; ++i) acc = mv_dot8(w[k][i], xs + i * kMvChunk + 8 * lane, acc);
        acc = wave_sum_lane0(acc);
        if (lane == 0) y[rk] = acc;
      }
      if (rk + PF * n_waves < rows) load_row(w[k], rk + PF * n_waves);
    }
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
// freq[i] the layer's table of yarn_freq(i), into the token's cache row
// k_rope[len] (pair blocks); the latent row c_kv[len] = rms_norm(kv_a[:512],
// kv_a_norm) by the norm block (rms_norm_row: bit-exact).  kv_a is the raw
// projection of k_mv_f16_xw: kv_a * (*kv_scale) its values.
constexpr int kRopeBlocks = (128 * 32 + 32 + 255) / 256;

__device__ __forceinline__ void mla_rope(float* __restrict__ q, const float* __restrict__ kv_a, float kv_mul,
                                         const float* __restrict__ freq, int pos, float* __restrict__ cache_k,
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
      const float a = kv_a[512 + 2 * i] * kv_mul, b = kv_a[512 + 2 * i + 1] * kv_mul;
      cache_k[(size_t)len * 64 + 2 * i] = a * c - b * s;
      cache_k[(size_t)len * 64 + 2 * i + 1] = a * s + b * c;
    }
  }
}

// Workgroup 0: the latent norm and its cache row; the next kRopeBlocks:
// RoPE; the rest: Q_abs[h] = k_b[h] (512 x 128) . q_nope[h] (q_nope is not
// rotated, so all three are independent and share one launch).
__global__ __launch_bounds__(256) void k_mla_prep(float* __restrict__ q, const float* __restrict__ kv_a,
                                                  const float* __restrict__ kv_scale,
                                                  const float* __restrict__ kv_a_norm,
                                                  const float* __restrict__ freq, int pos,
                                                  float* __restrict__ cache_c, float* __restrict__ cache_k, int len,
                                                  const uint16_t* __restrict__ k_b, float* __restrict__ q_abs) {
  __shared__ RmsSmem sm;
  if (blockIdx.x == 0)
    rms_norm_row(kv_a, kv_a_norm, cache_c + (size_t)len * 512, 512, sm, *kv_scale);
  else if ((int)blockIdx.x <= kRopeBlocks)
    mla_rope(q, kv_a, *kv_scale, freq, pos, cache_k, len, (int)blockIdx.x - 1);
  else
    mv_f16_heads(k_b, q, 192, q_abs, 128, 512, 128, (int)blockIdx.x - 1 - kRopeBlocks,
                 (int)gridDim.x - 1 - kRopeBlocks);
}

// fp32 MFMA step (v_mfma_f32_16x16x4f32: fp32 products, fp32 accumulation, as
// the reference's sgemm calls).
__device__ __forceinline__ f32x4 mfma_f32x4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ---- scores, softmax and the weighted latent sum in one pass ----------------------------
// Flash-decoding over chunks of POS cache positions (infer.m:829-867, the
// softmax of 385-389 taken apart per chunk and put back together exactly as
// a rescaled sum).  One workgroup of 8 waves per (chunk c, 16 heads):
//   1. scores of its 16 heads x POS positions on fp32 MFMA (16 x 16 tiles;
//      the 512 latent dims of a tile split over 8 / (POS / 16) waves, whose
//      partial sums are added in split order; the rope dims by the last
//      split's wave; scale (Q_abs . c_kv) + scale (q_rope . k_rope), the
//      two sgemm calls' sum) into LDS;
//   2. per head: the chunk's max m_c, p = exp(score - m_c), l_c = sum p;
//   3. part[c][h][d] = sum_s p[h][s] c_kv[s][d] over the chunk on fp32 MFMA
//      (heads as rows, 16 latent dims per tile, 4 tiles per wave, their
//      loads issued before the MFMAs),
// and writes (m_c, l_c) for each head.  k_mla_combine_vb then merges the
// chunks: wc = sum_c exp(m_c - M) part_c / sum_c exp(m_c - M) l_c.  Every
// stage's loads are in flight at once, so a workgroup pays about one load
// latency per stage; the chunk length sets how many workgroups share the
// cache (S / POS x 8).  (Splitting the 512 dims over four workgroups, each
// recomputing the chunk's scores, measured slower: the scores' latent reads
// quadruple.)
template <int POS>
__global__ __launch_bounds__(512) void k_mla_attn_part(const float* __restrict__ q_abs, const float* __restrict__ q,
                                                       const float* __restrict__ cache_c,
                                                       const float* __restrict__ cache_k, int S, float scale,
                                                       float* __restrict__ part, float* __restrict__ stat) {
  constexpr int PT = POS / 16;  // position tiles
  constexpr int KS = 8 / PT;    // latent splits per tile
  constexpr int MS = 32 / KS;   // 16-dim steps per split
  static_assert(PT * KS == 8 && MS * KS == 32, "8 waves cover the tiles and splits");
  __shared__ float sp[KS][16][POS + 1];  // latent partial scores per split (row = head)
  __shared__ float sr[16][POS + 1];      // rope scores
  __shared__ float ps[16][POS + 1];      // p
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q4 = lane >> 4;
  const int c = blockIdx.x, h0 = 16 * blockIdx.y;
  const int base = c * POS;
  // 1. partial scores of positions base + 16 tile .. + 15, dims 16 MS ks ..
  {
    const int tile = wave % PT, ks = wave / PT;
    const bool rope = ks == KS - 1;
    const int s0 = base + 16 * tile;
    const int sp_row = min(s0 + r, S - 1);  // past the cache: a valid row, result not kept
    const float* qa = q_abs + (size_t)(h0 + r) * 512 + 16 * MS * ks + 4 * q4;
    const float* cc = cache_c + (size_t)sp_row * 512 + 16 * MS * ks + 4 * q4;
    const float* qr = q + (size_t)(h0 + r) * 192 + 128 + 4 * q4;
    const float* kr = cache_k + (size_t)sp_row * 64 + 4 * q4;
    f32x4 x[MS], y[MS], kx[4], ky[4];
#pragma unroll
    for (int m = 0; m < MS; ++m) {
      x[m] = *reinterpret_cast<const f32x4*>(qa + 16 * m);
      y[m] = *reinterpret_cast<const f32x4*>(cc + 16 * m);
    }
    if (rope) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        kx[m] = *reinterpret_cast<const f32x4*>(qr + 16 * m);
        ky[m] = *reinterpret_cast<const f32x4*>(kr + 16 * m);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    f32x4 a[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) a[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int m = 0; m < MS; ++m)
#pragma unroll
      for (int e = 0; e < 4; ++e) a[e] = mfma_f32x4(x[m][e], y[m][e], a[e]);
    // D: lane l holds heads 4 (l / 16) + v, position s0 + l % 16
#pragma unroll
    for (int v = 0; v < 4; ++v) sp[ks][4 * q4 + v][16 * tile + r] = (a[0][v] + a[1][v]) + (a[2][v] + a[3][v]);
    if (rope) {
      f32x4 b[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) b[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int e = 0; e < 4; ++e) b[e] = mfma_f32x4(kx[m][e], ky[m][e], b[e]);
#pragma unroll
      for (int v = 0; v < 4; ++v) sr[4 * q4 + v][16 * tile + r] = (b[0][v] + b[1][v]) + (b[2][v] + b[3][v]);
    }
  }
  __syncthreads();
  // 2. per head (16 threads each, POS / 16 positions per thread): the
  //    scores, max, exp, sum
  if (threadIdx.x < 256) {
    constexpr int PP = POS / 16;
    const int h = threadIdx.x >> 4, j = threadIdx.x & 15;
    float sc[PP];
    float m = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < PP; ++k) {
      const int p = PP * j + k;
      float lat = sp[0][h][p];
#pragma unroll
      for (int t = 1; t < KS; ++t) lat += sp[t][h][p];
      sc[k] = base + p < S ? scale * lat + scale * sr[h][p] : -__builtin_inff();
      m = fmaxf(m, sc[k]);
    }
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    float l = 0.0f;
#pragma unroll
    for (int k = 0; k < PP; ++k) {
      const float e = expf(sc[k] - m);  // positions past the cache: exp(-inf) = 0
      ps[h][PP * j + k] = e;
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
  // 3. the chunk's weighted latent sums: wave w takes dim tiles w, w + 8,
  //    w + 16, w + 24 (step e of a group of 16 positions takes from lane l
  //    the position 16 g + 4 (l / 16) + e).  Positions past the cache read
  //    the last row (finite) against p = 0.
  float y[4][PT][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d0 = 16 * (wave + 8 * i);
#pragma unroll
    for (int g = 0; g < PT; ++g)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int sidx = min(base + 16 * g + 4 * q4 + e, S - 1);
        y[i][g][e] = cache_c[(size_t)sidx * 512 + d0 + r];
      }
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d0 = 16 * (wave + 8 * i);
    f32x4 acc[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int g = 0; g < PT; ++g)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = mfma_f32x4(ps[r][16 * g + 4 * q4 + e], y[i][g][e], acc[e]);
#pragma unroll
    for (int v = 0; v < 4; ++v)
      part[((size_t)c * 128 + h0 + 4 * q4 + v) * 512 + d0 + r] = (acc[0][v] + acc[1][v]) + (acc[2][v] + acc[3][v]);
  }
}

// Per (head h, quarter of its v_b rows): the chunks merged,
//   M = max_c m_c,  L = sum_c exp(m_c - M) l_c,
//   wc[d] = (sum_c exp(m_c - M) part[c][h][d]) / L   (512 dims in LDS),
// then attn[h][r] = v_b[h][r] . wc for the quarter's 32 rows (infer.m:868-873).
// With PRE > 0 (at most PRE chunks) every load the workgroup needs -- its
// v_b rows, its head's part values of every chunk, the chunk statistics --
// is issued at dispatch and the merge takes one barrier; with PRE = 0
// (longer caches) the chunks are walked in batches of eight.
template <int PRE>
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
  if constexpr (PRE > 0) {
    // dims threadIdx.x and threadIdx.x + 256 of every chunk (a chunk past
    // the last reads the last one and is not summed)
    float pv[2][PRE];
#pragma unroll
    for (int c = 0; c < PRE; ++c) {
      const size_t at = ((size_t)min(c, n_chunks - 1) * 128 + h) * 512 + threadIdx.x;
      pv[0][c] = part[at];
      pv[1][c] = part[at + 256];
    }
    if (wave == 0) {  // lane c: chunk c
      const bool live = lane < n_chunks;
      const float mc = live ? stat[((size_t)lane * 128 + h) * 2] : -__builtin_inff();
      const float lc = live ? stat[((size_t)lane * 128 + h) * 2 + 1] : 0.0f;
      float m = mc;
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
      const float a = live ? expf(mc - m) : 0.0f;
      const float l = lane_sum(a * lc, 64);
      if (live) al[lane] = a;
      if (lane == 0) stat_l = 1.0f / l;
    }
    __syncthreads();
    const float inv = stat_l;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      float a = 0.0f;
#pragma unroll
      for (int c = 0; c < PRE; ++c)
        if (c < n_chunks) a = fmaf(al[c], pv[k][c], a);  // chunk order, as the batched walk below
      const int d = threadIdx.x + 256 * k;
      const float v = a * inv;
      wcs[d] = v;
      if (quarter == 0 && wc_out) wc_out[(size_t)h * 512 + d] = v;
    }
  } else {
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
  if (cols > 8192) {
    // o_proj: 64 KB of x allow two workgroups per CU; six waves each share
    // it (measured 97.0-97.3 against 97.6-97.7 us per token with four; five,
    // seven, or sixteen loads in flight no better)
    constexpr int WV = kMvWideWaves;
    const int wgs = min((rows + WV - 1) / WV, per_cu * g_num_cus);
    k_mv_f16<WV, kMvBatch><<<wgs, WV * 64, lds, s>>>(W, x, res, y, rows, cols);
  } else {
    const int wgs = min((rows + kMvWaves - 1) / kMvWaves, per_cu * g_num_cus);
    k_mv_f16<kMvWaves, kMvBatch><<<wgs, kMvWaves * 64, lds, s>>>(W, x, res, y, rows, cols);
  }
  return hipGetLastError();
}

hipError_t launch_mv_f16_xw(const uint16_t* W, const float* x, const float* nw, float* y, int rows, float* inv,
                            hipStream_t s) {
  // the norm workgroup, then as many row workgroups as are resident at once
  // (36 KB of LDS; 176 VGPRs with a row in flight: 2 per CU)
  const int wgs = 1 + min((rows + kMvWaves - 1) / kMvWaves, 2 * g_num_cus - 1);
  k_mv_f16_xw<<<wgs, kMvWaves * 64, 0, s>>>(W, x, nw, y, rows, inv);
  return hipGetLastError();
}

hipError_t launch_mv_f16_rn(const uint16_t* W, const float* x, const float* xmul, const float* nw, float* y, int rows,
                            int cols, hipStream_t s) {
  // as many workgroups as are resident at once (36 KB of LDS, 102 VGPRs)
  if (cols != 1536) return hipErrorInvalidValue;
  k_mv_f16_rn<1536, 4><<<min((rows + kMvWaves - 1) / kMvWaves, 4 * g_num_cus), kMvWaves * 64, 0, s>>>(W, x, xmul, nw,
                                                                                                     y, rows);
  return hipGetLastError();
}

hipError_t launch_mla_attend(const MlaArgs& a, hipStream_t s) {
  // RoPE + append, and Q_abs[h] = k_b[h] (512 x 128) . q_nope[h]: 16 lanes
  // per row, 4 rows per wave step, up to 4 workgroups per CU
  {
    const int waves = 128 * 512 / 4;
    const int wgs = min((waves + 3) / 4, 4 * g_num_cus);
    k_mla_prep<<<1 + kRopeBlocks + wgs, 256, 0, s>>>(a.q, a.kv_a, a.kv_scale, a.kv_a_norm, a.freq, a.pos, a.cache_c,
                                                    a.cache_k, a.len, a.k_b, a.q_abs);
    if (hipError_t e = hipGetLastError()) return e;
  }
  const int S = a.len + 1;
  const int n_chunks = (S + kMlaChunkPos - 1) / kMlaChunkPos;
  if (n_chunks > 1024) return hipErrorInvalidValue;  // k_mla_combine_vb holds <= 1024 chunk weights
  k_mla_attn_part<kMlaChunkPos><<<dim3(n_chunks, 128 / 16), 512, 0, s>>>(a.q_abs, a.q, a.cache_c, a.cache_k, S,
                                                                         a.scale, a.part, a.stat);
  if (hipError_t e = hipGetLastError()) return e;
  if (n_chunks <= 16)
    k_mla_combine_vb<16><<<128 * 4, 256, 0, s>>>(a.part, a.stat, n_chunks, a.v_b, a.wc, a.attn);
  else if (n_chunks <= 32)
    k_mla_combine_vb<32><<<128 * 4, 256, 0, s>>>(a.part, a.stat, n_chunks, a.v_b, a.wc, a.attn);
  else
    k_mla_combine_vb<0><<<128 * 4, 256, 0, s>>>(a.part, a.stat, n_chunks, a.v_b, a.wc, a.attn);
  return hipGetLastError();
}

}  // namespace fdm
