// gemm_kernels.hip -- the grouped expert GEMMs of batched decode and prefill
// on MFMA: per distinct expert (and the shared one), its tokens' activations
// against the expert's Q4_K rows, for gate/up (+ SwiGLU) and for a Q4_K down.
//
// Numerics.  Inside one Q4_K block a weight is d*sc*q - dmin*m (quant.c:49-57)
// with 6-bit sc, m and 4-bit q, so
//   sum_k w_k x_k = d * sum_k sc_k q_k x_k - dmin * sum_sb m_sb X_sb
// (X_sb: the sum of the sub-block's 32 activations).  The integer sc*q <= 945
// is exact in fp16 and is built per element pair by one mask-or and one
// packed fma: (0x6400 | q) is the half 1024 + q, and (1024 + q) sc - 1024 sc
// is sc q exactly (one rounding of an exact half).  The MFMA
// (v_mfma_f32_16x16x32_f16, fp32 accumulation) contracts it with the
// activations over a whole block and the scales are applied once per block:
//   y += d * C  -  sum_sb X_sb dmin m_sb
// the second term by a 16x16x4 fp32 MFMA over the block's eight sub-blocks.
// (Weights carried as 1024 + sc q, with 1024 X cancelled afterwards, would
// inflate the accumulator several times over the sum it carries and cost
// the batched path its fp32 grade on SwiGLU activations.)
// Activations enter as P fp16 planes of x' = x * 2^s (a per-row power of
// two: the largest |x'| lies in [2^13, 2^14)): P = 3 carries every fp32
// value exactly (hi + mid + lo, 33 significant bits) -- batched decode, fp32
// grade; P = 1 carries 11 bits -- prefill, whose bar is 1e-2.  X_sb is the
// fp32 sum of the planes' values.
//
// Mapping.  A workgroup of 4 waves owns 64 gate and 64 up rows (wave w:
// rows 16 w .. 16 w + 15 of both, so SwiGLU is applied in registers) or 128
// down rows (wave w: two tiles of 16) -- the three-plane gate/up GEMM twice
// that, 32 rows of gate and of up per wave -- for one chunk of <= 16 NB
// tokens of one expert.  Weight rows are the MFMA columns (B operand): lane (c, j)
// holds row c and group j (qs bytes 32 j .. 32 j + 31, sub-blocks 2j, 2j+1)
// of every block, read as two whole 16-byte pieces of the resident expert
// layout, so the four lanes of a row read one 64-byte line per load and
// each lane needs only its own group's two scales and mins.  MFMA step m
// (0..7) of a block takes from lane j the 8 elements 64 j + 8 m .. + 7 (low
// nibbles for m < 4, high nibbles for m >= 4); the token operand (A, from
// LDS) reads the same elements.  Per block the chunk's token planes are
// copied global -> LDS by direct loads into one of two buffers, so block
// b + 1 streams in while block b is contracted.
#include "fdm_internal.h"
#include "planes_device.h"

namespace fdm {

namespace {

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kQWaves = 4;            // waves per workgroup
constexpr int kQRowB = kQK * 2;       // LDS token row: one block of fp16 (512 B)
// Weight tiles of 16 rows per wave (TL): a gate/up GEMM holds TL / 2 tiles of
// gate and as many of up (SwiGLU pairs tile t with tile t + TL / 2), a down
// GEMM TL tiles; every token operand read from LDS serves all of them.  Four
// tiles for the fp32-grade gate/up (three planes: twice the weights per token
// operand read, 252 VGPRs), two elsewhere (168 VGPRs for the three-plane down:
// 3 waves per SIMD; 213-229 for one plane: 2 waves per SIMD, no spills).
__host__ __device__ constexpr int qgemm_tiles(int planes, bool down) { return (planes == 3 && !down) ? 4 : 2; }
__host__ __device__ constexpr int qgemm_rows(int tiles, bool down) {  // rows per workgroup (of gate for gate/up)
  return (down ? 16 : 8) * tiles * kQWaves;
}

// One lane's share of one block of one weight row (resident expert layout):
// its group's 32 qs bytes and the 16-byte block header.
struct QLane {
  u32x4 q0, q1, hdr;
};

// A block's q0 (and q1) pieces of a row pair (gate / up) or quad (down) fill
// whole 128-byte lines of the resident layout, read once per chunk of the
// expert.  Odd blocks are read with the nontemporal policy, even ones with
// the default policy: measured a little faster than either policy for every
// block (the default lines stay in the L2 for the expert's other chunks,
// the streamed half leaves room).
template <bool DOWN, bool LAST>
__device__ __forceinline__ QLane qlane_load(const uint8_t* mat, int row, int block, int j) {
  constexpr int N = DOWN ? kRelDnPieces : kRelGuPieces;
  const uint8_t* st = rel_step<DOWN>(mat, row, block);
  const int L0 = rel_piece<DOWN>(row, block, 0);
  const u32x4* p0 = reinterpret_cast<const u32x4*>(st + 16 * (L0 + j));
  const u32x4* p1 = reinterpret_cast<const u32x4*>(st + 16 * N + 16 * (L0 + j));
  QLane r;
  if (LAST) {
    r.q0 = __builtin_nontemporal_load(p0);
    r.q1 = __builtin_nontemporal_load(p1);
  } else {
    r.q0 = *p0;
    r.q1 = *p1;
  }
  r.hdr = *reinterpret_cast<const u32x4*>(st + 32 * N + 4 * L0);
  return r;
}

// fp16 halves of sc * q for the two q held in bits 0-3 (MASK 0x000F000F)
// of the halves of w, the rest of w arbitrary: 0x6400 | q is the half
// 1024 + q, and one fused multiply-add per half, (1024 + q) sc - 1024 sc,
// gives sc q exactly (q < 16, sc < 64: the exact result is a half, which the
// single rounding keeps).  For the q in bits 4-7 (MASK 0x00F000F0),
// 0x6400 | 16 q is the half 1024 + 16 q, and (1024 + 16 q) (sc / 16) - 64 sc
// is sc q exactly, with no shift to bring the nibble down.  k holds the
// multiplier in its low half and the addend in its high half; both halves of
// the fma read them (op_sel).
template <uint32_t MASK>
__device__ __forceinline__ uint32_t magic2(uint32_t w, f16x2 k) {
  // one v_and_or_b32 (mask from an SGPR, 0x64006400 from a VGPR: a VOP3
  // takes no literal and one SGPR), which the compiler otherwise splits
  uint32_t m;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(m) : "v"(w), "s"(MASK), "v"(0x64006400u));
  const f16x2 v = __builtin_bit_cast(f16x2, m);
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(v, (f16x2){k.x, k.x}, (f16x2){k.y, k.y}));
}

// The B operands of MFMA steps m (low nibbles) and m + 4 (high nibbles):
// bytes 8 m' .. 8 m' + 7 of the lane's group, m' = m & 3 (q0 for m' < 2).
// Elements are taken in the order 0 2 1 3 4 6 5 7 of each 8 (the order in
// which k_xplanes stores the activations): a dword of qs holds the low
// nibbles of elements 0 and 2 at bits 0 and 16 and their high nibbles at
// bits 4 and 20, elements 1 and 3 eight bits higher, so one shift per dword
// and per fp16 pair one mask-or and one packed fma suffice.
struct BPair {
  f16x8 lo, hi;
};

__device__ __forceinline__ BPair build_b(uint32_t w0, uint32_t w1, f16x2 k_lo, f16x2 k_hi) {
  const uint32_t v0 = w0 >> 8, v1 = w1 >> 8;
  u32x4 lo, hi;
  lo.x = magic2<0x000F000Fu>(w0, k_lo);
  lo.y = magic2<0x000F000Fu>(v0, k_lo);
  lo.z = magic2<0x000F000Fu>(w1, k_lo);
  lo.w = magic2<0x000F000Fu>(v1, k_lo);
  hi.x = magic2<0x00F000F0u>(w0, k_hi);
  hi.y = magic2<0x00F000F0u>(v0, k_hi);
  hi.z = magic2<0x00F000F0u>(w1, k_hi);
  hi.w = magic2<0x00F000F0u>(v1, k_hi);
  BPair b;
  b.lo = __builtin_bit_cast(f16x8, lo);
  b.hi = __builtin_bit_cast(f16x8, hi);
  return b;
}

// Per-block constants of the lane's row and group.
struct QScale {
  float d;
  f16x2 k_lo;          // {sc, -1024 sc} of sub-block 2j
  f16x2 k_hi;          // {sc / 16, -64 sc} of sub-block 2j+1
  float bc_lo, bc_hi;  // -dmin m of sub-blocks 2j, 2j+1
};

__device__ __forceinline__ QScale qscale(const u32x4 hdr, const Q4KScaleSel& sel) {
  int sc0, m0, sc1, m1;
  q4k_scale_min_pair(hdr.y, hdr.z, hdr.w, sel, sc0, m0, sc1, m1);
  QScale s;
  s.d = half_to_float(hdr.x);
  const float dmin = half_to_float(hdr.x >> 16);
  // the halves 1024 + sc0 and 1024 + sc1, then {sc0, -1024 sc0} and
  // {sc1 / 16, -64 sc1}, all exact
  const f16x2 h = __builtin_bit_cast(f16x2, (uint32_t)sc0 + ((uint32_t)sc1 << 16) + 0x64006400u);
  const f16x2 k = __builtin_elementwise_fma(h, (f16x2){(_Float16)1.0f, (_Float16)0.0625f},
                                            (f16x2){(_Float16)-1024.0f, (_Float16)-64.0f});  // {sc0, sc1 / 16}
  s.k_lo = (f16x2){k.x, k.x * (_Float16)-1024.0f};
  s.k_hi = (f16x2){k.y, k.y * (_Float16)-1024.0f};
  s.bc_lo = -(dmin * (float)m0);
  s.bc_hi = -(dmin * (float)m1);
  return s;
}

__device__ __forceinline__ f32x4 mfma_h(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_f(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// One 16-byte direct global -> LDS load per lane (lane i writes lds_dst + 16 i).
__device__ __forceinline__ void lds_dma16(const void* gsrc, void* lds_dst) {
  __builtin_amdgcn_global_load_lds(gsrc, lds_dst, 16, 0, 0);
}

__device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

}  // namespace

// ---- activation planes ---------------------------------------------------------------
// Rows of KD fp32 into the planes (planes_device.h).  One thread per
// 32-element sub-block holds it in registers: the row is read once, its
// largest |x| reduced across the row's threads, then converted.  KD = 2048:
// one wave per row, four rows per workgroup; KD = 7168: one workgroup per
// row (224 of its 256 threads hold a sub-block).
template <int P, int KD>
__global__ __launch_bounds__(256) void k_xplanes(const float* __restrict__ x, size_t n_rows,
                                                 _Float16* __restrict__ xp, float* __restrict__ xs,
                                                 float* __restrict__ xe) {
  constexpr int NSB = KD / 32;
  constexpr int TPR = NSB <= 64 ? 64 : 256;  // threads per row
  static_assert(NSB * 32 == KD && NSB <= TPR, "sub-blocks of a row fit its threads");
  constexpr int RPB = 256 / TPR;
  __shared__ float red[4];
  const size_t row = (size_t)blockIdx.x * RPB + threadIdx.x / TPR;
  const int sb = threadIdx.x % TPR;
  const bool live = row < n_rows && sb < NSB;
  f32x4 v[8];
  float m = 0.0f;
  if (live) {
    const f32x4* src = reinterpret_cast<const f32x4*>(x + row * KD + 32 * sb);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = src[i];
    m = subblock_absmax(v);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  if constexpr (TPR == 256) {
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  }
  if (!live) return;
  const int s = planes_shift(m);
  if (sb == 0) xe[row] = ldexpf(1.0f, -s);
  xs[row * NSB + sb] = planes_subblock<P>(v, s, xp + row * KD + 32 * sb, n_rows * KD);
}

// ---- the grouped GEMM ------------------------------------------------------------------
template <int P, int NB, bool DOWN, int TL>
__device__ __forceinline__ void qgemm_body(const QGemmArgs& g, uint8_t* lds0, uint8_t* lds1, int* rows, int chunk, int rg) {
  constexpr int KD = DOWN ? kFfn : kHidden;  // contraction length
  constexpr int NBLK = KD / kQK;             // 8 or 28 (even)
  constexpr int NT = 16 * NB;                // token rows per buffer and plane
  constexpr int BUF = P * NT * kQRowB;       // bytes per buffer
  constexpr int ROUNDS = P * NT / (2 * kQWaves);  // direct loads per wave per block (2 rows each)
  static_assert(ROUNDS * 2 * kQWaves == P * NT, "the direct loads tile the buffer");
  const int4 ck = g.chunks[chunk];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c16 = lane & 15, j = lane >> 4;
  const int n = ck.z;
  const bool shared = ck.x < 0;
  const int P0 = g.T * g.K;
  int* rin = rows;          // input row of chunk token t (activation plane row)
  int* rout = rows + NT;    // output row
  if (threadIdx.x < NT) {
    const int t = min((int)threadIdx.x, n - 1);  // pad rows repeat the last token
    const int orow = shared ? P0 + ck.y + t : ck.y + t;
    rout[threadIdx.x] = orow;
    rin[threadIdx.x] = DOWN ? orow : (shared ? ck.y + t : g.pair_tok[ck.y + t]);
  }
  __syncthreads();
  const uint8_t* blob = shared ? g.shared : g.experts + (size_t)ck.x * g.expert_size;
  constexpr int ROWS = qgemm_rows(TL, DOWN);
  const uint8_t* mat[TL];
  int row[TL];
#pragma unroll
  for (int t = 0; t < TL; ++t) {
    if (DOWN) {
      mat[t] = blob + 2 * (size_t)kGateBytes;
      row[t] = rg * ROWS + 16 * TL * wave + 16 * t + c16;
    } else {
      // tiles 0 .. TL/2 - 1: gate rows, TL/2 .. TL - 1: the same rows of up
      mat[t] = blob + (t < TL / 2 ? 0 : (size_t)kGateBytes);
      row[t] = rg * ROWS + 8 * TL * wave + 16 * (t % (TL / 2)) + c16;
    }
  }
  // direct-load sources: round k of wave w fills LDS rows 2 (w + 8 k), +1 of
  // the buffer (row rho = plane * NT + token t); lane i: row rho0 + i / 32,
  // slot i % 32 holds piece (i % 32) ^ (t & 7) of that row's block.  The
  // token operand's 16-byte reads (lane (c16, j): row c16, piece
  // (8 j + m) ^ (c16 & 7)) are then free of bank conflicts; an XOR with all
  // four bits of c16 measured twice the cycles per read (2-way conflicts).
  uint32_t src[ROUNDS];
#pragma unroll
  for (int k = 0; k < ROUNDS; ++k) {
    const int rho = 2 * (wave + kQWaves * k) + (lane >> 5);
    const int p = rho / NT, t = rho - p * NT;
    const uint32_t piece = (uint32_t)((lane & 31) ^ (t & 7));
    src[k] = (uint32_t)((size_t)rin[t] * KD) + 8u * piece;  // element offset inside plane p
  }
  auto dma = [&](int b, int buf) {
    uint8_t* base = buf ? lds1 : lds0;
#pragma unroll
    for (int k = 0; k < ROUNDS; ++k) {
      const int rho0 = 2 * (wave + kQWaves * k);
      const int p = rho0 / NT;
      lds_dma16(g.xp + (size_t)p * g.plane + src[k] + (size_t)b * kQK, base + rho0 * kQRowB);
    }
  };
  const Q4KScaleSel sel = q4k_scale_sel(j);
  // corr operand A: token c16 of block nb, sub-blocks 2j and 2j+1 of block b
  auto load_xs = [&](int b, int nb) {
    const float2 v = *reinterpret_cast<const float2*>(g.xs + (size_t)rin[16 * nb + c16] * (KD / 32) + 8 * b + 2 * j);
    return v;
  };
  f32x4 acc[TL][NB];
#pragma unroll
  for (int tt = 0; tt < TL; ++tt)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[tt][nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // One block: the token operands of an MFMA step are read from LDS once and
  // serve every tile, whose B operands are built per step.
  auto block = [&](int buf, const QLane (&w)[TL], const float2 (&xsv)[NB]) {
    const uint8_t* base = buf ? lds1 : lds0;
    QScale sc[TL];
#pragma unroll
    for (int t = 0; t < TL; ++t) sc[t] = qscale(w[t].hdr, sel);
    f32x4 C[TL][NB];
#pragma unroll
    for (int t = 0; t < TL; ++t)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) C[t][nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int i0 = 2 * (m & 1);
      if constexpr (TL == 2) {
        // both tiles' B operands first, then each token operand read once
        // and used by both
        const u32x4& qa = m < 2 ? w[0].q0 : w[0].q1;
        const u32x4& qb = m < 2 ? w[1].q0 : w[1].q1;
        const BPair B0 = build_b(qa[i0], qa[i0 + 1], sc[0].k_lo, sc[0].k_hi);
        const BPair B1 = build_b(qb[i0], qb[i0 + 1], sc[1].k_lo, sc[1].k_hi);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
          for (int p = 0; p < P; ++p) {
            const uint8_t* r = base + (p * NT + 16 * nb + c16) * kQRowB;
            const f16x8 alo = *reinterpret_cast<const f16x8*>(r + 16 * ((8 * j + m) ^ (c16 & 7)));
            const f16x8 ahi = *reinterpret_cast<const f16x8*>(r + 16 * ((8 * j + m + 4) ^ (c16 & 7)));
            C[0][nb] = mfma_h(alo, B0.lo, C[0][nb]);
            C[1][nb] = mfma_h(alo, B1.lo, C[1][nb]);
            C[0][nb] = mfma_h(ahi, B0.hi, C[0][nb]);
            C[1][nb] = mfma_h(ahi, B1.hi, C[1][nb]);
          }
        }
        continue;
      }
      f16x8 alo[NB][P], ahi[NB][P];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int p = 0; p < P; ++p) {
          const uint8_t* r = base + (p * NT + 16 * nb + c16) * kQRowB;
          alo[nb][p] = *reinterpret_cast<const f16x8*>(r + 16 * ((8 * j + m) ^ (c16 & 7)));
          ahi[nb][p] = *reinterpret_cast<const f16x8*>(r + 16 * ((8 * j + m + 4) ^ (c16 & 7)));
        }
#pragma unroll
      for (int t = 0; t < TL; ++t) {
        const u32x4& qa = m < 2 ? w[t].q0 : w[t].q1;
        const BPair B = build_b(qa[i0], qa[i0 + 1], sc[t].k_lo, sc[t].k_hi);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int p = 0; p < P; ++p) {
            C[t][nb] = mfma_h(alo[nb][p], B.lo, C[t][nb]);
            C[t][nb] = mfma_h(ahi[nb][p], B.hi, C[t][nb]);
          }
      }
    }
#pragma unroll
    for (int t = 0; t < TL; ++t)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        f32x4 a = acc[t][nb];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = fmaf(sc[t].d, C[t][nb][i], a[i]);
        a = mfma_f(xsv[nb].x, sc[t].bc_lo, a);
        a = mfma_f(xsv[nb].y, sc[t].bc_hi, a);
        acc[t][nb] = a;
      }
  };
  auto load_w = [&](QLane (&w)[TL], int b, bool last) {
#pragma unroll
    for (int t = 0; t < TL; ++t)
      w[t] = last ? qlane_load<DOWN, true>(mat[t], row[t], b, j) : qlane_load<DOWN, false>(mat[t], row[t], b, j);
  };

  dma(0, 0);
  QLane wa[TL], wb[TL];
  load_w(wa, 0, false);
  float2 xa[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) xa[nb] = load_xs(0, nb);
  for (int b = 0; b < NBLK; b += 2) {
    // even block b from buffer 0 while b + 1 lands in buffer 1, then odd
    // block b + 1 from buffer 1 while b + 2 lands in buffer 0 (the last pair
    // re-stages the final block into the idle buffer: branch-free, so the
    // wait counts stay exact)
    wait_vm();
    __syncthreads();  // block b staged by every wave; buffer 1 read by all (block b - 1)
    dma(b + 1, 1);
    load_w(wb, b + 1, true);
    float2 xb[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) xb[nb] = load_xs(b + 1, nb);
    // keep the next block's loads ahead of this block's contraction (the
    // scheduler otherwise sinks them to just before the wait, to save
    // registers, and the stream is no longer a block ahead)
    __builtin_amdgcn_sched_barrier(0);
    block(0, wa, xa);
    const int b2 = min(b + 2, NBLK - 1);
    wait_vm();
    __syncthreads();  // block b + 1 staged; buffer 0 read by all (block b)
    dma(b2, 0);
    load_w(wa, b2, false);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) xa[nb] = load_xs(b2, nb);
    __builtin_amdgcn_sched_barrier(0);
    block(1, wb, xb);
  }
  wait_vm();  // the re-staged copy has landed before the LDS is released
  // D of a 16x16 MFMA: lane (c16, j) holds row (column) c16 of the tile and
  // tokens 4 j .. 4 j + 3 of the token block
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * nb + 4 * j + i;
      if (t >= n) continue;
      const float e = g.xe[rin[t]];
      if (DOWN) {
        float* o = g.out + (size_t)rout[t] * kHidden;
#pragma unroll
        for (int tt = 0; tt < TL; ++tt) o[row[tt]] = acc[tt][nb][i] * e;
      } else {
#pragma unroll
        for (int tt = 0; tt < TL / 2; ++tt)
          g.out[(size_t)rout[t] * kFfn + row[tt]] = silu_mul(acc[tt][nb][i] * e, acc[tt + TL / 2][nb][i] * e);
      }
    }
  }
}

// NB: the largest token block count of a chunk (1 for the 16-token chunks
// of batched decode, 4 for the 64-token chunks of prefill); a chunk runs the
// body of the fewest 16-token blocks that hold its tokens, so its weight
// operands are built once for up to 64 tokens and no MFMA runs on an empty
// block.  One-dimensional grid, mapped so that all the
// chunks of one expert that share a row group run on the same XCD, back to
// back: workgroups are handed to the eight XCDs in turn (id % 8), so
// id -> (xcd = id % 8, k = id / 8); XCD x owns row groups x, x + 8, ...
// (RG / 8 of them) of every chunk, and its k-th item is, within the item
// range q f .. q (f + c) - 1 of the expert whose chunks are f .. f + c - 1
// (q = RG / 8), row group 8 ((k - q f) / c) + x of chunk f + (k - q f) % c.
// An expert's weights are then read from HBM once per row group and served
// from that XCD's L2 to its other chunks; every XCD does the same work.
template <int P, int NB, bool DOWN>
__global__ __launch_bounds__(kQWaves * 64) __attribute__((amdgpu_waves_per_eu((P == 3 && DOWN) ? 3 : 2))) void k_qgemm(QGemmArgs g) {
  constexpr int TL = qgemm_tiles(P, DOWN);
  constexpr int RG = (DOWN ? kHidden : kFfn) / qgemm_rows(TL, DOWN);
  constexpr int Q = RG / 8;
  static_assert(Q * 8 == RG, "row groups split evenly over the XCDs");
  const int id = blockIdx.x, xcd = id & 7, k = id >> 3;
  const int m = k / Q;  // a chunk of the item's expert
  if (m >= *g.n_chunks) return;
  const int grp = g.chunks[m].w, f = grp & 0xFFFF, c = grp >> 16;
  const int off = k - Q * f;
  const int chunk = f + off % c, rg = 8 * (off / c) + xcd;
  constexpr int NT = 16 * NB;
  // two arrays, not one: the compiler then sees that the direct loads into
  // one buffer cannot alias the reads of the other, and does not wait for
  // them (with all outstanding loads) before the contraction
  __shared__ __attribute__((aligned(16))) uint8_t lds0[P * NT * kQRowB];
  __shared__ __attribute__((aligned(16))) uint8_t lds1[P * NT * kQRowB];
  __shared__ int rows[2 * NT];
  const int n = g.chunks[chunk].z;
  if constexpr (NB == 4) {
    if (n > 48) return qgemm_body<P, 4, DOWN, TL>(g, lds0, lds1, rows, chunk, rg);
    if (n > 32) return qgemm_body<P, 3, DOWN, TL>(g, lds0, lds1, rows, chunk, rg);
  }
  if constexpr (NB >= 2) {
    if (n > 16) return qgemm_body<P, 2, DOWN, TL>(g, lds0, lds1, rows, chunk, rg);
  }
  qgemm_body<P, 1, DOWN, TL>(g, lds0, lds1, rows, chunk, rg);
}

hipError_t launch_xplanes(const float* x, int kd, size_t n_rows, int planes, _Float16* xp, float* xs, float* xe,
                          hipStream_t s) {
  if (kd != kHidden && kd != kFfn) return hipErrorInvalidValue;
  const dim3 blk(256);
  const unsigned wide = (unsigned)n_rows, narrow = (unsigned)((n_rows + 3) / 4);
  if (planes == 3) {
    if (kd == kHidden)
      hipLaunchKernelGGL((k_xplanes<3, kHidden>), dim3(wide), blk, 0, s, x, n_rows, xp, xs, xe);
    else
      hipLaunchKernelGGL((k_xplanes<3, kFfn>), dim3(narrow), blk, 0, s, x, n_rows, xp, xs, xe);
  } else {
    if (kd == kHidden)
      hipLaunchKernelGGL((k_xplanes<1, kHidden>), dim3(wide), blk, 0, s, x, n_rows, xp, xs, xe);
    else
      hipLaunchKernelGGL((k_xplanes<1, kFfn>), dim3(narrow), blk, 0, s, x, n_rows, xp, xs, xe);
  }
  return hipGetLastError();
}

int qgemm_chunk_tokens(int planes) { return planes == 3 ? 16 : 64; }

hipError_t launch_qgemm(const QGemmArgs& g, int planes, bool down, int max_chunks, hipStream_t s) {
  const dim3 blk(kQWaves * 64);
  const int RG = (down ? kHidden : kFfn) / qgemm_rows(qgemm_tiles(planes, down), down);
  const dim3 grid((unsigned)(RG * max_chunks));
  if (planes == 3) {
    if (down)
      hipLaunchKernelGGL((k_qgemm<3, 1, true>), grid, blk, 0, s, g);
    else
      hipLaunchKernelGGL((k_qgemm<3, 1, false>), grid, blk, 0, s, g);
  } else {
    if (down)
      hipLaunchKernelGGL((k_qgemm<1, 4, true>), grid, blk, 0, s, g);
    else
      hipLaunchKernelGGL((k_qgemm<1, 4, false>), grid, blk, 0, s, g);
  }
  return hipGetLastError();
}

}  // namespace fdm
