/*
 * moe_ref.c -- CPU restatement of the reference's MoE expert path: router
 * logits, route(), the expert FFN and the combine.  TEST INFRASTRUCTURE
 * ONLY (the checker); the shipped library never calls it.
 *
 * Numerics.
 *  - Expert outputs are computed in double from the bit-exact dequantised
 *    weights and rounded to float once: that is the truth the kernels are
 *    held to (1e-3 relative L2).  The single-precision column-order matvec
 *    the reference runs (cblas_sgemv, infer.m:1081-1090) is provided
 *    separately (orc_matvec_*_f32) for the CPU baseline.
 *  - Router logits use one fixed summation order, shared with the HIP
 *    router kernel, so both sides produce the same bits and routing can be
 *    compared exactly.  The reference's cblas_sgemv order is unspecified
 *    (Accelerate is closed), so any fixed order is an equally faithful
 *    restatement of infer.m:350-353.
 *  - sigmoidf is the reference's formula 1.0f/(1.0f+expf(-x)) (infer.m:376)
 *    with expf evaluated by orc_expf: exp in double from fma/mul/add only,
 *    rounded once to float, i.e. the correctly rounded expf except when the
 *    exact value lies within ~1e-16 relative of a rounding boundary.  The
 *    HIP router evaluates the identical sequence of IEEE operations.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------- */
/* Deterministic exp.  exp(x) = 2^k * e^r, k = floor(x/ln2 + 1/2),
 * r = x - k ln2 (two-constant Cody-Waite reduction with fma), e^r by its
 * Taylor series to r^13 (|r| <= 0.347: truncation < 5e-18) in Horner form. */
static double exp_det(double x) {
    if (x != x) return x;
    if (x > 709.0) return INFINITY;
    if (x < -746.0) return 0.0;
    const double inv_ln2 = 1.4426950408889634;
    const double ln2_hi = 0x1.62e42fefa39efp-1;
    const double ln2_lo = 0x1.abc9e3b39803fp-56;
    double t = x * inv_ln2;
    double k = floor(t + 0.5);
    double r = fma(-k, ln2_hi, x);
    r = fma(-k, ln2_lo, r);
    static const double inv_fact[14] = {
        1.0, 1.0, 1.0 / 2, 1.0 / 6, 1.0 / 24, 1.0 / 120, 1.0 / 720, 1.0 / 5040,
        1.0 / 40320, 1.0 / 362880, 1.0 / 3628800, 1.0 / 39916800, 1.0 / 479001600,
        1.0 / 6227020800.0};
    double p = inv_fact[13];
    for (int i = 12; i >= 0; --i) p = fma(p, r, inv_fact[i]);
    return ldexp(p, (int)k);
}

float orc_expf(float x) { return (float)exp_det((double)x); }

/* infer.m:376 */
float orc_sigmoidf(float x) { return 1.0f / (1.0f + orc_expf(-x)); }

/* infer.m:378-383 */
void orc_silu_mul(const float *g, const float *u, float *o, int d) {
    for (int i = 0; i < d; ++i) {
        const float v = g[i];
        o[i] = (v / (1.0f + orc_expf(-v))) * u[i];
    }
}

/* infer.m:369-374: inv = 1/sqrt(ss/d + eps); o = x * inv * w. */
void orc_rms_norm(const float *x, const float *w, float *o, int d) {
    /* `ss += x[i]*x[i]` is one statement: the reference's compiler (clang,
     * -O3 without fast-math, Makefile:2) contracts it to a fused multiply-add
     * (its default -ffp-contract=on), still in index order; the other
     * expressions have no multiply feeding an add. */
    float ss = 0.0f;
    for (int i = 0; i < d; ++i) ss = fmaf(x[i], x[i], ss);
    const float inv = 1.0f / sqrtf(ss / (float)d + ORC_RMS_EPS);
    for (int i = 0; i < d; ++i) o[i] = w ? x[i] * inv * w[i] : x[i] * inv;
}

/* ---------------------------------------------------------------------- */
/* Matvec oracles: bit-exact dequant of one row at a time, then a dot. */
typedef void (*deq_fn)(const void *, float *, size_t);

static void matvec_generic(deq_fn deq, size_t row_bytes, const void *W, const float *x,
                           float *y, int rows, int cols, int f32_order) {
    float *row = (float *)malloc(sizeof(float) * (size_t)cols);
    const uint8_t *w = (const uint8_t *)W;
    for (int r = 0; r < rows; ++r) {
        deq(w + (size_t)r * row_bytes, row, (size_t)cols);
        if (f32_order) {
            float acc = 0.0f;
            for (int c = 0; c < cols; ++c) acc += row[c] * x[c];
            y[r] = acc;
        } else {
            double acc = 0.0;
            for (int c = 0; c < cols; ++c) acc += (double)row[c] * (double)x[c];
            y[r] = (float)acc;
        }
    }
    free(row);
}

void orc_matvec_q4k(const void *W, const float *x, float *y, int rows, int cols) {
    matvec_generic(orc_dequantize_row_q4_K, (size_t)cols / ORC_QK_K * ORC_Q4K_BLOCK, W, x, y,
                   rows, cols, 0);
}
void orc_matvec_q6k(const void *W, const float *x, float *y, int rows, int cols) {
    matvec_generic(orc_dequantize_row_q6_K, (size_t)cols / ORC_QK_K * ORC_Q6K_BLOCK, W, x, y,
                   rows, cols, 0);
}
void orc_matvec_q4k_f32(const void *W, const float *x, float *y, int rows, int cols) {
    matvec_generic(orc_dequantize_row_q4_K, (size_t)cols / ORC_QK_K * ORC_Q4K_BLOCK, W, x, y,
                   rows, cols, 1);
}
void orc_matvec_q6k_f32(const void *W, const float *x, float *y, int rows, int cols) {
    matvec_generic(orc_dequantize_row_q6_K, (size_t)cols / ORC_QK_K * ORC_Q6K_BLOCK, W, x, y,
                   rows, cols, 1);
}

/* Double-precision matvec over a dequantised row stream (internal). */
static void matvec_d(deq_fn deq, size_t row_bytes, const void *W, const double *x, double *y,
                     int rows, int cols) {
    float *row = (float *)malloc(sizeof(float) * (size_t)cols);
    const uint8_t *w = (const uint8_t *)W;
    for (int r = 0; r < rows; ++r) {
        deq(w + (size_t)r * row_bytes, row, (size_t)cols);
        double acc = 0.0;
        for (int c = 0; c < cols; ++c) acc += (double)row[c] * x[c];
        y[r] = acc;
    }
    free(row);
}

/* infer.m:1069-1091 (expert_worker): gate = Wg.x, up = Wu.x,
 * act = silu(gate) * up, out = Wd.act; blob offsets infer.m:71-78. */
void orc_expert_ffn(const void *blob, int down_is_q6, const float *x, float *out,
                    float *gate_out, float *up_out, float *act_out) {
    const int H = ORC_HIDDEN, F = ORC_FFN;
    const uint8_t *b = (const uint8_t *)blob;
    const size_t q4_row_h = (size_t)H / ORC_QK_K * ORC_Q4K_BLOCK;
    double *xd = (double *)malloc(sizeof(double) * H);
    double *g = (double *)malloc(sizeof(double) * F);
    double *u = (double *)malloc(sizeof(double) * F);
    double *a = (double *)malloc(sizeof(double) * F);
    double *o = (double *)malloc(sizeof(double) * H);
    for (int i = 0; i < H; ++i) xd[i] = x[i];
    matvec_d(orc_dequantize_row_q4_K, q4_row_h, b, xd, g, F, H);
    matvec_d(orc_dequantize_row_q4_K, q4_row_h, b + ORC_GATE_BYTES, xd, u, F, H);
    for (int i = 0; i < F; ++i) a[i] = g[i] / (1.0 + exp(-g[i])) * u[i];
    if (down_is_q6)
        matvec_d(orc_dequantize_row_q6_K, (size_t)F / ORC_QK_K * ORC_Q6K_BLOCK,
                 b + 2 * ORC_GATE_BYTES, a, o, H, F);
    else
        matvec_d(orc_dequantize_row_q4_K, (size_t)F / ORC_QK_K * ORC_Q4K_BLOCK,
                 b + 2 * ORC_GATE_BYTES, a, o, H, F);
    for (int i = 0; i < H; ++i) out[i] = (float)o[i];
    for (int i = 0; i < F; ++i) {
        if (gate_out) gate_out[i] = (float)g[i];
        if (up_out) up_out[i] = (float)u[i];
        if (act_out) act_out[i] = (float)a[i];
    }
    free(xd);
    free(g);
    free(u);
    free(a);
    free(o);
}

/* (__fp16)x as f32_to_f16_alloc (infer.m:521-528) does it on the
 * reference's AArch64 host (FCVT with the default FPCR): IEEE round to
 * nearest even, subnormal halves kept, overflow to infinity, NaN quieted
 * with the top 9 payload bits kept.  Computed in double: x is scaled by the
 * half quantum of its binade (an exact power-of-two scaling), rounded to an
 * integer by nearbyint in the default round-to-nearest-even mode, and the
 * result encoded. */
uint16_t orc_fp32_to_fp16(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    if (isnan(f)) return (uint16_t)(sign | 0x7E00u | ((bits >> 13) & 0x1FFu));
    const double a = fabs((double)f);
    if (a >= 65520.0) return (uint16_t)(sign | 0x7C00u); /* rounds to 2^16 or beyond */
    if (a == 0.0) return sign;
    int e;
    (void)frexp(a, &e);                          /* a = m 2^e, m in [0.5, 1) */
    const int qexp = (e - 11 > -24) ? e - 11 : -24; /* 11 significant bits, or subnormal */
    const double n = nearbyint(ldexp(a, -qexp));  /* integer count of quanta */
    const double v = ldexp(n, qexp);
    if (v < ldexp(1.0, -14)) return (uint16_t)(sign | (uint16_t)n); /* subnormal (or 0) */
    int e2;
    const double m2 = frexp(v, &e2);              /* v = m2 2^e2 */
    const unsigned mant = (unsigned)((m2 * 2.0 - 1.0) * 1024.0);
    return (uint16_t)(sign | (uint16_t)((unsigned)(e2 - 1 + 15) << 10) | mant);
}

void orc_fp32_to_fp16_array(const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = orc_fp32_to_fp16(src[i]);
}

/* Double-precision matvec over F16 rows (internal). */
static void matvec_f16_d(const uint16_t *W, const double *x, double *y, int rows, int cols) {
    for (int r = 0; r < rows; ++r) {
        const uint16_t *w = W + (size_t)r * cols;
        double acc = 0.0;
        for (int c = 0; c < cols; ++c) acc += (double)orc_fp16_to_fp32(w[c]) * x[c];
        y[r] = acc;
    }
}

/* infer.m:1852-1868 (the dense branch of layer_forward): g = W_gate.h_post,
 * u = W_up.h_post (mv_f16, infer.m:459-513: F16 weights widened to fp32),
 * act = silu(g) * u (infer.m:378-383), out = h_in + W_down.act.  Gate and up
 * are [inter][7168], down [7168][inter], row-major F16.  Accumulated in
 * double: the truth the kernels are held to.  h_in may be NULL (0). */
void orc_dense_ffn(const uint16_t *gate, const uint16_t *up, const uint16_t *down, int inter,
                   const float *h_post, const float *h_in, float *out, float *act_out) {
    const int H = ORC_HIDDEN;
    double *x = (double *)malloc(sizeof(double) * H);
    double *g = (double *)malloc(sizeof(double) * inter);
    double *u = (double *)malloc(sizeof(double) * inter);
    double *o = (double *)malloc(sizeof(double) * H);
    for (int i = 0; i < H; ++i) x[i] = h_post[i];
    matvec_f16_d(gate, x, g, inter, H);
    matvec_f16_d(up, x, u, inter, H);
    for (int i = 0; i < inter; ++i) {
        g[i] = g[i] / (1.0 + exp(-g[i])) * u[i];
        if (act_out) act_out[i] = (float)g[i];
    }
    matvec_f16_d(down, g, o, H, inter);
    for (int i = 0; i < H; ++i) out[i] = (float)((h_in ? (double)h_in[i] : 0.0) + o[i]);
    free(x);
    free(g);
    free(u);
    free(o);
}

/* yarn_freq(i), i < 32 (infer.m:586-624): YaRN correction range of the 64
 * rope dims (base 10000, original context 4096, beta 32 / 1), factor 40,
 * evaluated in float as the reference does. */
void orc_yarn_freq(float *freq) {
    const int dim = 64;
    const float base = 10000.0f, orig = 4096.0f, twopi = 2.0f * (float)M_PI;
    const float lo_f = ((float)dim * logf(orig / (32.0f * twopi))) / (2.0f * logf(base));
    const float hi_f = ((float)dim * logf(orig / (1.0f * twopi))) / (2.0f * logf(base));
    int lo = (int)floorf(lo_f), hi = (int)ceilf(hi_f);
    if (lo < 0) lo = 0;
    if (hi > dim / 2 - 1) hi = dim / 2 - 1;
    if (hi <= lo) hi = lo + 1;
    for (int i = 0; i < dim / 2; ++i) {
        const float extra = 1.0f / powf(base, (float)(2 * i) / (float)dim);
        const float inter = extra / 40.0f;
        float denom = (float)(hi - lo);
        if (denom < 1e-3f) denom = 1e-3f;
        float ramp = ((float)i - (float)lo) / denom;
        if (ramp < 0.0f) ramp = 0.0f;
        if (ramp > 1.0f) ramp = 1.0f;
        const float mask = 1.0f - ramp;
        freq[i] = inter * (1.0f - mask) + extra * mask;
    }
}

/* The softmax scale of mla_forward (infer.m:802-815), in float. */
float orc_mla_scale(void) {
    const float m = 0.1f * logf(40.0f) + 1.0f;
    return (m * m) / sqrtf(192.0f);
}

static void mv_f16_rows_d(const uint16_t *W, const double *x, double *y, int rows, int cols) {
    for (int r = 0; r < rows; ++r) {
        const uint16_t *w = W + (size_t)r * cols;
        double acc = 0.0;
        for (int c = 0; c < cols; ++c) acc += (double)orc_fp16_to_fp32(w[c]) * x[c];
        y[r] = acc;
    }
}

/* The cache row of one token at position pos (infer.m:786-800, 817-827):
 * c_kv = rms_norm(kv_a[:512] . rms_norm(hidden, attn_norm), kv_a_norm) and
 * the YaRN-rotated k_rope = kv_a[512:576], the matvec in double and rounded
 * to float as orc_mla_forward stores them (it calls this). */
static void mla_cache_row(const float *attn_norm, const uint16_t *kv_a, const float *kv_a_norm,
                          const float *hidden, int pos, float *c_row, float *k_row) {
    const int H = ORC_HIDDEN, KVL = 512, ROPE = 64;
    float *normed = (float *)malloc(sizeof(float) * H);
    double *xd = (double *)malloc(sizeof(double) * H);
    double kva[576];
    float kvf[512];
    float freq[32];
    orc_yarn_freq(freq);
    orc_rms_norm(hidden, attn_norm, normed, H);
    for (int i = 0; i < H; ++i) xd[i] = normed[i];
    mv_f16_rows_d(kv_a, xd, kva, 576, H);
    for (int i = 0; i < KVL; ++i) kvf[i] = (float)kva[i];
    orc_rms_norm(kvf, kv_a_norm, c_row, KVL);
    for (int i = 0; i < ROPE / 2; ++i) {
        const float ang = (float)pos * freq[i];
        const double c = cos((double)ang), sn = sin((double)ang);
        const double a = kva[KVL + 2 * i], b = kva[KVL + 2 * i + 1];
        k_row[2 * i] = (float)(a * c - b * sn);
        k_row[2 * i + 1] = (float)(a * sn + b * c);
    }
    free(normed); free(xd);
}

/* Only the cache append of mla_forward: row len of the cache for a token at
 * position pos, without its attention output (tests fill long caches with
 * it and check the forward of the tokens after). */
void orc_mla_append(const float *attn_norm, const uint16_t *kv_a, const float *kv_a_norm, const float *hidden,
                    float *cache_c, float *cache_k, int len, int pos) {
    mla_cache_row(attn_norm, kv_a, kv_a_norm, hidden, pos, cache_c + (size_t)len * 512, cache_k + (size_t)len * 64);
}

/* mla_forward (infer.m:766-903) of one token at position pos; the cache holds
 * len rows before it and receives row len.  Dot products, softmax and the
 * latent sums in double (the truth); the three rms_norms are the reference's
 * float function on the float-rounded inputs; the YaRN table, the rope angle
 * (float)pos * freq and the softmax scale in float as the reference computes
 * them.  Weights as LayerAttnDense holds them (see fdm_attn_weights). */
void orc_mla_forward(const float *attn_norm, const uint16_t *q_a, const float *q_a_norm, const uint16_t *q_b,
                     const uint16_t *kv_a, const float *kv_a_norm, const uint16_t *k_b, const uint16_t *v_b,
                     const uint16_t *o_proj, float *hidden, float *cache_c, float *cache_k, int len, int pos) {
    const int H = ORC_HIDDEN, NH = 128, QA = 1536, KVL = 512, NOPE = 128, ROPE = 64, QK = 192, VH = 128;
    const int S = len + 1;
    float *normed = (float *)malloc(sizeof(float) * H);
    double *xd = (double *)malloc(sizeof(double) * (H > NH * VH ? H : NH * VH));
    double *qa = (double *)malloc(sizeof(double) * QA);
    float *qaf = (float *)malloc(sizeof(float) * QA);
    double *q = (double *)malloc(sizeof(double) * NH * QK);
    double *qabs = (double *)malloc(sizeof(double) * NH * KVL);
    double *p = (double *)malloc(sizeof(double) * S);
    double *wc = (double *)malloc(sizeof(double) * KVL);
    double *attn = (double *)malloc(sizeof(double) * NH * VH);
    double *o = (double *)malloc(sizeof(double) * H);
    float freq[32];
    orc_yarn_freq(freq);

    orc_rms_norm(hidden, attn_norm, normed, H);
    for (int i = 0; i < H; ++i) xd[i] = normed[i];
    mv_f16_rows_d(q_a, xd, qa, QA, H);
    for (int i = 0; i < QA; ++i) qaf[i] = (float)qa[i];
    orc_rms_norm(qaf, q_a_norm, qaf, QA);
    for (int i = 0; i < QA; ++i) qa[i] = qaf[i];
    mv_f16_rows_d(q_b, qa, q, NH * QK, QA);
    /* the cache row: c_kv and the rotated k_rope */
    mla_cache_row(attn_norm, kv_a, kv_a_norm, hidden, pos, cache_c + (size_t)len * KVL, cache_k + (size_t)len * ROPE);
    /* interleaved-pair YaRN rotation of q_rope (infer.m:626-655) */
    for (int i = 0; i < ROPE / 2; ++i) {
        const float ang = (float)pos * freq[i];
        const double c = cos((double)ang), sn = sin((double)ang);
        for (int h = 0; h < NH; ++h) {
            double *qr = q + (size_t)h * QK + NOPE;
            const double a = qr[2 * i], b = qr[2 * i + 1];
            qr[2 * i] = a * c - b * sn;
            qr[2 * i + 1] = a * sn + b * c;
        }
    }
    const double scale = orc_mla_scale();
    for (int h = 0; h < NH; ++h) {
        /* Q_abs[h] = k_b[h] (KV_LORA x NOPE) . q_nope[h] (infer.m:722-731) */
        mv_f16_rows_d(k_b + (size_t)h * KVL * NOPE, q + (size_t)h * QK, qabs + (size_t)h * KVL, KVL, NOPE);
    }
    for (int h = 0; h < NH; ++h) {
        const double *qb = qabs + (size_t)h * KVL, *qr = q + (size_t)h * QK + NOPE;
        double m = -INFINITY;
        for (int t = 0; t < S; ++t) {
            double a = 0.0, b = 0.0;
            for (int i = 0; i < KVL; ++i) a += qb[i] * cache_c[(size_t)t * KVL + i];
            for (int i = 0; i < ROPE; ++i) b += qr[i] * cache_k[(size_t)t * ROPE + i];
            p[t] = scale * a + scale * b;
            if (p[t] > m) m = p[t];
        }
        double sum = 0.0;
        for (int t = 0; t < S; ++t) {
            p[t] = exp(p[t] - m);
            sum += p[t];
        }
        for (int i = 0; i < KVL; ++i) wc[i] = 0.0;
        for (int t = 0; t < S; ++t)
            for (int i = 0; i < KVL; ++i) wc[i] += p[t] / sum * cache_c[(size_t)t * KVL + i];
        /* attn[h] = v_b[h] (V_HEAD x KV_LORA) . wc (infer.m:740-749) */
        mv_f16_rows_d(v_b + (size_t)h * VH * KVL, wc, attn + (size_t)h * VH, VH, KVL);
    }
    mv_f16_rows_d(o_proj, attn, o, H, NH * VH);
    for (int i = 0; i < H; ++i) hidden[i] = (float)((double)hidden[i] + o[i]);
    free(normed); free(xd); free(qa); free(qaf); free(q);
    free(qabs); free(p); free(wc); free(attn); free(o);
}

/* ---------------------------------------------------------------------- */
/* Router logits, canonical order.  For output row e, 256 partial sums are
 * formed: partial t accumulates, with one fmaf per element, the float4
 * chunks c = t, t+256, t+512, ... (c indexes groups of 4 consecutive
 * columns), components in order.  The 256 partials are split into four
 * runs of 64; each run is reduced by an xor butterfly (v[l] += v[l ^ m] for
 * m = 32,16,8,4,2,1, all l at once) and the four results are combined as
 * (s0 + s1) + (s2 + s3).  The HIP router kernel computes exactly this. */
void orc_router_logits(const float *Wg, const float *x, float *logits, int n_exp, int dim) {
    const int n4 = dim / 4;
    for (int e = 0; e < n_exp; ++e) {
        const float *w = Wg + (size_t)e * dim;
        float part[256];
        for (int t = 0; t < 256; ++t) {
            float acc = 0.0f;
            for (int c = t; c < n4; c += 256)
                for (int q = 0; q < 4; ++q) acc = fmaf(w[4 * c + q], x[4 * c + q], acc);
            part[t] = acc;
        }
        float s[4];
        for (int run = 0; run < 4; ++run) {
            float v[64], nv[64];
            memcpy(v, part + 64 * run, sizeof v);
            for (int m = 32; m >= 1; m >>= 1) {
                for (int l = 0; l < 64; ++l) nv[l] = v[l] + v[l ^ m];
                memcpy(v, nv, sizeof v);
            }
            s[run] = v[0];
        }
        logits[e] = (s[0] + s[1]) + (s[2] + s[3]);
    }
}

/* infer.m:920-991, DeepSeek-V3 noaux_tc routing:
 *   score = sigmoid(logit) (weights), choice = score + bias (selection);
 *   group score = sum of the top two choices in the group (running top-2
 *   from -1e30, strict >); the top `topk_group` groups are taken by repeated
 *   strict-> argmax passes (lowest index wins a tie); other groups are
 *   masked to -1e30; the top K are picked by one pass over the experts in
 *   index order that replaces the first minimum slot when strictly greater;
 *   weights are the unbiased scores of the picks, summed in slot order and
 *   scaled by scale/sum when the sum is positive.
 * One deviation: where every remaining group score is <= -1e30 (all
 * choices NaN or -inf), the reference stores group -1 and then indexes out
 * of bounds; here such a group is skipped. */
void orc_route_ex(const float *logits, const float *bias, int n_exp, int n_group,
                  int topk_group, int K, float scale, int *exp_idx, float *exp_w) {
    float score[1024], choice[1024], masked[1024];
    const int per = n_exp / n_group;
    for (int i = 0; i < n_exp; ++i) {
        score[i] = orc_sigmoidf(logits[i]);
        choice[i] = score[i] + (bias ? bias[i] : 0.0f);
    }
    float gscore[64];
    for (int g = 0; g < n_group; ++g) {
        float t1 = -1e30f, t2 = -1e30f;
        for (int e = 0; e < per; ++e) {
            const float s = choice[g * per + e];
            if (s > t1) {
                t2 = t1;
                t1 = s;
            } else if (s > t2) {
                t2 = s;
            }
        }
        gscore[g] = t1 + t2;
    }
    int chosen[64];
    for (int k = 0; k < topk_group; ++k) {
        int best = -1;
        float bs = -1e30f;
        for (int g = 0; g < n_group; ++g) {
            int taken = 0;
            for (int j = 0; j < k; ++j) taken |= (chosen[j] == g);
            if (!taken && gscore[g] > bs) {
                bs = gscore[g];
                best = g;
            }
        }
        chosen[k] = best;
    }
    for (int i = 0; i < n_exp; ++i) masked[i] = -1e30f;
    for (int k = 0; k < topk_group; ++k) {
        const int g = chosen[k];
        if (g < 0) continue;
        for (int e = 0; e < per; ++e) masked[g * per + e] = choice[g * per + e];
    }
    float key[ORC_MAX_K];
    for (int k = 0; k < K; ++k) {
        key[k] = -1e30f;
        exp_idx[k] = 0;
    }
    for (int i = 0; i < n_exp; ++i) {
        int slot = 0;
        for (int k = 1; k < K; ++k)
            if (key[k] < key[slot]) slot = k;
        if (masked[i] > key[slot]) {
            key[slot] = masked[i];
            exp_idx[slot] = i;
        }
    }
    for (int k = 0; k < K; ++k) exp_w[k] = score[exp_idx[k]];
    float sum = 0.0f;
    for (int k = 0; k < K; ++k) sum += exp_w[k];
    if (sum > 0.0f) {
        const float f = scale / sum;
        for (int k = 0; k < K; ++k) exp_w[k] *= f;
    }
}

void orc_route(const float *logits, const float *bias, int K, int *exp_idx, float *exp_w) {
    orc_route_ex(logits, bias, ORC_N_EXPERTS, ORC_N_GROUP, ORC_TOPK_GROUP, K, ORC_ROUTED_SCALE,
                 exp_idx, exp_w);
}

/* ---------------------------------------------------------------------- */
static int down_is_q6_for(size_t expert_size) {
    return expert_size == 2 * ORC_GATE_BYTES + ORC_DOWN_Q6K_BYTES;
}

/* metal_moe_forward, infer.m:1604-1700: moe_out = 0, then moe_out +=
 * w[k] * E_k for k = 0..K-1 (the saxpy loop at infer.m:1690-1695). */
void orc_moe_forward(const void *experts, size_t expert_size, const float *h_post,
                     const int *exp_idx, const float *exp_w, int K, float *moe_out) {
    const int q6 = down_is_q6_for(expert_size);
    float *eo = (float *)malloc(sizeof(float) * ORC_HIDDEN);
    for (int i = 0; i < ORC_HIDDEN; ++i) moe_out[i] = 0.0f;
    for (int k = 0; k < K; ++k) {
        const uint8_t *blob = (const uint8_t *)experts + (size_t)exp_idx[k] * expert_size;
        orc_expert_ffn(blob, q6, h_post, eo, NULL, NULL, NULL);
        for (int i = 0; i < ORC_HIDDEN; ++i) moe_out[i] = fmaf(exp_w[k], eo[i], moe_out[i]);
    }
    free(eo);
}

/* The MoE branch of layer_forward, infer.m:1878-1922. */
void orc_moe_layer(const void *experts, size_t expert_size, const float *Wg, const float *bias,
                   const void *shared_blob, const float *h_post, const float *h_in, int K,
                   float *hidden_out, int *idx_out, float *w_out, float *moe_out,
                   float *shared_out) {
    float logits[ORC_N_EXPERTS];
    int idx[ORC_MAX_K];
    float w[ORC_MAX_K];
    orc_router_logits(Wg, h_post, logits, ORC_N_EXPERTS, ORC_HIDDEN);
    orc_route(logits, bias, K, idx, w);
    float *moe = (float *)malloc(sizeof(float) * ORC_HIDDEN);
    float *sd = (float *)malloc(sizeof(float) * ORC_HIDDEN);
    orc_moe_forward(experts, expert_size, h_post, idx, w, K, moe);
    if (shared_blob)
        orc_expert_ffn(shared_blob, down_is_q6_for(expert_size), h_post, sd, NULL, NULL, NULL);
    else
        memset(sd, 0, sizeof(float) * ORC_HIDDEN);
    for (int i = 0; i < ORC_HIDDEN; ++i) {
        const float hin = h_in ? h_in[i] : 0.0f;
        if (hidden_out) hidden_out[i] = hin + moe[i] + sd[i];
        if (moe_out) moe_out[i] = moe[i];
        if (shared_out) shared_out[i] = sd[i];
    }
    for (int k = 0; k < K; ++k) {
        if (idx_out) idx_out[k] = idx[k];
        if (w_out) w_out[k] = w[k];
    }
    free(moe);
    free(sd);
}
