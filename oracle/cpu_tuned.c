/*
 * cpu_tuned.c -- a tuned CPU version of the MoE branch (the "tuned" CPU
 * baseline): the reference's arithmetic (quant.c dequant, fp32 dot products,
 * infer.m:1069-1091 expert order, infer.m:1878-1922 combine) with the
 * dequant fused into the dot product row by row -- no fp32 copy of the
 * matrices -- and every row spread over all host cores by a persistent team
 * of pthreads.  AVX2 + FMA (the x86-64-v3 baseline of current servers); the
 * dequantised weight d*sc*q - dmin*m is formed exactly as quant.c:49-57
 * (multiply, then subtract), only the accumulation into the dot product is
 * fused.  Used only by bench.py's cpu_baseline leg (and a test).
 */
#include "oracle.h"

#include <immintrin.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

static float hsum8(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
    return _mm_cvtss_f32(s);
}

/* 8 bytes -> 8 floats of (byte >> shift) & mask */
static __m256 bytes8(const uint8_t *p, int shift, int mask) {
    __m128i b = _mm_loadl_epi64((const __m128i *)p);
    __m256i v = _mm256_cvtepu8_epi32(b);
    v = _mm256_and_si256(_mm256_srli_epi32(v, shift), _mm256_set1_epi32(mask));
    return _mm256_cvtepi32_ps(v);
}

/* One Q4_K row (cols / 256 blocks) dotted with x. */
static float q4k_row_dot(const uint8_t *row, const float *x, int cols) {
    __m256 acc = _mm256_setzero_ps();
    for (int b = 0; b < cols / ORC_QK_K; ++b) {
        const uint8_t *blk = row + (size_t)b * ORC_Q4K_BLOCK;
        uint16_t hd, hm;
        memcpy(&hd, blk, 2);
        memcpy(&hm, blk + 2, 2);
        const float d = orc_fp16_to_fp32(hd), dmin = orc_fp16_to_fp32(hm);
        const uint8_t *sc = blk + 4, *qs = blk + 16;
        const float *xb = x + (size_t)b * ORC_QK_K;
        for (int c = 0; c < 4; ++c) {
            uint8_t s1, m1, s2, m2;
            orc_get_scale_min_k4(2 * c, sc, &s1, &m1);
            orc_get_scale_min_k4(2 * c + 1, sc, &s2, &m2);
            const __m256 d1 = _mm256_set1_ps(d * s1), mm1 = _mm256_set1_ps(dmin * m1);
            const __m256 d2 = _mm256_set1_ps(d * s2), mm2 = _mm256_set1_ps(dmin * m2);
            const uint8_t *q = qs + 32 * c;
            for (int l = 0; l < 32; l += 8) {
                const __m256 y1 = _mm256_sub_ps(_mm256_mul_ps(d1, bytes8(q + l, 0, 15)), mm1);
                const __m256 y2 = _mm256_sub_ps(_mm256_mul_ps(d2, bytes8(q + l, 4, 15)), mm2);
                acc = _mm256_fmadd_ps(y1, _mm256_loadu_ps(xb + 64 * c + l), acc);
                acc = _mm256_fmadd_ps(y2, _mm256_loadu_ps(xb + 64 * c + 32 + l), acc);
            }
        }
    }
    return hsum8(acc);
}

/* One Q6_K row dotted with x (quant.c:63-92 decode). */
static float q6k_row_dot(const uint8_t *row, const float *x, int cols) {
    __m256 acc = _mm256_setzero_ps();
    const __m256i k32 = _mm256_set1_epi32(32);
    for (int b = 0; b < cols / ORC_QK_K; ++b) {
        const uint8_t *blk = row + (size_t)b * ORC_Q6K_BLOCK;
        const uint8_t *ql = blk, *qh = blk + 128;
        const int8_t *sc = (const int8_t *)(blk + 192);
        uint16_t hd;
        memcpy(&hd, blk + 208, 2);
        const float d = orc_fp16_to_fp32(hd);
        const float *xb = x + (size_t)b * ORC_QK_K;
        for (int h = 0; h < 2; ++h) {
            for (int l = 0; l < 32; l += 8) {
                const int is = l / 16;
                const __m256i a = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)(ql + l)));
                const __m256i a2 = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)(ql + 32 + l)));
                const __m256i hh = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)(qh + l)));
                const __m256i f = _mm256_set1_epi32(15), t3 = _mm256_set1_epi32(3);
                __m256i q1 = _mm256_or_si256(_mm256_and_si256(a, f), _mm256_slli_epi32(_mm256_and_si256(hh, t3), 4));
                __m256i q2 = _mm256_or_si256(_mm256_and_si256(a2, f),
                                             _mm256_slli_epi32(_mm256_and_si256(_mm256_srli_epi32(hh, 2), t3), 4));
                __m256i q3 = _mm256_or_si256(_mm256_srli_epi32(a, 4),
                                             _mm256_slli_epi32(_mm256_and_si256(_mm256_srli_epi32(hh, 4), t3), 4));
                __m256i q4 = _mm256_or_si256(_mm256_srli_epi32(a2, 4),
                                             _mm256_slli_epi32(_mm256_and_si256(_mm256_srli_epi32(hh, 6), t3), 4));
                const __m256i qs[4] = {_mm256_sub_epi32(q1, k32), _mm256_sub_epi32(q2, k32),
                                       _mm256_sub_epi32(q3, k32), _mm256_sub_epi32(q4, k32)};
                for (int k = 0; k < 4; ++k) {
                    const __m256 ds = _mm256_set1_ps(d * (float)sc[is + 2 * k]);
                    const __m256 y = _mm256_mul_ps(ds, _mm256_cvtepi32_ps(qs[k]));
                    acc = _mm256_fmadd_ps(y, _mm256_loadu_ps(xb + 128 * h + 32 * k + l), acc);
                }
            }
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
    return hsum8(acc);
}

static float f32_row_dot(const float *row, const float *x, int cols) {
    __m256 acc = _mm256_setzero_ps();
    for (int c = 0; c < cols; c += 8) acc = _mm256_fmadd_ps(_mm256_loadu_ps(row + c), _mm256_loadu_ps(x + c), acc);
    return hsum8(acc);
}

typedef struct {
    /* inputs */
    const void *const *blobs;
    int K, n, down_is_q6, n_threads;
    const float *Wg, *bias, *x, *h_in;
    /* scratch */
    float logits[ORC_N_EXPERTS];
    int idx[ORC_MAX_K];
    float w[ORC_MAX_K];
    float *gate, *up, *act, *eo; /* [n][FFN] x 3, [n][HIDDEN] */
    float *out;
    pthread_barrier_t bar;
} team_t;

typedef struct {
    team_t *t;
    int id;
    int reps;
    double *times;
} member_t;

static double now_us(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e6 + ts.tv_nsec * 1e-3;
}

static void span(int total, int nt, int id, int *a, int *b) {
    *a = (int)((long)total * id / nt);
    *b = (int)((long)total * (id + 1) / nt);
}

static void one_token(team_t *t, int id) {
    const int nt = t->n_threads, n = t->n, K = t->K;
    const size_t gu_row = (size_t)ORC_HIDDEN / ORC_QK_K * ORC_Q4K_BLOCK;
    const size_t dn_row = (size_t)ORC_FFN / ORC_QK_K * (t->down_is_q6 ? ORC_Q6K_BLOCK : ORC_Q4K_BLOCK);
    int a, b;
    span(ORC_N_EXPERTS, nt, id, &a, &b);
    for (int r = a; r < b; ++r) t->logits[r] = f32_row_dot(t->Wg + (size_t)r * ORC_HIDDEN, t->x, ORC_HIDDEN);
    pthread_barrier_wait(&t->bar);
    if (id == 0) orc_route(t->logits, t->bias, K, t->idx, t->w);
    pthread_barrier_wait(&t->bar);
    /* gate and up rows of every expert (routed slots in order, then shared) */
    span(n * 2 * ORC_FFN, nt, id, &a, &b);
    for (int i = a; i < b; ++i) {
        const int e = i / (2 * ORC_FFN), rr = i % (2 * ORC_FFN);
        const uint8_t *blob = (const uint8_t *)t->blobs[e];
        const int up = rr >= ORC_FFN, r = rr % ORC_FFN;
        const float v = q4k_row_dot(blob + (up ? ORC_GATE_BYTES : 0) + (size_t)r * gu_row, t->x, ORC_HIDDEN);
        (up ? t->up : t->gate)[(size_t)e * ORC_FFN + r] = v;
    }
    pthread_barrier_wait(&t->bar);
    span(n * ORC_FFN, nt, id, &a, &b);
    if (b > a) orc_silu_mul(t->gate + a, t->up + a, t->act + a, b - a);
    pthread_barrier_wait(&t->bar);
    span(n * ORC_HIDDEN, nt, id, &a, &b);
    for (int i = a; i < b; ++i) {
        const int e = i / ORC_HIDDEN, r = i % ORC_HIDDEN;
        const uint8_t *dn = (const uint8_t *)t->blobs[e] + 2 * (size_t)ORC_GATE_BYTES + (size_t)r * dn_row;
        const float *act = t->act + (size_t)e * ORC_FFN;
        t->eo[i] = t->down_is_q6 ? q6k_row_dot(dn, act, ORC_FFN) : q4k_row_dot(dn, act, ORC_FFN);
    }
    pthread_barrier_wait(&t->bar);
    span(ORC_HIDDEN, nt, id, &a, &b);
    for (int i = a; i < b; ++i) {
        float acc = 0.0f;
        for (int k = 0; k < K; ++k) acc += t->w[k] * t->eo[(size_t)k * ORC_HIDDEN + i];
        t->out[i] = t->h_in[i] + acc + t->eo[(size_t)K * ORC_HIDDEN + i];
    }
    pthread_barrier_wait(&t->bar);
}

static void *member(void *arg) {
    member_t *m = (member_t *)arg;
    for (int r = 0; r < m->reps; ++r) {
        pthread_barrier_wait(&m->t->bar);
        const double t0 = now_us();
        one_token(m->t, m->id);
        if (m->id == 0) m->times[r] = now_us() - t0;
    }
    return NULL;
}

static int cmp_double(const void *a, const void *b) {
    double x = *(const double *)a, y = *(const double *)b;
    return (x > y) - (x < y);
}

/* The MoE branch of one token (router, route(), blobs[0..K-1] routed and
 * blobs[K] shared, combine, residual) on n_threads host threads (0: every
 * online core).  Returns the median microseconds per token over `reps`; out
 * receives the last result and *threads_used the team size. */
double orc_cpu_layer_tuned(const void *const *blobs, int K, int down_is_q6, const float *Wg, const float *bias,
                           const float *x, const float *h_in, float *out, int reps, int n_threads,
                           int *threads_used) {
    if (K <= 0 || K > ORC_MAX_K || reps <= 0) return -1.0;
    if (n_threads <= 0) n_threads = (int)sysconf(_SC_NPROCESSORS_ONLN);
    if (n_threads < 1) n_threads = 1;
    if (threads_used) *threads_used = n_threads;
    team_t *t = (team_t *)calloc(1, sizeof(team_t));
    t->blobs = blobs;
    t->K = K;
    t->n = K + 1;
    t->down_is_q6 = down_is_q6;
    t->n_threads = n_threads;
    t->Wg = Wg;
    t->bias = bias;
    t->x = x;
    t->h_in = h_in;
    t->out = out;
    t->gate = (float *)malloc(sizeof(float) * (size_t)t->n * ORC_FFN);
    t->up = (float *)malloc(sizeof(float) * (size_t)t->n * ORC_FFN);
    t->act = (float *)malloc(sizeof(float) * (size_t)t->n * ORC_FFN);
    t->eo = (float *)malloc(sizeof(float) * (size_t)t->n * ORC_HIDDEN);
    pthread_barrier_init(&t->bar, NULL, (unsigned)n_threads);
    double *times = (double *)malloc(sizeof(double) * (size_t)reps);
    member_t *ms = (member_t *)calloc((size_t)n_threads, sizeof(member_t));
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)n_threads);
    for (int i = 0; i < n_threads; ++i) {
        ms[i].t = t;
        ms[i].id = i;
        ms[i].reps = reps;
        ms[i].times = times;
        if (i) pthread_create(&th[i], NULL, member, &ms[i]);
    }
    member(&ms[0]);
    for (int i = 1; i < n_threads; ++i) pthread_join(th[i], NULL);
    qsort(times, (size_t)reps, sizeof(double), cmp_double);
    const double med = times[reps / 2];
    pthread_barrier_destroy(&t->bar);
    free(t->gate);
    free(t->up);
    free(t->act);
    free(t->eo);
    free(t);
    free(times);
    free(ms);
    free(th);
    return med;
}
