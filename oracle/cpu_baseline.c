/*
 * cpu_baseline.c -- the reference's CPU expert path, timed on the host.
 * Used only by bench.py's cpu_baseline leg (and a test).
 *
 * Restates expert_worker (infer.m:1069-1091) and the combine loop
 * (infer.m:1915-1917): one thread per expert dequantises the expert's three
 * matrices in full to fp32 scratch with the quant.c decoders, runs three
 * single-precision matvecs (cblas_sgemv in the reference; a plain C loop
 * here, since Accelerate does not exist on Linux) and
 * SiLU*mul, then the outputs are combined with their routing weights in
 * slot order.  The shared expert is passed as one more blob with weight 1.
 */
#include "oracle.h"

#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

typedef struct {
    const void *blob;
    int down_is_q6;
    const float *x;
    float *gate_mat, *up_mat, *down_mat; /* fp32 scratch, as infer.m:1048-1057 */
    float gate[ORC_FFN], up[ORC_FFN], act[ORC_FFN];
    float out[ORC_HIDDEN];
} job_t;

/* Row-major single-precision matvec with eight interleaved partial sums
 * (n is a multiple of 8 for every R1 shape), so the compiler can keep it
 * in vector registers the way a BLAS sgemv would. */
static void sgemv_rows(const float *A, const float *x, float *y, int m, int n) {
    for (int r = 0; r < m; ++r) {
        const float *a = A + (size_t)r * n;
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int c = 0; c < n; c += 8)
            for (int j = 0; j < 8; ++j) acc[j] += a[c + j] * x[c + j];
        y[r] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    }
}

static void *expert_job(void *arg) {
    job_t *j = (job_t *)arg;
    const uint8_t *b = (const uint8_t *)j->blob;
    const size_t nel = (size_t)ORC_FFN * ORC_HIDDEN;
    orc_dequantize_row_q4_K(b, j->gate_mat, nel);
    orc_dequantize_row_q4_K(b + ORC_GATE_BYTES, j->up_mat, nel);
    if (j->down_is_q6)
        orc_dequantize_row_q6_K(b + 2 * ORC_GATE_BYTES, j->down_mat, nel);
    else
        orc_dequantize_row_q4_K(b + 2 * ORC_GATE_BYTES, j->down_mat, nel);
    sgemv_rows(j->gate_mat, j->x, j->gate, ORC_FFN, ORC_HIDDEN);
    sgemv_rows(j->up_mat, j->x, j->up, ORC_FFN, ORC_HIDDEN);
    orc_silu_mul(j->gate, j->up, j->act, ORC_FFN);
    sgemv_rows(j->down_mat, j->act, j->out, ORC_HIDDEN, ORC_FFN);
    return NULL;
}

static double now_us(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e6 + ts.tv_nsec * 1e-3;
}

static int cmp_double(const void *a, const void *b) {
    double x = *(const double *)a, y = *(const double *)b;
    return (x > y) - (x < y);
}

double orc_cpu_expert_baseline(const void *const *blobs, int n_experts, int down_is_q6,
                               const float *x, const float *w, float *out, int reps,
                               int n_threads) {
    if (n_experts <= 0 || n_experts > ORC_MAX_K + 1 || reps <= 0) return -1.0;
    if (n_threads <= 0 || n_threads > n_experts) n_threads = n_experts;
    const size_t nel = (size_t)ORC_FFN * ORC_HIDDEN;
    job_t *jobs = (job_t *)calloc((size_t)n_experts, sizeof(job_t));
    for (int k = 0; k < n_experts; ++k) {
        jobs[k].blob = blobs[k];
        jobs[k].down_is_q6 = down_is_q6;
        jobs[k].x = x;
        jobs[k].gate_mat = (float *)malloc(nel * sizeof(float));
        jobs[k].up_mat = (float *)malloc(nel * sizeof(float));
        jobs[k].down_mat = (float *)malloc(nel * sizeof(float));
    }
    double *t = (double *)malloc(sizeof(double) * (size_t)reps);
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)n_experts);
    for (int r = 0; r < reps; ++r) {
        const double t0 = now_us();
        for (int base = 0; base < n_experts; base += n_threads) {
            int end = base + n_threads < n_experts ? base + n_threads : n_experts;
            for (int k = base; k < end; ++k) pthread_create(&th[k], NULL, expert_job, &jobs[k]);
            for (int k = base; k < end; ++k) pthread_join(th[k], NULL);
        }
        for (int i = 0; i < ORC_HIDDEN; ++i) out[i] = 0.0f;
        for (int k = 0; k < n_experts; ++k)
            for (int i = 0; i < ORC_HIDDEN; ++i) out[i] += w[k] * jobs[k].out[i];
        t[r] = now_us() - t0;
    }
    qsort(t, (size_t)reps, sizeof(double), cmp_double);
    const double med = t[reps / 2];
    for (int k = 0; k < n_experts; ++k) {
        free(jobs[k].gate_mat);
        free(jobs[k].up_mat);
        free(jobs[k].down_mat);
    }
    free(jobs);
    free(t);
    free(th);
    return med;
}

/* The whole MoE branch of layer_forward on the CPU, as the reference runs it
 * with USE_CPU_EXPERTS (infer.m:1878-1922): router sgemv on the calling
 * thread, route(), then one thread per routed expert plus one for the
 * shared expert (infer.m:1886-1914), slot-order combine and the residual.
 * blobs[0..K-1] are the routed experts to run (a bounded sample: the same K
 * blobs whatever route() picks), blobs[K] the shared expert.  Returns the
 * median microseconds per token over `reps`; out receives the last result. */
double orc_cpu_layer_baseline(const void *const *blobs, int K, int down_is_q6, const float *Wg,
                              const float *bias, const float *x, const float *h_in,
                              float *out, int reps) {
    if (K <= 0 || K > ORC_MAX_K || reps <= 0) return -1.0;
    const int n = K + 1;
    const size_t nel = (size_t)ORC_FFN * ORC_HIDDEN;
    job_t *jobs = (job_t *)calloc((size_t)n, sizeof(job_t));
    for (int k = 0; k < n; ++k) {
        jobs[k].blob = blobs[k];
        jobs[k].down_is_q6 = down_is_q6;
        jobs[k].x = x;
        jobs[k].gate_mat = (float *)malloc(nel * sizeof(float));
        jobs[k].up_mat = (float *)malloc(nel * sizeof(float));
        jobs[k].down_mat = (float *)malloc(nel * sizeof(float));
    }
    double *t = (double *)malloc(sizeof(double) * (size_t)reps);
    pthread_t th[ORC_MAX_K + 1];
    float logits[ORC_N_EXPERTS];
    int idx[ORC_MAX_K];
    float w[ORC_MAX_K];
    for (int r = 0; r < reps; ++r) {
        const double t0 = now_us();
        sgemv_rows(Wg, x, logits, ORC_N_EXPERTS, ORC_HIDDEN);
        orc_route(logits, bias, K, idx, w);
        for (int k = 0; k < n; ++k) pthread_create(&th[k], NULL, expert_job, &jobs[k]);
        for (int k = 0; k < n; ++k) pthread_join(th[k], NULL);
        for (int i = 0; i < ORC_HIDDEN; ++i) {
            float acc = 0.0f;
            for (int k = 0; k < K; ++k) acc += w[k] * jobs[k].out[i];
            out[i] = h_in[i] + acc + jobs[K].out[i];
        }
        t[r] = now_us() - t0;
    }
    qsort(t, (size_t)reps, sizeof(double), cmp_double);
    const double med = t[reps / 2];
    for (int k = 0; k < n; ++k) {
        free(jobs[k].gate_mat);
        free(jobs[k].up_mat);
        free(jobs[k].down_mat);
    }
    free(jobs);
    free(t);
    return med;
}
