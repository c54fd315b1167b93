/*
 * oracle.h -- CPU restatement of the flash_deepseek MoE expert hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links or loads
 * this code; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, as the checker.
 *
 * Every function cites the reference file:line whose behaviour it restates.
 * The whole directory is compiled with -ffp-contract=off so that every
 * multiply and add written here rounds separately, exactly as the C source
 * of the reference reads (see quant_ref.c for the contraction discussion).
 */
#ifndef FDM_ORACLE_H
#define FDM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Block geometry: quant.h:6-8. */
#define ORC_QK_K 256
#define ORC_Q4K_BLOCK 144
#define ORC_Q6K_BLOCK 210

/* DeepSeek-R1 MoE shape: infer.m:41-80. */
#define ORC_HIDDEN 7168
#define ORC_FFN 2048
#define ORC_N_EXPERTS 256
#define ORC_N_GROUP 8
#define ORC_TOPK_GROUP 4
#define ORC_ROUTED_SCALE 2.5f
#define ORC_MAX_K 16
#define ORC_RMS_EPS 1e-6f

/* Byte sizes of one packed expert (infer.m:69-78, repack_experts.c:157-160). */
#define ORC_GATE_BYTES (57344ull * ORC_Q4K_BLOCK)
#define ORC_DOWN_Q4K_BYTES (57344ull * ORC_Q4K_BLOCK)
#define ORC_DOWN_Q6K_BYTES (57344ull * ORC_Q6K_BLOCK)

/* ---- quant codec (quant.c) ------------------------------------------- */
float orc_fp16_to_fp32(uint16_t h);                                   /* quant.c:4-24  */
void orc_fp16_to_fp32_array(const uint16_t *src, float *dst, size_t n);
void orc_get_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m); /* quant.c:26-34 */
void orc_dequantize_row_q4_K(const void *src, float *dst, size_t n); /* quant.c:36-61 */
void orc_dequantize_row_q6_K(const void *src, float *dst, size_t n); /* quant.c:63-92 */

/* ---- dense helpers (infer.m) --------------------------------------- */
float orc_expf(float x);        /* deterministic expf, see moe_ref.c */
float orc_sigmoidf(float x);    /* infer.m:376 */
void orc_silu_mul(const float *g, const float *u, float *o, int d);  /* infer.m:378-383 */
void orc_rms_norm(const float *x, const float *w, float *o, int d);  /* infer.m:369-374 */

/* ---- matvec oracles -------------------------------------------------- */
/* y = deq(W) . x with the dot product accumulated in double (the truth the
 * kernels are held to).  W is rows x cols, row-major Q4_K / Q6_K blocks. */
void orc_matvec_q4k(const void *W, const float *x, float *y, int rows, int cols);
void orc_matvec_q6k(const void *W, const float *x, float *y, int rows, int cols);
/* Same, but the dot product in single precision in column order: the
 * reference's CPU expert path (infer.m:1075-1090, dequant then sgemv). */
void orc_matvec_q4k_f32(const void *W, const float *x, float *y, int rows, int cols);
void orc_matvec_q6k_f32(const void *W, const float *x, float *y, int rows, int cols);

/* ---- expert FFN ------------------------------------------------------ */
/* One SwiGLU expert from a packed blob [gate Q4_K | up Q4_K | down Q4_K/Q6_K]
 * (infer.m:1069-1091).  Computed in double from the bit-exact dequantised
 * weights, rounded to float at the end.  gate_out/up_out/act_out may be NULL. */
/* (__fp16)x of f32_to_f16_alloc (infer.m:521-528) and the dense FFN of
 * layer_forward (infer.m:1852-1868), see moe_ref.c. */
uint16_t orc_fp32_to_fp16(float f);
void orc_fp32_to_fp16_array(const float *src, uint16_t *dst, size_t n);
void orc_dense_ffn(const uint16_t *gate, const uint16_t *up, const uint16_t *down, int inter,
                   const float *h_post, const float *h_in, float *out, float *act_out);
/* MLA attention of one decode token (infer.m:586-655, 766-903), see moe_ref.c. */
void orc_yarn_freq(float *freq);
float orc_mla_scale(void);
void orc_mla_append(const float *attn_norm, const uint16_t *kv_a, const float *kv_a_norm, const float *hidden,
                    float *cache_c, float *cache_k, int len, int pos);
void orc_mla_forward(const float *attn_norm, const uint16_t *q_a, const float *q_a_norm, const uint16_t *q_b,
                     const uint16_t *kv_a, const float *kv_a_norm, const uint16_t *k_b, const uint16_t *v_b,
                     const uint16_t *o_proj, float *hidden, float *cache_c, float *cache_k, int len, int pos);
void orc_expert_ffn(const void *blob, int down_is_q6, const float *x, float *out,
                    float *gate_out, float *up_out, float *act_out);

/* ---- router ---------------------------------------------------------- */
/* Router logits in the canonical summation order shared with the HIP
 * kernel (so that routing is bit-identical); infer.m:350-353 / 1881. */
void orc_router_logits(const float *Wg, const float *x, float *logits, int n_exp, int dim);
/* route(): infer.m:920-991, with n_group/topk_group/scale as parameters. */
void orc_route_ex(const float *logits, const float *bias, int n_exp, int n_group,
                  int topk_group, int K, float scale, int *exp_idx, float *exp_w);
void orc_route(const float *logits, const float *bias, int K, int *exp_idx, float *exp_w);
double orc_cpu_layer_tuned(const void *const *blobs, int K, int down_is_q6, const float *Wg, const float *bias,
                           const float *x, const float *h_in, float *out, int reps, int n_threads,
                           int *threads_used);

/* ---- MoE layer ------------------------------------------------------- */
/* The MoE branch of layer_forward for one token (infer.m:1878-1922):
 * logits -> route -> K routed experts + shared expert -> combine ->
 * hidden_out = h_in + moe_out + shared_out.  experts points at n_exp packed
 * expert blobs of expert_size bytes each.  Any of the optional outputs may
 * be NULL.  h_in may be NULL (treated as zeros). */
void orc_moe_layer(const void *experts, size_t expert_size, const float *Wg, const float *bias,
                   const void *shared_blob, const float *h_post, const float *h_in, int K,
                   float *hidden_out, int *idx_out, float *w_out, float *moe_out,
                   float *shared_out);
/* metal_moe_forward (infer.m:1604-1700) with routing given: moe_out =
 * sum_k w[k] * E_idx[k](h_post), summed in slot order. */
void orc_moe_forward(const void *experts, size_t expert_size, const float *h_post,
                     const int *exp_idx, const float *exp_w, int K, float *moe_out);

/* ---- seeded synthetic data (counter-based, splitmix64) --------------- */
uint64_t orc_rand_u64(uint64_t seed, uint64_t i);
void orc_synth_bytes(uint8_t *dst, size_t n, uint64_t seed);
void orc_synth_normal(float *dst, size_t n, float mean, float std, uint64_t seed);
void orc_synth_q4k(uint8_t *dst, size_t n_blocks, uint64_t seed);
void orc_synth_q6k(uint8_t *dst, size_t n_blocks, uint64_t seed);

/* ---- CPU baseline (reference-shaped expert path) ---------------------- */
/* Times the reference's CPU expert path on a bounded sample: n_experts
 * threads, each dequantising its expert's three matrices to fp32 scratch
 * and running three single-precision matvecs plus SiLU*mul, exactly the
 * work of expert_worker (infer.m:1069-1091) and shared_expert_worker.
 * Returns the median wall time in microseconds over `reps` runs and
 * writes the combined output to out (for a sanity check). */
double orc_cpu_expert_baseline(const void *const *blobs, int n_experts, int down_is_q6,
                               const float *x, const float *w, float *out, int reps,
                               int n_threads);
/* Router + route + K routed experts + shared expert + combine + residual,
 * K+1 threads (infer.m:1878-1922 with USE_CPU_EXPERTS). */
double orc_cpu_layer_baseline(const void *const *blobs, int K, int down_is_q6, const float *Wg,
                              const float *bias, const float *x, const float *h_in,
                              float *out, int reps);

#ifdef __cplusplus
}
#endif
#endif
