/*
 * fdm.h -- C ABI of the MI355X (gfx950) MoE expert hot path.
 *
 * This library replaces the Metal dispatch of the reference's inference
 * program (infer.m "Metal GPU MoE" and "Per-expert pipeline" sections) with
 * hand-written HIP kernels.  The host keeps the reference's quant.h block
 * formats and its packed-expert layout; it calls the GPU only through the
 * functions below.  Each declaration cites the reference interface it
 * replaces.
 *
 * Conventions
 *  - Every function returns int: FDM_OK (0) or a negative FDM_E* code.  No
 *    function aborts.  fdm_last_error() gives a thread-local description.
 *  - Pointers named d_* are device pointers; h_* are host pointers.
 *  - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *    Launches are asynchronous on that stream unless stated otherwise.
 *  - One device per process (fdm_init).  The library keeps one workspace
 *    per device for intermediate vectors (activation digits, expert
 *    outputs, routing results), as the reference keeps one set of shared
 *    Metal buffers (infer.m:1351-1373): calls that overlap in time on
 *    different streams of the same device race on it.
 *  - Layouts are the reference's: Q4_K 144-byte and Q6_K 210-byte blocks of
 *    256 weights (quant.h:6-8), matrices row-major with in_dim/256 blocks
 *    per row, a packed expert = [gate Q4_K 2048x7168 | up Q4_K | down Q4_K
 *    or Q6_K 7168x2048] (infer.m:69-78, repack_experts.c:157-160).
 */
#ifndef FDM_H
#define FDM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- constants (quant.h:6-8, infer.m:41-80) ------------------------------ */
#define FDM_QK_K 256
#define FDM_Q4K_BLOCK_SIZE 144
#define FDM_Q6K_BLOCK_SIZE 210
#define FDM_HIDDEN 7168
#define FDM_MOE_FFN 2048
#define FDM_N_EXPERTS 256
#define FDM_N_GROUP 8
#define FDM_TOPK_GROUP 4
#define FDM_MAX_K 16
#define FDM_MAX_LAYERS 61
#define FDM_MAX_TOKENS 512
#define FDM_EXPERT_Q4K_BYTES 24772608ull /* 2 x 8,257,536 + 8,257,536  */
#define FDM_EXPERT_Q6K_BYTES 28557312ull /* 2 x 8,257,536 + 12,042,240 */

/* ---- error codes --------------------------------------------------------- */
#define FDM_OK 0
#define FDM_E_INVAL (-1)   /* bad argument (null pointer, size, K, index)   */
#define FDM_E_NODEV (-2)   /* no usable HIP device                          */
#define FDM_E_HIP (-3)     /* a HIP runtime call failed                     */
#define FDM_E_STATE (-4)   /* fdm_init not called / layer not resident      */
#define FDM_E_NOMEM (-5)   /* device allocation failed                      */
#define FDM_E_SIZE (-6)    /* expert size matches neither R1 layout          */
#define FDM_E_IO (-7)      /* file open/read failed (host ingest)           */

/* ---- lifecycle: replaces metal_init (infer.m:1276-1400) -------------------
 * fdm_init selects `device`, checks it is gfx950 and allocates the
 * workspace.  Unlike metal_init (1 = ok, 0 = unavailable) it returns FDM_OK
 * or an error code; fdm_available() gives the reference's 1/0 answer. */
int fdm_init(int device);
int fdm_shutdown(void);
int fdm_available(void);
const char *fdm_strerror(int code);
const char *fdm_last_error(void);
/* Number of compute units of the initialised device (grid sizing info). */
int fdm_device_cus(void);

/* ---- memory helpers (so a C host needs no HIP headers) ------------------- */
int fdm_malloc(void **d_ptr, size_t bytes);
int fdm_free(void *d_ptr);
int fdm_memcpy_h2d(void *d_dst, const void *h_src, size_t bytes, void *stream);
int fdm_memcpy_d2h(void *h_dst, const void *d_src, size_t bytes, void *stream);
int fdm_stream_sync(void *stream);

/* ---- quant.h device twins (quant.h:11-15, quant.c:4-92) -------------------
 * Bit-exact with quant.c read as C with FP_CONTRACT off: every product and
 * difference rounds separately.  n must be a multiple of 256. */
int fdm_fp16_to_fp32(const uint16_t *d_src, float *d_dst, size_t n, void *stream);
int fdm_dequant_q4k(const void *d_src, float *d_dst, size_t n, void *stream);
int fdm_dequant_q6k(const void *d_src, float *d_dst, size_t n, void *stream);

/* ---- fused dequant matvec: replaces enc_matvec_q with the
 * dequant_matvec_q4k / dequant_matvec_q6k kernels (infer.m:1525-1540,
 * shaders.metal:43-179).  y[r] = sum_c deq(W[r,c]) * x[c]; W is out_dim rows
 * of in_dim/256 blocks; in_dim must be a multiple of 256 and at most
 * FDM_HIDDEN * 4. */
int fdm_matvec_q4k(const void *d_W, const float *d_x, float *d_y, uint32_t out_dim,
                   uint32_t in_dim, void *stream);
int fdm_matvec_q6k(const void *d_W, const float *d_x, float *d_y, uint32_t out_dim,
                   uint32_t in_dim, void *stream);

/* ---- one SwiGLU expert: replaces encode_expert (infer.m:1559-1575), i.e.
 * gate and up matvecs, swiglu_fused (shaders.metal:210-220) and the down
 * matvec.  expert_size selects the down type exactly as infer.m:1810-1821.
 * d_act (optional, 2048 floats) receives silu(gate) * up. */
int fdm_expert_ffn(const void *d_blob, size_t expert_size, const float *d_x, float *d_out,
                   float *d_act, void *stream);

/* ---- router: replaces the router sgemv (infer.m:350-353, 1881) and
 * route() (infer.m:920-991).  Logits use a fixed summation order (so that a
 * CPU restatement reproduces them bit for bit); route reproduces the
 * reference's selection, tie rules and slot order exactly.  T tokens,
 * row-major: d_x is T x dim, d_logits T x n_exp, d_idx / d_w T x K. */
int fdm_router_logits(const float *d_Wg, const float *d_x, int n_exp, int dim, int T,
                      float *d_logits, void *stream);
int fdm_route(const float *d_logits, const float *d_bias, int T, int K, int *d_idx,
              float *d_w, void *stream);

/* ---- resident layers: replaces load_layer_weights' MoE part
 * (infer.m:1794-1823) and the per-token pread of the selected experts
 * (infer.m:1577-1602): all experts of a layer stay resident in HBM.
 * expert_size must be FDM_EXPERT_Q4K_BYTES or FDM_EXPERT_Q6K_BYTES.
 * attach: the caller keeps ownership of the device buffers.
 * upload: the library allocates and copies from host memory.
 * d_shared / h_shared: the shared expert as one more packed blob (may be
 * NULL: no shared expert). */
int fdm_layer_attach(int L, const void *d_experts, size_t expert_size, int n_experts,
                     const float *d_Wg, const float *d_bias, const void *d_shared);
int fdm_layer_upload(int L, const void *h_experts, size_t expert_size, int n_experts,
                     const float *h_Wg, const float *h_bias, const void *h_shared);
int fdm_layer_release(int L);
int fdm_layer_query(int L, size_t *expert_size, int *down_is_q6, int *n_experts);

/* ---- MoE forward with routing given: replaces metal_moe_forward
 * (infer.m:1604-1700).  moe_out = sum_k w[k] * E_{idx[k]}(h_post), summed in
 * slot order.  K <= FDM_MAX_K.  Device pointers, asynchronous. */
int fdm_moe_forward(int L, const float *d_h_post, const int *d_idx, const float *d_w, int K,
                    float *d_moe_out, void *stream);
/* Same with the reference's exact calling convention: host pointers,
 * synchronous, moe_out overwritten. */
int fdm_moe_forward_host(int L, const float *h_post, const int *exp_idx, const float *exp_w,
                         int K, float *moe_out);

/* ---- the whole MoE branch of layer_forward on the device
 * (infer.m:1878-1922): router logits, route, K routed experts plus the
 * shared expert, combine, and the residual:
 *   hidden = h_in + sum_k w[k] E_k(h_post) + S(h_post).
 * d_h_in may be NULL (no residual).  d_idx / d_w (optional) receive the
 * routing.  One cooperative launch; calls on one device must not overlap
 * (they share the library's workspace).  A launch whose internal waits
 * time out (never expected; it would mean a broken device) completes with
 * an unspecified result and makes the next fdm_stream_sync return
 * FDM_E_STATE. */
int fdm_moe_layer(int L, const float *d_h_post, const float *d_h_in, int K, float *d_hidden,
                  int *d_idx, float *d_w, void *stream);

/* Kernel behind fdm_moe_layer (no counterpart in the reference, which has
 * one Metal path; a tuning and test switch): FDM_LAYER_ITEMS runs the
 * ordered work list, FDM_LAYER_STREAM streams the layer through 256
 * resident workgroups (fails with FDM_E_INVAL on a device with fewer than
 * 256 CUs) and FDM_LAYER_AUTO picks the faster one, currently ITEMS.
 * Stores the previous mode in *prev when prev is not NULL. */
#define FDM_LAYER_AUTO 0
#define FDM_LAYER_ITEMS 1
#define FDM_LAYER_STREAM 2
int fdm_set_layer_kernel(int mode, int *prev);

/* ---- batched decode: T tokens through the MoE branch of layer L in one
 * step, with token -> expert dispatch so that each selected expert's weights
 * are read once per step (config 3; the reference decodes one token at a
 * time, infer.m:2219-2229).  Per token t the result is fdm_moe_layer's:
 *   hidden[t] = h_in[t] + sum_k w[t][k] E_k(h_post[t]) + S(h_post[t])
 * with route() per token (bit-exact idx / w).  d_X, d_H_in, d_hidden:
 * [T][7168] fp32 (d_H_in may be NULL).  d_idx / d_w ([T][K], optional)
 * receive the routing; d_n_distinct (optional, device int) the number of
 * distinct routed experts of the step.  1 <= T <= FDM_MAX_TOKENS. */
int fdm_moe_forward_batched(int L, const float *d_X, const float *d_H_in, int T, int K,
                            float *d_hidden, int *d_idx, float *d_w, int *d_n_distinct,
                            void *stream);

/* ---- rms_norm on the device (infer.m:369-374, the h_post of infer.m:1850):
 * o[t] = x[t] * (1 / sqrt(sum_i x[t][i]^2 / d + 1e-6)) * w, bit-exact with
 * the reference's sequential loop.  d_w may be NULL (w = 1); d_o may alias
 * d_x.  [T][d] fp32, d <= 7168. */
int fdm_rms_norm(const float *d_x, const float *d_w, float *d_o, int T, int d, void *stream);

/* ---- prefill: T tokens through n_layers resident MoE layers,
 *   h <- h + MoE_l(rms_norm(h, norm_w[l]))   for l = 0 .. n_layers-1
 * (infer.m:1850, 1878-1922), in place on d_H [T][7168] fp32.  Routing is
 * route() per token on the fp32 rms_norm output (bit-exact); the expert
 * GEMMs dequantise Q4_K to bf16 and run on MFMA with fp32 accumulation
 * (layers must have Q4_K down).  layers / d_norm_w: host arrays of
 * n_layers layer ids / device pointers to [7168] fp32.  d_idx (optional,
 * [n_layers][T][K]) receives every layer's routing.  1 <= T <= FDM_MAX_TOKENS. */
int fdm_moe_prefill(const int *layers, int n_layers, float *d_H, int T, int K,
                    const float *const *d_norm_w, int *d_idx, void *stream);

/* ---- per-kernel GPU timing: replaces the host-clock moe_prof_t ring
 * (infer.m:177-261) with HIP events recorded on the launch stream around
 * every kernel of the entry points above.  fdm_prof_read synchronises on
 * the recorded events and returns the count, total, min and max duration
 * (milliseconds) of one phase since the last reset. */
#define FDM_PROF_ROUTER 0   /* fdm_router_logits / fdm_route kernels    */
#define FDM_PROF_GATEUP 1   /* gate/up matvecs + SwiGLU (routing given) */
#define FDM_PROF_DOWN 2     /* down matvecs + combine (routing given)   */
#define FDM_PROF_XDIGITS 3  /* activation digits (routing given)        */
#define FDM_PROF_MATVEC 4   /* fdm_matvec_q4k / _q6k kernel             */
#define FDM_PROF_LAYER 5    /* fdm_moe_layer: the whole layer, 1 launch */
#define FDM_PROF_BATCH 6    /* fdm_moe_forward_batched: the whole step  */
#define FDM_PROF_PREFILL 7  /* fdm_moe_prefill: all layers              */
#define FDM_PROF_PHASES 8
int fdm_prof_enable(int on);
int fdm_prof_reset(void);
int fdm_prof_read(int phase, int *count, double *total_ms, double *min_ms, double *max_ms);

/* ---- seeded synthetic tensors (benchmark inputs; same generator as the
 * C restatement's synth.c) ---------------------------------------------- */
int fdm_synth_q4k(void *d_dst, size_t n_blocks, uint64_t seed, void *stream);
int fdm_synth_q6k(void *d_dst, size_t n_blocks, uint64_t seed, void *stream);
int fdm_synth_normal(float *d_dst, size_t n, float mean, float std_dev, uint64_t seed,
                     void *stream);

#ifdef __cplusplus
}
#endif
#endif /* FDM_H */
