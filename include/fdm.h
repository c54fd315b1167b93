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
 *  - One device per process (fdm_init).  Intermediate vectors (activation
 *    digits, expert outputs, routing results) live in a workspace per
 *    stream, where the reference keeps one set of shared Metal buffers
 *    (infer.m:1351-1373): calls on different streams may overlap (see
 *    "streams and host threads" below).
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
#define FDM_E_FORMAT (-8)  /* malformed GGUF or layer file                  */

/* ---- lifecycle: replaces metal_init (infer.m:1276-1400) -------------------
 * fdm_init selects `device`, checks it is gfx950 and allocates the null
 * stream's workspace.  Unlike metal_init (1 = ok, 0 = unavailable) it returns FDM_OK
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

/* ---- streams and host threads ----------------------------------------------
 * Every call that needs scratch memory takes it from the workspace of its
 * stream: calls on one stream run in stream order and share it, calls on
 * different streams use different workspaces, so host threads that each use
 * their own stream may call concurrently.  The null stream's workspace is
 * made by fdm_init; another stream's at its first call, kept until
 * fdm_stream_release(stream) or fdm_shutdown (at most 64 streams at a time:
 * FDM_E_STATE beyond).  Release a stream's workspace before destroying the
 * stream if its handle may be reused.  Shared across streams, by design:
 * a streamed layer's expert cache (calls take turns), an attention layer's
 * KV cache (one sequence: one stream at a time), the scratch of
 * fdm_moe_forward_batched_noalloc, and the timing pool of fdm_prof_*.
 * (Concurrency rule of the reference: one GPU queue per process,
 * infer.m:1276-1400; no counterpart of fdm_stream_release.) */
int fdm_stream_release(void *stream);

/* ---- quant.h device twins (quant.h:11-15, quant.c:4-92) -------------------
 * Bit-exact with quant.c read as C with FP_CONTRACT off: every product and
 * difference rounds separately.  n must be a multiple of 256. */
int fdm_fp16_to_fp32(const uint16_t *d_src, float *d_dst, size_t n, void *stream);
/* the reverse, for the dense weights: (__fp16)x as f32_to_f16_alloc
 * (infer.m:521-528), round to nearest even, subnormals kept, NaN quieted. */
int fdm_f32_to_f16(const float *d_src, uint16_t *d_dst, size_t n, void *stream);
int fdm_dequant_q4k(const void *d_src, float *d_dst, size_t n, void *stream);
int fdm_dequant_q6k(const void *d_src, float *d_dst, size_t n, void *stream);

/* ---- fused dequant matvec: replaces enc_matvec_q with the
 * dequant_matvec_q4k / dequant_matvec_q6k kernels (infer.m:1525-1540,
 * shaders.metal:43-179).  y[r] = sum_c deq(W[r,c]) * x[c]; W is out_dim rows
 * of in_dim/256 blocks; in_dim must be a multiple of 256 and at most
 * FDM_HIDDEN * 4.  One launch (the digits of x and the rows) when in_dim is
 * 1024 n <= 7168 (Q4_K) or 2048 n <= 6144 (Q6_K), two otherwise; a bounded
 * wait inside the one-launch kernel that gives up is reported by
 * fdm_stream_sync (FDM_E_STATE). */
int fdm_matvec_q4k(const void *d_W, const float *d_x, float *d_y, uint32_t out_dim,
                   uint32_t in_dim, void *stream);
int fdm_matvec_q6k(const void *d_W, const float *d_x, float *d_y, uint32_t out_dim,
                   uint32_t in_dim, void *stream);

/* ---- one SwiGLU expert: replaces encode_expert (infer.m:1559-1575), i.e.
 * gate and up matvecs, swiglu_fused (shaders.metal:210-220) and the down
 * matvec.  expert_size selects the down type exactly as infer.m:1810-1821.
 * d_act (optional, 2048 floats) receives silu(gate) * up.  One launch (the
 * batch-1 layer kernel's work list without router; waits reported as for
 * fdm_moe_layer). */
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
 * The experts (and the shared expert) are copied into library-owned device
 * memory in the resident expert layout, a permutation of the packed blobs'
 * bytes that lets every load of the expert kernels read whole contiguous
 * lines (values unchanged); both calls are synchronous.
 * attach: from device buffers, which the caller may free after the call;
 *   d_Wg and d_bias stay the caller's and must live while the layer does.
 * upload: from host memory; the library owns every buffer.
 * d_shared / h_shared: the shared expert as one more packed blob (may be
 * NULL: no shared expert). */
int fdm_layer_attach(int L, const void *d_experts, size_t expert_size, int n_experts,
                     const float *d_Wg, const float *d_bias, const void *d_shared);
int fdm_layer_upload(int L, const void *h_experts, size_t expert_size, int n_experts,
                     const float *h_Wg, const float *h_bias, const void *h_shared);
int fdm_layer_release(int L);
int fdm_layer_query(int L, size_t *expert_size, int *down_is_q6, int *n_experts);

/* ---- real-weight ingest: GGUF shards (replaces gguf_load_manifest,
 * gguf_find, gguf_find_kv and gguf_tensor_pread, gguf.h:163-192,
 * gguf.c:285-551).  Host-side only; none of these calls needs fdm_init.
 * GGUF v2 and v3; general.alignment (u32 or u64, default 32) places the
 * data section.  Errors (FDM_E_FORMAT): bad magic or version, 0 or more
 * than 4 dims, a shape that is not whole blocks of its type, a tensor past
 * the end of its file, the same tensor name in two shards. */
typedef struct fdm_gguf fdm_gguf;

/* metadata value types (the GGUF format's) */
#define FDM_GGUF_UINT8 0
#define FDM_GGUF_INT8 1
#define FDM_GGUF_UINT16 2
#define FDM_GGUF_INT16 3
#define FDM_GGUF_UINT32 4
#define FDM_GGUF_INT32 5
#define FDM_GGUF_FLOAT32 6
#define FDM_GGUF_BOOL 7
#define FDM_GGUF_STRING 8
#define FDM_GGUF_ARRAY 9
#define FDM_GGUF_UINT64 10
#define FDM_GGUF_INT64 11
#define FDM_GGUF_FLOAT64 12

/* ggml tensor types used by the MoE path (ids are ggml's) */
#define FDM_GGML_F32 0
#define FDM_GGML_F16 1
#define FDM_GGML_Q4_K 12
#define FDM_GGML_Q6_K 14
#define FDM_GGML_BF16 30

typedef struct fdm_gguf_tensor_info {
  int type;           /* ggml type id */
  int n_dims;         /* 1..4 */
  uint64_t dims[4];   /* ne[0] (innermost) .. ne[3]; 1 beyond n_dims */
  uint64_t nbytes;    /* from type and shape */
  uint64_t offset;    /* absolute byte offset of the data in its shard file */
  int shard;          /* index into the paths given to fdm_gguf_open */
} fdm_gguf_tensor_info;

int fdm_gguf_open(const char *const *paths, int n_paths, fdm_gguf **out);
int fdm_gguf_close(fdm_gguf *m);
int fdm_gguf_count(const fdm_gguf *m, int *n_shards, uint64_t *n_tensors);
int fdm_gguf_shard_info(const fdm_gguf *m, int shard, uint32_t *version, uint64_t *alignment,
                        uint64_t *data_start, uint64_t *n_kv, uint64_t *n_tensors);
/* tensor by name (FDM_E_STATE if absent), or the i-th in shard, then file, order */
int fdm_gguf_find(const fdm_gguf *m, const char *name, fdm_gguf_tensor_info *info);
int fdm_gguf_tensor_at(const fdm_gguf *m, uint64_t i, char *name, size_t name_cap,
                       fdm_gguf_tensor_info *info);
/* metadata of one shard: type (FDM_GGUF_*), array element type and length */
int fdm_gguf_find_kv(const fdm_gguf *m, int shard, const char *key, int *type, int *arr_type,
                     uint64_t *arr_n);
int fdm_gguf_kv_int(const fdm_gguf *m, int shard, const char *key, int64_t *v);
int fdm_gguf_kv_float(const fdm_gguf *m, int shard, const char *key, double *v);
int fdm_gguf_kv_str(const fdm_gguf *m, int shard, const char *key, char *buf, size_t cap);
/* n bytes of a tensor starting `rel` bytes in, into host memory (FDM_E_INVAL
 * past the tensor's end) */
int fdm_gguf_read(const fdm_gguf *m, const char *name, void *h_buf, uint64_t n, uint64_t rel);
/* elements and bytes per block of a ggml type (ggml_blck_size / ggml_type_size) */
int fdm_ggml_type_geometry(int type, uint64_t *block_elems, uint64_t *block_bytes);

/* ---- a resident MoE layer straight from the model's files: replaces
 * repack_experts.c (stacked expert tensors -> per-expert blobs,
 * repack_experts.c:124-258) and the MoE part of load_layer_weights
 * (infer.m:1794-1823).  The library allocates the layer (as
 * fdm_layer_upload) and assembles the packed layout in HBM.
 *  - from GGUF: blk.L.ffn_{gate,up,down}_exps.weight (gate/up Q4_K
 *    [7168, 2048, 256], down Q4_K or Q6_K [2048, 7168, 256]: the down type is
 *    taken from the tensor, as repack_experts.c:140-155), the router
 *    blk.L.ffn_gate_inp.weight [7168, 256] and blk.L.exp_probs_b.bias (or
 *    .weight) [256] (F32, F16 or BF16, widened to fp32), and with
 *    with_shared the shared expert blk.L.ffn_{gate,up,down}_shexp.weight
 *    packed as one more blob (its down type must match the routed one).
 *  - from a packed layer file (repack_experts.c's layer_NN.bin, 256 blobs;
 *    the expert size and down type from the file size, infer.m:1806-1821),
 *    with the router, bias and shared expert from the GGUF.
 * Synchronous.  *down_is_q6 (optional) receives the layer's down type. */
int fdm_layer_load_gguf(int L, const fdm_gguf *m, int with_shared, int *down_is_q6);
int fdm_layer_load_packed(int L, const char *layer_file, const fdm_gguf *m, int with_shared,
                          int *down_is_q6);

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
 * routing.  One launch; its scratch is the stream's workspace, so calls on
 * different streams may overlap.  A launch whose internal waits
 * time out (never expected; it would mean a broken device) completes with
 * an unspecified result and makes the next fdm_stream_sync return
 * FDM_E_STATE. */
int fdm_moe_layer(int L, const float *d_h_post, const float *d_h_in, int K, float *d_hidden,
                  int *d_idx, float *d_w, void *stream);

/* ---- the same MoE branch with its rms_norm fused in (infer.m:1846-1850
 * and 1878-1922: h_in = hidden; h_post = rms_norm(hidden, ffn_norm_w);
 * hidden = h_in + moe + shared), in the same single launch:
 *   d_hidden = d_h + sum_k w[k] E_k(h_post) + S(h_post),
 *   h_post = rms_norm(d_h, d_norm_w), bit-exact with infer.m:369-374.
 * d_h, d_norm_w: [7168] fp32, 16-byte aligned; d_hidden may alias d_h;
 * d_h_post (optional) receives h_post and must not overlap d_h (FDM_E_INVAL:
 * the kernel writes it while other workgroups still read d_h).  Routing,
 * results and the rules for
 * overlapping calls are fdm_moe_layer's on that h_post. */
int fdm_moe_layer_norm(int L, const float *d_h, const float *d_norm_w, int K, float *d_hidden,
                       float *d_h_post, int *d_idx, float *d_w, void *stream);

/* ---- the streaming ceiling of a batch-1 layer's bytes (measurement only; no
 * counterpart in the reference).  One dependency-free launch that reads
 * exactly the bytes one fdm_moe_layer launch on layer L reads -- the router
 * weights and bias, the K routed experts d_idx[0..K) (device ints; an id
 * outside the layer reads expert 0), the shared expert, d_h_post and d_h_in
 * (may be NULL) -- with that kernel's load policy (16-byte nontemporal loads,
 * 64 KB per workgroup, four workgroups per CU), and writes FDM_HIDDEN words
 * to d_sink whose sum (mod 2^32) is the sum of every byte read.  No route, no
 * hand-off, no math: its time against fdm_moe_layer's separates the device's
 * streaming ceiling for these bytes from the kernel's own losses.
 * FDM_E_INVAL when the bytes exceed FDM_HIDDEN tiles of 64 KB (K = 16 with a
 * Q6_K down). */
int fdm_layer_read_ceiling(int L, const int *d_idx, int K, const float *d_h_post, const float *d_h_in,
                           uint32_t *d_sink, void *stream);

/* ---- the polls one wait inside fdm_moe_layer's kernel makes before it gives
 * up (no counterpart in the reference, whose Metal waits are host-side,
 * infer.m:1681).  0 restores the default (2^17 polls of >= ~1 us each).  A
 * small limit makes the waits give up from the host side -- every workgroup
 * still exits normally -- so the FDM_E_STATE report of fdm_stream_sync can be
 * exercised.  *prev (optional) receives the previous limit. */
int fdm_set_layer_spin_limit(unsigned polls, unsigned *prev);

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

/* ---- fdm_moe_forward_batched without allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and results as fdm_moe_forward_batched, but
 * every buffer of the step lives in one device array of the library
 * (FDM_NOALLOC_SCRATCH_BYTES, about 16 MiB per device, held until the
 * process ends) instead of the workspace fdm_moe_forward_batched grows on
 * demand; the call allocates nothing.  Limits: T <= FDM_NOALLOC_MAX_T and
 * T*K <= FDM_NOALLOC_MAX_PAIRS, else FDM_E_INVAL.  All calls on one device
 * share that array: calls that overlap on one device (on different
 * streams) race. */
#define FDM_NOALLOC_MAX_T 32
#define FDM_NOALLOC_MAX_PAIRS 256
#define FDM_NOALLOC_SCRATCH_BYTES 16949248ull
int fdm_moe_forward_batched_noalloc(int L, const float *d_X, const float *d_H_in, int T, int K,
                                    float *d_hidden, int *d_idx, float *d_w, int *d_n_distinct,
                                    void *stream);

/* Expert kernels behind fdm_moe_forward_batched (no counterpart in the
 * reference; a tuning and test switch).  FDM_BATCH_DOT4: per-token int8
 * digit dot products, each expert tile held in registers while its tokens
 * stream through LDS.  FDM_BATCH_MFMA: the grouped GEMMs on MFMA (exact
 * integer weights 1024 + sc*q in fp16, the activations as three fp16
 * planes: fp32 grade).  FDM_BATCH_AUTO: MFMA from FDM_BATCH_MFMA_MIN_T
 * tokens per step, DOT4 below.  Stores the previous mode in *prev when prev
 * is not NULL. */
#define FDM_BATCH_AUTO 0
#define FDM_BATCH_DOT4 1
#define FDM_BATCH_MFMA 2
#define FDM_BATCH_MFMA_MIN_T 12
int fdm_set_batch_kernel(int mode, int *prev);

/* ---- rms_norm on the device (infer.m:369-374, the h_post of infer.m:1850):
 * o[t] = x[t] * (1 / sqrt(sum_i x[t][i]^2 / d + 1e-6)) * w, bit-exact with
 * the reference's sequential loop.  d_w may be NULL (w = 1); d_o may alias
 * d_x.  [T][d] fp32, d <= 7168. */
int fdm_rms_norm(const float *d_x, const float *d_w, float *d_o, int T, int d, void *stream);

/* ---- prefill: T tokens through n_layers resident MoE layers,
 *   h <- h + MoE_l(rms_norm(h, norm_w[l]))   for l = 0 .. n_layers-1
 * (infer.m:1850, 1878-1922), in place on d_H [T][7168] fp32.  Routing is
 * route() per token on the fp32 rms_norm output (bit-exact); the Q4_K
 * expert GEMMs run on MFMA with fp32 accumulation, the weights as the exact
 * integers 1024 + sc*q in fp16 and the activations as one fp16 plane (a Q6_K
 * down runs on the digit kernels).  layers / d_norm_w: host arrays of
 * n_layers layer ids / device pointers to [7168] fp32.  d_idx (optional,
 * [n_layers][T][K]) receives every layer's routing.  1 <= T <= FDM_MAX_TOKENS. */
int fdm_moe_prefill(const int *layers, int n_layers, float *d_H, int T, int K,
                    const float *const *d_norm_w, int *d_idx, void *stream);

/* ---- streamed layers: the reference's expert streaming (infer.m:1478-1602:
 * route, then a parallel pread of the K selected experts from the packed
 * layer file, N_PREAD_CHUNKS chunks each, then the experts) for models whose
 * routed experts do not fit in HBM.  A streamed layer keeps the router
 * weights and bias (caller-owned device memory, as fdm_layer_attach) and a
 * library copy of the shared expert (packed blob, may be NULL) resident; its
 * routed experts stay in layer_file (repack_experts.c layout: expert e at
 * e * expert_size, n_experts = 256) and are read into an LRU cache of
 * n_cache expert slots in HBM (K <= n_cache <= 256; n_cache = 256 keeps
 * every expert once read).  n_threads host threads read (0: 8).
 * fdm_moe_layer_streamed computes the same layer as fdm_moe_layer: it
 * routes on the device (bit-exact), synchronises the stream to read the
 * routed ids, reads the missing experts, then runs the experts, the combine
 * and the residual on `stream`; it returns after queuing them.  Calls on
 * different streams take turns on the layer's cache (a fill waits for the
 * previous call's kernels).  Opening a layer streamed releases it as a
 * resident layer and the other way round; fdm_layer_release releases both.
 * fdm_stream_stats: cumulative cache hits and misses (routed experts) and
 * bytes read from the file. */
int fdm_layer_stream_open(int L, const char *layer_file, size_t expert_size, int n_experts,
                          const float *d_Wg, const float *d_bias, const void *d_shared, int n_cache,
                          int n_threads);
int fdm_moe_layer_streamed(int L, const float *d_h_post, const float *d_h_in, int K, float *d_hidden,
                           int *d_idx, float *d_w, void *stream);
int fdm_stream_stats(int L, uint64_t *hits, uint64_t *misses, uint64_t *bytes_read);

/* ---- MLA attention (mla_forward, infer.m:766-903) of one decode token:
 *   hidden <- hidden + W_o . MLA(rms_norm(hidden, attn_norm), pos)
 * with the latent KV cache (c_kv 512 + k_rope 64 per position, fp32) on the
 * device: q = W_qb . rms_norm(W_qa . x, q_a_norm) [128 heads][128 nope | 64
 * rope], kv = W_kva . x (rms_norm on the 512 latent dims), YaRN RoPE of the
 * rope parts at position pos (interleaved pairs, infer.m:586-655), the
 * absorbed scores scale (k_b[h] . q_nope[h]) . c_kv + scale q_rope . k_rope
 * with scale = mscale^2 / sqrt(192), mscale = 0.1 ln 40 + 1, softmax over
 * the cache, the latent weighted sum, v_b per head and o_proj.  Weights in
 * the layout LayerAttnDense holds them (infer.m:687-706), row-major; the
 * library keeps its own copy (synchronous upload).  Each fdm_attn_forward
 * appends the token at the cache's next row (fdm_attn_reset empties it);
 * max_seq <= FDM_ATTN_MAX_SEQ.  An attention layer holds one sequence: its
 * calls belong on one stream (its cache length is host state). */
#define FDM_ATTN_MAX_SEQ 16384 /* MAX_SEQ, infer.m:67 */
typedef struct fdm_attn_weights {
  const float *attn_norm;  /* [7168]                                 */
  const uint16_t *q_a;     /* F16 [1536][7168]                       */
  const float *q_a_norm;   /* [1536]                                 */
  const uint16_t *q_b;     /* F16 [128 * 192][1536]                  */
  const uint16_t *kv_a;    /* F16 [576][7168]                        */
  const float *kv_a_norm;  /* [512]                                  */
  const uint16_t *k_b;     /* F16 [128][512][128]: per head (KV_LORA, NOPE) */
  const uint16_t *v_b;     /* F16 [128][128][512]: per head (V_HEAD, KV_LORA) */
  const uint16_t *o_proj;  /* F16 [7168][128 * 128]                  */
} fdm_attn_weights;
int fdm_attn_upload(int L, const fdm_attn_weights *host_weights, int max_seq);
/* From the model file: blk.L.attn_{norm,q_a,q_a_norm,q_b,kv_a_mqa,kv_a_norm,
 * output}.weight and attn_k_b / attn_v_b (or attn_kv_b), converted as
 * load_layer_weights does (infer.m:1736-1778: norms widened to fp32,
 * matrices through dequant_tensor_f16, k_b transposed per head). */
int fdm_attn_load_gguf(int L, const fdm_gguf *m, int max_seq);
int fdm_attn_forward(int L, float *d_hidden, int pos, void *stream);
int fdm_attn_reset(int L);
int fdm_attn_len(int L, int *len);
int fdm_attn_release(int L);

/* ---- dense FFN layers (the layers before the first MoE layer, L < 3 in
 * R1): replaces the dense branch of layer_forward (infer.m:1852-1868),
 *   hidden = h_in + W_down . (silu(W_gate . h_post) * (W_up . h_post)),
 * with F16 weights and fp32 activations and accumulation as mv_f16
 * (infer.m:459-513).  The weights are held as dequant_tensor_f16 leaves
 * them (infer.m:530-538, 1786-1792): row-major F16, gate and up
 * [inter][7168], down [7168][inter]; inter = DENSE_INTERMEDIATE (18432) in
 * R1, any multiple of 512 up to it is accepted.  The library keeps its own
 * copy of the weights (upload: from host, attach: from device; both
 * synchronous, the caller's buffers may be freed afterwards).
 * fdm_dense_load_gguf reads blk.L.ffn_{gate,up,down}.weight (F32, F16,
 * BF16, Q4_K or Q6_K, as dequant_tensor_full, infer.m:314-355), widens to
 * fp32 and rounds to F16 on the device, bit-exact with the reference's
 * (__fp16) cast; *inter receives the intermediate size (may be NULL).
 * fdm_dense_ffn: d_h_post 16-byte aligned, d_h_in may be NULL (no residual),
 * d_hidden must not alias d_h_post; its activations live in the stream's
 * workspace. */
#define FDM_DENSE_FFN 18432
int fdm_dense_upload(int L, const uint16_t *h_gate, const uint16_t *h_up, const uint16_t *h_down,
                     int inter);
int fdm_dense_attach(int L, const uint16_t *d_gate, const uint16_t *d_up, const uint16_t *d_down,
                     int inter);
int fdm_dense_load_gguf(int L, const fdm_gguf *m, int *inter);
int fdm_dense_release(int L);
int fdm_dense_query(int L, int *inter);
int fdm_dense_ffn(int L, const float *d_h_post, const float *d_h_in, float *d_hidden, void *stream);

/* ---- per-kernel GPU timing: replaces the host-clock moe_prof_t ring
 * (infer.m:177-261) with HIP events recorded on the launch stream around
 * every kernel of the entry points above.  fdm_prof_read synchronises on
 * the recorded events and returns the count, total, min and max duration
 * (milliseconds) of one phase since the last reset. */
#define FDM_PROF_ROUTER 0   /* fdm_router_logits / fdm_route kernels    */
#define FDM_PROF_GATEUP 1   /* gate/up matvecs + SwiGLU (routing given); fdm_expert_ffn */
#define FDM_PROF_DOWN 2     /* down matvecs + combine (routing given)   */
#define FDM_PROF_XDIGITS 3  /* activation digits (routing given)        */
#define FDM_PROF_MATVEC 4   /* fdm_matvec_q4k / _q6k kernel             */
#define FDM_PROF_LAYER 5    /* fdm_moe_layer: the whole layer, 1 launch */
#define FDM_PROF_BATCH 6    /* fdm_moe_forward_batched: the whole step  */
#define FDM_PROF_PREFILL 7  /* fdm_moe_prefill: all layers              */
#define FDM_PROF_DENSE 8    /* fdm_dense_ffn: both launches             */
#define FDM_PROF_ATTN 9     /* fdm_attn_forward: the whole token        */
#define FDM_PROF_CEILING 10 /* fdm_layer_read_ceiling                   */
#define FDM_PROF_PHASES 11
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
