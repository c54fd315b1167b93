// fdm_internal.h -- launchers shared between the kernel translation units
// and the C ABI (capi.hip).  All launchers are asynchronous on `stream` and
// return the hipError_t of the launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <functional>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "fdm_device.h"

struct fdm_gguf;  // the C ABI's opaque manifest handle

namespace fdm {

// quant_kernels.hip
hipError_t launch_fp16_to_fp32(const uint16_t* src, float* dst, size_t n, hipStream_t s);
hipError_t launch_dequant_q4k(const uint8_t* src, float* dst, size_t n_blocks, hipStream_t s);
hipError_t launch_dequant_q6k(const uint8_t* src, float* dst, size_t n_blocks, hipStream_t s);
// n packed expert blobs (src + b * src_stride) -> the resident expert layout
// (dst + b * expert_size): gate, up and a Q4_K down permuted, a Q6_K down copied.
hipError_t launch_rel_pack(const uint8_t* src, size_t src_stride, uint8_t* dst, size_t expert_size,
                           int n_blobs, bool down_q6, hipStream_t s);

// matvec_kernels.hip
// Digits of `n_groups` consecutive 64-element groups of x.
hipError_t launch_xdigits(const float* x, size_t n_groups, XGroup* xd, hipStream_t s);
hipError_t launch_matvec_q4k(const uint8_t* W, const XGroup* xd, float* y, int rows,
                             int in_dim, hipStream_t s);
hipError_t launch_matvec_q6k(const uint8_t* W, const XGroup* xd, float* y, int rows,
                             int in_dim, hipStream_t s);
// One launch: the digits of x, then the rows (work list, see matvec_kernels.hip).
struct MatvecArgs {
  const uint8_t* W;   // Q4_K or Q6_K rows, packed
  const float* x;     // [in_dim]
  float* y;           // [rows]
  int rows, gr;       // output rows, 64-element groups per row (in_dim / 64)
  XGroup* xd;         // workspace: the digit records of x [gr]
  int* counter;       // arrivals of the digit items (zero at first use, left zero)
  unsigned* flag;     // set to epoch by the last digit item
  unsigned* err;      // receives epoch when a wait gives up
  unsigned epoch, spin_limit;
};
// false when this in_dim has no one-launch kernel (the caller then runs
// launch_xdigits + launch_matvec_q4k / q6k)
// Q4_K by column parts of 1024 (see matvec_kernels.hip): in_dim = 1024 P,
// P <= 7; part holds (P - 1) x rows tagged partial sums.
struct Matvec2Args {
  const uint8_t* W;
  const float* x;
  float* y;
  int rows;
  uint64_t* part;   // workspace: tagged partial sums [P - 1][rows]
  unsigned* err;    // receives epoch when a wait gives up
  unsigned epoch, spin_limit;
};
bool matvec2_supported(int in_dim, int rows, size_t part_words);
hipError_t launch_matvec2_q4k(const Matvec2Args& a, int in_dim, hipStream_t s);
bool matvec1_supported(bool q6, int in_dim);
bool matvec3_supported(int in_dim);
hipError_t launch_matvec3_q4k(const uint8_t* W, const float* x, float* y, int rows, int in_dim, hipStream_t s);
hipError_t launch_matvec1(const MatvecArgs& a, bool q6, hipStream_t s);

// router_kernels.hip
hipError_t launch_router_logits(const float* Wg, const float* x, int n_exp, int dim, int T,
                                float* logits, hipStream_t s);
hipError_t launch_route(const float* logits, const float* bias, int T, int K, int* idx,
                        float* w, hipStream_t s);

// moe_kernels.hip
struct SlotTable {
  const uint8_t* experts;  // n_experts packed blobs
  size_t expert_size;
  int n_experts;
  const uint8_t* shared;   // slot K (may be null)
  const int* idx;          // K routed expert ids (device), one per slot
  const float* w;          // K routing weights (device)
  int K;                   // routed slots
  int n_slots;             // K or K + 1 (shared)
  bool rel;                // blobs in the resident expert layout (else packed)
  int slot0 = 0;           // the first slot a launch runs (set by the launch functions)
  uint32_t skip = 0;       // bit k: slot k is not run by this launch (another launch runs it)
};
// gate/up matvecs + SwiGLU for slots slot0 .. slot0 + n_run - 1 (n_run < 0:
// every slot), except those t.skip names; writes act[slot][2048] and the digits of act
// (act_xd[slot][32]).  counters: (FDM_MAX_K + 1) x 64 ints, zero on entry
// and left zero.
hipError_t launch_gateup(const SlotTable& t, const XGroup* xd, float* act, XGroup* act_xd,
                         int* counters, hipStream_t s, int slot0 = 0, int n_run = -1);
// down matvecs for slots slot0 .. slot0 + n_run - 1 (n_run < 0: every slot),
// except those t.skip names, into eo[slot][7168]; the launches of one call
// may split the slots
// between them, and whichever launch completes a row tile's n_slots-th
// slot combines it:
//   out[i] = (h_in[i] + sum_{k<K} w[k] * E_k[i]) + S[i]
// moe_out (optional) receives sum_k w[k] * E_k[i].  counters: 448 ints,
// zero on entry and left zero once every slot of the call has run.
hipError_t launch_down_combine(const SlotTable& t, bool down_q6, const XGroup* act_xd,
                               const float* h_in, float* out, float* moe_out, float* eo,
                               int* counters, hipStream_t s, int slot0 = 0, int n_run = -1);

// layer_kernel.hip
// The batch-1 MoE layer of one token in one launch: digits, router, route,
// shared + routed experts, combine, residual.  Values handed between
// workgroups are tagged 64-bit words {epoch, payload}.
constexpr int kLayerStride = 64;                 // ints between counters / flags
constexpr int kLayerMaxSlots = 17;               // FDM_MAX_K routed + 1 shared
constexpr int kLayerCounters = 1;                // arrivals of the digit items
constexpr int kLayerFlags = 4;                   // digits ready, -, error, -
constexpr int kLayerFlagErr = 2;                 // flag slot of the timed-out epoch
constexpr int kLayerMaxParts = 8;               // down matrices split in <= 8 column parts
// tagged words: scores 256, prov 16, route_w 16, route_perm 16,
// act 17 x 2048, eo 17 x 8 x 7168 (per-part down outputs), act_xd 17 x 32 x 52
// (the words of the activations' digit records)
constexpr size_t kLayerActXdWords = (size_t)kLayerMaxSlots * 32 * (sizeof(XGroup) / 4);
constexpr size_t kLayerTagged = 256 + 3 * 16 +
                                (size_t)kLayerMaxSlots * (2048 + (size_t)kLayerMaxParts * 7168) +
                                kLayerActXdWords + 16;  // + the rms line
struct LayerArgs {
  const float* Wg;         // router weights [256][7168] fp32
  const float* bias;       // [256] or null
  const float* h;          // h_post [7168]; with norm_w: the hidden state h_post is the rms_norm of
  const float* norm_w = nullptr;  // or the rms_norm weight [7168]: h_post = rms_norm(h, norm_w) inside
  float* h_post_out = nullptr;    // or receives h_post [7168] (with norm_w)
  uint64_t* norm_inv = nullptr;   // tagged: 1 / sqrt(mean h^2 + eps) of the fused rms_norm
  const float* h_in;       // residual [7168] or null
  float* out;              // hidden = h_in + moe + shared [7168]
  float* moe_out;          // sum_k w_k E_k [7168] or null
  const uint8_t* experts;  // n_experts packed blobs
  size_t expert_size;
  int n_experts;
  const uint8_t* shared;   // shared expert blob or null
  int down_q6;
  int K;                   // routed experts
  int n_slots;             // K (+1 with a shared expert)
  int* idx;                // out: route() slot order [K]
  float* w;                // out: route() weights [K]
  XGroup* xd;              // workspace: digits of h [112]
  uint64_t* scores;        // tagged: 256 sigmoid scores
  uint64_t* prov;          // tagged: the expert set, one per slot [K]
  uint64_t* route_w;       // tagged: weights in the reference's slot order [K]
  uint64_t* route_perm;    // tagged: slot running the k-th expert of that order [K]
  uint64_t* act;           // tagged: [kLayerMaxSlots][2048]
  uint64_t* eo;            // tagged: [kLayerMaxSlots][kLayerMaxParts][7168] down partial sums
  uint64_t* act_xd;        // tagged: [kLayerMaxSlots][32][52] words of the activations' digit records
  int* counters;           // kLayerCounters x kLayerStride ints, zero at first use
  unsigned* flags;         // kLayerFlags x kLayerStride, zero at first use
  unsigned epoch;          // non-zero, different from every earlier call's
  unsigned spin_limit;     // polls before a wait gives up (kLayerSpinLimit)
  float* act_out = nullptr;  // launch_expert_f32: receives the SwiGLU activations [2048] (or null)
};
constexpr unsigned kLayerSpinLimit = 1u << 17;  // polls of one wait (each >= ~1 us)
hipError_t launch_layer(const LayerArgs& a, hipStream_t s);
// expert_kernels.hip: one expert with a Q4_K down matrix in one fp32 launch
// (a.shared: the caller's packed blob; a.act, a.epoch, a.flags, a.spin_limit).
hipError_t launch_expert_f32(const LayerArgs& a, hipStream_t s);

// read_ceiling.hip: the batch-1 layer's bytes read with the layer kernel's
// load policy and nothing else (the streaming ceiling of those bytes).
// Segment s covers tiles tile0[s] .. tile0[s + 1] - 1 of 64 KB; segments
// first_routed .. first_routed + K - 1 are the routed experts idx[k]
// (device ids, resolved in the kernel).
constexpr int kReadCeilMaxSeg = 4 + 1 + 16;
struct ReadCeilArgs {
  const uint8_t* seg[kReadCeilMaxSeg];
  size_t bytes[kReadCeilMaxSeg];
  int tile0[kReadCeilMaxSeg + 1];
  int n_seg, first_routed, K, n_tiles;
  const uint8_t* experts;
  size_t expert_size;
  int n_experts;   // an id outside 0 .. n_experts - 1 reads expert 0
  const int* idx;
  uint32_t* sink;  // [7168]
};
int read_ceiling_tiles(size_t bytes);
hipError_t launch_read_ceiling(const ReadCeilArgs& a, hipStream_t s);

// batched_kernels.hip
// Batched decode of T tokens through one layer with token -> expert
// dispatch (each selected expert's weights read once per step).  Routing
// (idx, w: [T][K]) is computed beforehand by the router kernels.
struct BatchArgs {
  int T, K;
  const uint8_t* experts;  // 256 packed blobs
  size_t expert_size;
  const uint8_t* shared;   // shared expert blob or null
  const float* x;          // h_post [T][7168]
  const float* h_in;       // residual [T][7168] or null
  float* out;              // hidden [T][7168]
  const int* idx;          // [T][K]
  const float* w;          // [T][K]
  XGroup* xd;              // workspace: digits of x [T][112]
  float* act;              // workspace: [rows][2048], rows = T*K (+ T shared)
  XGroup* act_xd;          // workspace: [rows][32]
  float* eo;               // workspace: [rows][7168]
  int* seg_start;          // workspace: [257] pair segment of each expert
  int* pair_tok;           // workspace: [T*K] token of each pair position
  int* pair_of;            // workspace: [T*K] position of pair (t, k), -1 if invalid id
  int* distinct;           // workspace: [256] distinct experts, ascending
  int* n_distinct;         // out: number of distinct experts (device int)
  // optional: the dispatch also writes the grouped GEMMs' chunk list (ch > 0)
  int ch = 0;              // tokens per chunk
  int4* chunks = nullptr;  // {expert or -1 (shared), first pair / token, count, first chunk | count << 16}
  int* n_chunks = nullptr;
};
hipError_t launch_batched_experts(const BatchArgs& b, bool down_q6, hipStream_t s);
// The grouped down (digits of b.act, then the dot4 down kernel) on its own.
hipError_t launch_batched_down(const BatchArgs& b, bool down_q6, hipStream_t s);
// The dispatch and the combine of the batched path on their own (prefill).
hipError_t launch_dispatch(const BatchArgs& b, hipStream_t s);
hipError_t launch_combine(const BatchArgs& b, hipStream_t s);

// prefill_kernels.hip
// rms_norm per token (infer.m:369-374), bit-exact: o = x * inv * w.  d <= 7168.
hipError_t launch_rms_norm(const float* x, const float* w, float* o, int T, int d, hipStream_t s);
// rms_norm of T tokens of 7168 (o, as launch_rms_norm) and the one-plane
// activation planes of o for the grouped GEMMs (launch_xplanes, planes = 1).
hipError_t launch_rms_norm_planes(const float* x, const float* w, float* o, int T, _Float16* xp, float* xs,
                                  float* xe, hipStream_t s);

// gemm_kernels.hip: grouped expert GEMMs (batched decode, prefill) on MFMA.
// Rows: pair position p (routed), T*K + t (shared expert of token t).
struct QGemmArgs {
  int T, K;
  const uint8_t* experts;  // resident expert layout
  size_t expert_size;
  const uint8_t* shared;
  const _Float16* xp;      // activation planes [P][plane]: input row r at r * kd
  size_t plane;            // elements per plane
  const float* xs;         // [rows][kd / 32] sub-block sums of the planes
  const float* xe;         // [rows] 2^-s of each input row
  const int* pair_tok;     // token of each pair position (gate/up input rows)
  const int4* chunks;      // {expert or -1, first pair / token, count, first chunk | count << 16}
  const int* n_chunks;
  float* out;              // gate/up: act [rows][2048] (SwiGLU); down: eo [rows][7168]
};
// n_rows x [kd] fp32 -> `planes` (1 or 3) fp16 planes of x * 2^s, the
// sub-block sums and 2^-s per row.
hipError_t launch_xplanes(const float* x, int kd, size_t n_rows, int planes, _Float16* xp, float* xs, float* xe,
                          hipStream_t s);
int qgemm_chunk_tokens(int planes);
constexpr int kQMaxChunks = 1024;  // >= 256 + 512 * 16 / 16 + 512 / 16
// Q4_K gate/up + SwiGLU (down = false) or Q4_K down (down = true) over the
// chunk list; max_chunks bounds the list length.
hipError_t launch_qgemm(const QGemmArgs& g, int planes, bool down, int max_chunks, hipStream_t s);

// dense_kernels.hip: the dense FFN of the first layers (F16 weights)
constexpr int kDenseMaxFfn = 18432;  // DENSE_INTERMEDIATE (infer.m:59): the down kernel's LDS bound
constexpr int kGgmlF32 = 0, kGgmlF16 = 1, kGgmlBF16 = 30;  // ggml type ids of k_to_f16's inputs
struct DenseArgs {
  const uint16_t *gate, *up, *down;  // F16 row-major: [inter][7168] x 2, [7168][inter]
  const float* x;                    // h_post [7168]
  const float* h_in;                 // residual [7168] or null
  float* act;                        // workspace [inter]
  float* out;                        // [7168]
  int inter;                         // multiple of 512, <= kDenseMaxFfn
  int n_cus;
};
hipError_t launch_dense_ffn(const DenseArgs& a, hipStream_t s);
// n elements of ggml type F32 / BF16 / F16 -> F16 bits (round to nearest even)
hipError_t launch_to_f16(const void* src, int type, uint16_t* dst, size_t n, hipStream_t s);
// dst[h][c][r] = src[h * head_stride + r * cols + c] (F16 bits)
hipError_t launch_transpose_heads(const uint16_t* src, size_t head_stride, uint16_t* dst, int heads, int rows,
                                  int cols, hipStream_t s);

// attn_kernels.hip: MLA attention of one decode token
constexpr int kMlaChunkPos = 64;  // cache positions per attention chunk (16 or 32 or 64)
struct MlaArgs {
  float* q;              // [128][192] (q_b output; the rope part rotated in place)
  const float* kv_a;     // [576]: latent (512) + k_rope (64), before RoPE, times *kv_scale
  const float* kv_scale;  // the attention norm's 1 / rms that kv_a still owes
  const float* kv_a_norm;  // [512]: the latent's norm weights
  const float* freq;     // [32]: yarn_freq(i)
  int pos, len;          // RoPE position; cache rows before this token
  float *cache_c, *cache_k;  // [max_seq][512], [max_seq][64]
  const uint16_t *k_b, *v_b;  // F16 [128][512][128], [128][128][512]
  float *q_abs, *wc, *attn;  // [128][512], [128][512], [128][128]
  float* part;                        // [ceil(S / kMlaChunkPos)][128][512] partial latent sums
  float* stat;                        // [ceil(S / kMlaChunkPos)][128][2]: each chunk's max score and exp sum
  float scale;
};
// y[r] = (res ? res[r] : 0) + W[r] . x; cols % 512 == 0, cols <= 16384
hipError_t launch_mv_f16(const uint16_t* W, const float* x, const float* res, float* y, int rows, int cols,
                         hipStream_t s);
// y[r] = W[r] . (x * nw) (x of 7168), *inv = the exact 1 / rms of x
hipError_t launch_mv_f16_xw(const uint16_t* W, const float* x, const float* nw, float* y, int rows, float* inv,
                            hipStream_t s);
// y[r] = W[r] . rms_norm(x * (*xmul), nw) (the norm bit-exact); cols 1536
hipError_t launch_mv_f16_rn(const uint16_t* W, const float* x, const float* xmul, const float* nw, float* y, int rows,
                            int cols, hipStream_t s);
// RoPE + cache append, Q_abs, then scores + softmax + weighted latent sum by
// chunks, the chunks merged and v_b
hipError_t launch_mla_attend(const MlaArgs& a, hipStream_t s);

// expert_stream.hip: routed experts read from a packed layer file into an
// LRU cache of expert blobs in HBM (host side).
class ExpertStream {
 public:
  ~ExpertStream();
  // FDM_OK or an FDM_E_* code with *err set
  int open(const char* path, size_t expert_size, int n_experts, int n_cache, int n_threads, int device,
           std::string* err);
  // The cache bookkeeping of one token: slots[k] = the cache slot of
  // ids[k]; miss[k] = its blob is to be read by read().  FDM_OK or
  // FDM_E_INVAL with *err set.
  int plan(const int* ids, int K, int* slots, bool* miss, std::string* err);
  // Reads the planned misses with the pool's threads (4 MB chunks, each
  // copied host-to-device on its thread's stream behind an event) and, on
  // the calling thread, as the last chunk copy of a miss is queued: makes
  // `compute` wait for that miss's copies, then calls ready(k) for each
  // slot k holding it, so its kernels run as soon as it lands while other
  // misses are still read.  Returns once every read and every ready() call
  // is done (the copies may still be in flight).  On a read or copy error
  // the misses not read in full leave the cache, ready() is still called
  // for their slots (so the caller's launches complete its call), and the
  // error is returned.
  int read(hipStream_t compute, const std::function<int(int)>& ready, std::string* err);
  uint8_t* cache() const { return cache_; }
  int n_cache() const { return n_cache_; }
  uint64_t hits() const { return hits_; }
  uint64_t misses() const { return misses_; }
  uint64_t bytes_read() const { return bytes_; }

 private:
  int fd_ = -1;
  size_t es_ = 0;
  int n_experts_ = 0, n_cache_ = 0, n_threads_ = 0;
  uint8_t* cache_ = nullptr;
  std::vector<int> slot_of_, expert_in_;
  std::vector<uint64_t> last_use_;
  uint64_t tick_ = 0, hits_ = 0, misses_ = 0, bytes_ = 0;
  struct Miss {
    int expert, slot;
    std::vector<int> ks;  // the token's slots holding it
  };
  std::vector<Miss> plan_;           // the planned misses of the current token
  std::vector<hipEvent_t> chunk_ev_;  // one per chunk of up to FDM_MAX_K misses
};
// frees the pinned read buffers shared by all streamed layers
void release_stream_pool();

// synth_kernels.hip
hipError_t launch_synth_q4k(uint8_t* dst, size_t n_blocks, uint64_t seed, hipStream_t s);
hipError_t launch_synth_q6k(uint8_t* dst, size_t n_blocks, uint64_t seed, hipStream_t s);
hipError_t launch_synth_normal(float* dst, size_t n, float mean, float std_dev, uint64_t seed,
                               hipStream_t s);

// grid sizing: number of CUs of the current device (set by fdm_init)
extern int g_num_cus;

// capi.hip: the thread's fdm_last_error() text
void set_last_error(const char* msg);

// gguf_host.hip: GGUF shards and the multi-shard manifest (host side)
struct GgufKv {
  std::string key;
  uint32_t type = 0;      // FDM_GGUF_* value type
  uint64_t raw = 0;       // scalar payload, little-endian bits
  std::string str;        // string payload
  uint32_t arr_type = 0;  // array element type
  uint64_t arr_n = 0;     // array length
};
struct GgufTensor {
  std::string name;
  uint32_t n_dims = 0;
  uint64_t dims[4] = {1, 1, 1, 1};
  uint32_t type = 0;      // ggml type id
  uint64_t rel_offset = 0, abs_offset = 0, nbytes = 0;
  int shard = -1;
};
struct GgufShard {
  std::string path;
  int fd = -1;
  uint32_t version = 0;
  uint64_t alignment = 32, data_start = 0, file_size = 0;
  std::vector<GgufKv> kvs;
  std::vector<GgufTensor> tensors;
};
struct GgufManifest {
  std::vector<GgufShard> shards;
  std::unordered_map<std::string, std::pair<int, size_t>> index;  // name -> (shard, tensor)
  std::vector<std::pair<int, size_t>> order;                       // shard order, file order
  ~GgufManifest();
  const GgufTensor* find(const char* name) const;
  const GgufKv* find_kv(int shard, const char* key) const;
  // n bytes of t starting `rel` bytes in, into host memory
  int read(const GgufTensor& t, void* dst, uint64_t n, uint64_t rel) const;
};
uint64_t ggml_nbytes(uint32_t type, const uint64_t* dims, uint32_t n_dims);
const GgufManifest* gguf_manifest(const fdm_gguf* g);

}  // namespace fdm
