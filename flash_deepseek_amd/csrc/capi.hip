// capi.hip -- the C ABI declared in include/fdm.h: argument checks, the
// per-device workspace, the resident-layer table and the kernel sequences.
// The kernels themselves live in *_kernels.hip.
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <atomic>
#include <initializer_list>
#include <math.h>
#include <memory>
#include <mutex>
#include <utility>
#include <vector>

#include "../../include/fdm.h"
#include "epoch_book.h"
#include "fdm_internal.h"

namespace fdm {
// ---- the scratch of fdm_moe_forward_batched_noalloc ------------------------------------
// A file-scope device array holding every BatchScratch buffer of a step of
// up to FDM_NOALLOC_MAX_T tokens and FDM_NOALLOC_MAX_PAIRS (token, expert)
// pairs, each at a 256-byte boundary.  Each device holds its own copy until
// the process ends.  In host code `scratch` is only a stand-in for the
// symbol: its device address comes from hipGetSymbolAddress at fdm_init
// (g_scratch_ptr), and only that address is handed to kernels.
constexpr size_t kNaRows = (size_t)FDM_NOALLOC_MAX_PAIRS + FDM_NOALLOC_MAX_T;
constexpr size_t kNaElems = (size_t)FDM_NOALLOC_MAX_T * FDM_HIDDEN > kNaRows * FDM_MOE_FFN
                                ? (size_t)FDM_NOALLOC_MAX_T * FDM_HIDDEN
                                : kNaRows * FDM_MOE_FFN;
enum NaPart { kNaXd, kNaLogits, kNaIdx, kNaW, kNaSeg, kNaPairTok, kNaPairOf, kNaDistinct, kNaNDistinct,
              kNaAct, kNaActXd, kNaEo, kNaPlanes, kNaXs, kNaXe, kNaChunks, kNaNChunks, kNaParts };
constexpr size_t kNaBytes[kNaParts] = {
    (size_t)FDM_NOALLOC_MAX_T * (FDM_HIDDEN / 64) * sizeof(XGroup),  // xd
    (size_t)FDM_NOALLOC_MAX_T * FDM_N_EXPERTS * sizeof(float),      // logits
    (size_t)FDM_NOALLOC_MAX_PAIRS * sizeof(int),                    // idx
    (size_t)FDM_NOALLOC_MAX_PAIRS * sizeof(float),                  // w
    (FDM_N_EXPERTS + 1) * sizeof(int),                              // seg
    (size_t)FDM_NOALLOC_MAX_PAIRS * sizeof(int),                    // pair_tok
    (size_t)FDM_NOALLOC_MAX_PAIRS * sizeof(int),                    // pair_of
    FDM_N_EXPERTS * sizeof(int),                                    // distinct
    sizeof(int),                                                    // n_distinct
    kNaRows * FDM_MOE_FFN * sizeof(float),                          // act
    kNaRows * (FDM_MOE_FFN / 64) * sizeof(XGroup),                  // act_xd
    kNaRows * FDM_HIDDEN * sizeof(float),                           // eo
    3 * kNaElems * sizeof(_Float16),                                // planes
    kNaElems / 32 * sizeof(float),                                  // xs
    kNaRows * sizeof(float),                                        // xe
    kQMaxChunks * sizeof(int4),                                     // chunks
    sizeof(int),                                                    // n_chunks
};
constexpr size_t na_offset(int part) {
  size_t o = 0;
  for (int i = 0; i < part; ++i) o += (kNaBytes[i] + 255) / 256 * 256;
  return o;
}
constexpr size_t kNaTotal = na_offset(kNaParts);
static_assert(kNaTotal == FDM_NOALLOC_SCRATCH_BYTES, "FDM_NOALLOC_SCRATCH_BYTES is out of date");
}  // namespace fdm

static __device__ __align__(256) unsigned char scratch[fdm::kNaTotal];

namespace fdm {

int g_num_cus = 0;
int g_batch_mode = FDM_BATCH_AUTO;
unsigned g_layer_spin_limit = kLayerSpinLimit;

namespace {

thread_local char t_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(t_err, sizeof t_err, fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(FDM_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define FDM_HIP(call)                                   \
  do {                                                  \
    hipError_t e_ = (call);                             \
    if (e_ != hipSuccess) return hip_fail(e_, #call);   \
  } while (0)

constexpr int kMaxDevices = 64;
unsigned char* g_scratch_ptr[kMaxDevices] = {};  // device address of `scratch`, per device

// Records the device address of `scratch` on the current device (once).
int bind_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return fail(FDM_E_INVAL, "device %d >= %d", device, kMaxDevices);
  if (g_scratch_ptr[device]) return FDM_OK;
  void* ptr = nullptr;
  FDM_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
  g_scratch_ptr[device] = static_cast<unsigned char*>(ptr);
  return FDM_OK;
}

// Per-token scratch of the attention (grown to the largest max_seq).
struct AttnScratch {
  float *normed = nullptr, *q_a = nullptr, *q = nullptr, *kv_a = nullptr;
  float *q_abs = nullptr, *wc = nullptr, *attn = nullptr, *part = nullptr, *stat = nullptr;
  int seq = 0;
  void release() {
    // kv_a lives in q_a's allocation (the two projections run as one matvec)
    for (float* p : {normed, q_a, q, q_abs, wc, attn, part, stat})
      if (p) (void)hipFree(p);
    *this = AttnScratch();
  }
};

struct Workspace {
  XGroup* xd = nullptr;       // digits of activations (up to FDM_MAX_TOKENS x 112)
  float* logits = nullptr;    // FDM_MAX_TOKENS x 256 (the layer path: sigmoid scores)
  int* idx = nullptr;         // FDM_MAX_TOKENS x 16
  int* layer_cnt = nullptr;   // layer kernel arrival counters (kLayerCounters x stride)
  uint64_t* layer_tagged = nullptr;  // layer kernel tagged words (kLayerTagged)
  unsigned* layer_flags = nullptr;  // layer kernel epoch flags (kLayerFlags x stride)
  EpochBook epochs;           // layer kernel call epochs and reported timeouts
  // batched decode (fdm_moe_forward_batched); per-row buffers grow on demand
  int* b_seg = nullptr;       // [257]
  int* b_pair_tok = nullptr;  // [FDM_MAX_TOKENS * FDM_MAX_K]
  int* b_pair_of = nullptr;   // [FDM_MAX_TOKENS * FDM_MAX_K]
  int* b_distinct = nullptr;  // [256]
  int* b_ndistinct = nullptr; // [1]
  size_t b_rows = 0;          // rows the three buffers below hold
  float* b_act = nullptr;     // [b_rows][2048]
  XGroup* b_act_xd = nullptr; // [b_rows][32]
  float* b_eo = nullptr;      // [b_rows][7168]
  // grouped GEMMs (batched decode, prefill): activation planes of the GEMM
  // inputs, grown on demand
  size_t q_elems = 0;         // elements per plane the buffers below hold (x 3 planes)
  _Float16* q_planes = nullptr;  // [3][q_elems]
  float* q_xs = nullptr;      // [q_elems / 32] sub-block sums
  float* q_xe = nullptr;      // [q_rows] row scales
  size_t q_rows = 0;
  int4* q_chunks = nullptr;   // chunk list (kQMaxChunks)
  int* q_nchunks = nullptr;   // [1]
  // prefill (fdm_moe_prefill)
  int p_tokens = 0;           // tokens the buffer below holds
  float* p_hpost = nullptr;   // [p_tokens][7168] rms_norm output
  float* w = nullptr;         // FDM_MAX_TOKENS x 16
  float* act = nullptr;       // (FDM_MAX_K + 1) x 2048
  XGroup* act_xd = nullptr;   // (FDM_MAX_K + 1) x 32
  int* gu_count = nullptr;    // arrival counters: (FDM_MAX_K + 1) x 64 act sub-blocks
  int* dn_count = nullptr;    // arrival counters: 448 down row tiles
  float* eo = nullptr;        // per-slot expert outputs (FDM_MAX_K + 1) x 7168
  float* stage_x = nullptr;   // host-API staging: h_post
  float* stage_y = nullptr;   //                   moe_out
  int* stage_idx = nullptr;   //                   exp_idx
  float* stage_w = nullptr;   //                   exp_w
  float* dense_act = nullptr; // dense FFN activations [kDenseMaxFfn]
  AttnScratch attn;           // MLA attention, grown to the largest max_seq used
  int* ids_h = nullptr;       // pinned host: the routed ids of a streamed call
  int* slots_h = nullptr;     //              their cache slots
};

struct Layer {
  bool resident = false;
  bool owned = false;  // router weights and bias allocated by the library (upload / load)
  // experts and shared expert: library-owned, in the resident expert layout
  const uint8_t* experts = nullptr;
  size_t expert_size = 0;
  int n_experts = 0;
  bool down_q6 = false;
  const float* Wg = nullptr;
  const float* bias = nullptr;
  const uint8_t* shared = nullptr;
};

// A dense FFN layer: library-owned F16 weights (gate, up [inter][7168],
// down [7168][inter]), as dequant_tensor_f16 leaves them.
struct DenseLayer {
  uint16_t *gate = nullptr, *up = nullptr, *down = nullptr;
  int inter = 0;  // 0: not resident
};

// A streamed layer: router, bias (caller-owned) and shared expert (packed,
// library-owned) resident; the routed experts read from the layer file into
// an HBM cache on demand.
struct StreamedLayer {
  ExpertStream es;
  const float* Wg = nullptr;
  const float* bias = nullptr;
  uint8_t* shared = nullptr;
  size_t expert_size = 0;
  bool q6 = false;
  // Calls on several streams take turns: one call at a time fills the cache,
  // after the kernels of the previous call (on whichever stream) have read it.
  std::mutex mu;
  hipEvent_t done = nullptr;  // recorded after each call's kernels
  ~StreamedLayer() {
    if (done) (void)hipEventDestroy(done);
    if (shared) (void)hipFree(shared);
  }
};

// An MLA attention layer: library-owned weights (F16 matrices, fp32 norm
// vectors) in the reference's in-memory layout, its latent KV cache and the
// YaRN frequency table.
struct AttnLayer {
  float *attn_norm = nullptr, *q_a_norm = nullptr, *kv_a_norm = nullptr, *freq = nullptr;
  uint16_t *q_a = nullptr, *q_b = nullptr, *kv_a = nullptr, *k_b = nullptr, *v_b = nullptr, *o_proj = nullptr;
  float *cache_c = nullptr, *cache_k = nullptr;
  int max_seq = 0, len = 0;
  ~AttnLayer() {
    // kv_a lives in q_a's allocation: rows 1536 .. 2111 of one stacked matrix
    for (void* p : {(void*)attn_norm, (void*)q_a_norm, (void*)kv_a_norm, (void*)freq, (void*)q_a, (void*)q_b,
                    (void*)k_b, (void*)v_b, (void*)o_proj, (void*)cache_c, (void*)cache_k})
      if (p) (void)hipFree(p);
  }
};

// Event pairs recorded around kernel launches when profiling is on.
struct Prof {
  static constexpr int kPool = 8192;
  std::atomic<bool> on{false};
  std::recursive_mutex mu;  // held by a ProfScope from its start event to its stop event
  hipEvent_t start[kPool], stop[kPool];
  int phase[kPool];
  int created = 0;
  int pending = 0;  // pairs recorded and not yet read
  int count[FDM_PROF_PHASES];
  double total[FDM_PROF_PHASES], mn[FDM_PROF_PHASES], mx[FDM_PROF_PHASES];
};

struct State {
  bool ready = false;
  Prof prof;
  int device = -1;
  Workspace ws;  // the null stream's
  std::mutex ws_mu;  // guards stream_ws
  std::vector<std::pair<hipStream_t, std::unique_ptr<Workspace>>> stream_ws;  // any other stream's
  Layer layers[FDM_MAX_LAYERS];
  DenseLayer dense[FDM_MAX_LAYERS];
  std::unique_ptr<StreamedLayer> streamed[FDM_MAX_LAYERS];
  std::unique_ptr<AttnLayer> attn[FDM_MAX_LAYERS];
};

State g;

constexpr size_t kXdGroups = (size_t)FDM_MAX_TOKENS * (FDM_HIDDEN / 64);

int check_ready() {
  if (!g.ready) return fail(FDM_E_STATE, "fdm_init has not been called");
  return FDM_OK;
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Down type from the packed expert size, as infer.m:1810-1821.
int down_type(size_t expert_size, bool* q6) {
  if (expert_size == FDM_EXPERT_Q4K_BYTES) {
    *q6 = false;
    return FDM_OK;
  }
  if (expert_size == FDM_EXPERT_Q6K_BYTES) {
    *q6 = true;
    return FDM_OK;
  }
  return fail(FDM_E_SIZE, "expert size %zu is neither %llu (Q4_K down) nor %llu (Q6_K down)",
              expert_size, FDM_EXPERT_Q4K_BYTES, FDM_EXPERT_Q6K_BYTES);
}

void free_workspace(Workspace& w) {
  void* ptrs[] = {w.xd,       w.logits,   w.idx,     w.w,       w.act,
                  w.act_xd,   w.gu_count, w.dn_count, w.eo,
                  w.stage_x,  w.stage_y,  w.stage_idx, w.stage_w,
                  w.layer_cnt, w.layer_flags, w.layer_tagged, w.b_seg, w.b_pair_tok,
                  w.b_pair_of, w.b_distinct, w.b_ndistinct, w.b_act, w.b_act_xd, w.b_eo,
                  w.p_hpost, w.q_planes, w.q_xs, w.q_xe, w.q_chunks, w.q_nchunks, w.dense_act};
  for (void* p : ptrs)
    if (p) (void)hipFree(p);
  w.attn.release();
  for (int* p : {w.ids_h, w.slots_h})
    if (p) (void)hipHostFree(p);
  w = Workspace();
}

int alloc_workspace(Workspace& w) {
  FDM_HIP(hipMalloc(&w.xd, kXdGroups * sizeof(XGroup)));
  FDM_HIP(hipMalloc(&w.logits, (size_t)FDM_MAX_TOKENS * FDM_N_EXPERTS * sizeof(float)));
  FDM_HIP(hipMalloc(&w.idx, (size_t)FDM_MAX_TOKENS * FDM_MAX_K * sizeof(int)));
  FDM_HIP(hipMalloc(&w.w, (size_t)FDM_MAX_TOKENS * FDM_MAX_K * sizeof(float)));
  FDM_HIP(hipMalloc(&w.act, (size_t)(FDM_MAX_K + 1) * FDM_MOE_FFN * sizeof(float)));
  FDM_HIP(hipMalloc(&w.act_xd, (size_t)(FDM_MAX_K + 1) * (FDM_MOE_FFN / 64) * sizeof(XGroup)));
  FDM_HIP(hipMalloc(&w.gu_count, (FDM_MAX_K + 1) * 64 * sizeof(int)));
  FDM_HIP(hipMemset(w.gu_count, 0, (FDM_MAX_K + 1) * 64 * sizeof(int)));
  FDM_HIP(hipMalloc(&w.dn_count, 448 * sizeof(int)));
  FDM_HIP(hipMemset(w.dn_count, 0, 448 * sizeof(int)));
  FDM_HIP(hipMalloc(&w.eo, (size_t)(FDM_MAX_K + 1) * FDM_HIDDEN * sizeof(float)));
  FDM_HIP(hipMalloc(&w.layer_cnt, (size_t)kLayerCounters * kLayerStride * sizeof(int)));
  FDM_HIP(hipMemset(w.layer_cnt, 0, (size_t)kLayerCounters * kLayerStride * sizeof(int)));
  FDM_HIP(hipMalloc(&w.layer_flags, (size_t)kLayerFlags * kLayerStride * sizeof(unsigned)));
  FDM_HIP(hipMemset(w.layer_flags, 0, (size_t)kLayerFlags * kLayerStride * sizeof(unsigned)));
  FDM_HIP(hipMalloc(&w.b_seg, (FDM_N_EXPERTS + 1) * sizeof(int)));
  FDM_HIP(hipMalloc(&w.b_pair_tok, (size_t)FDM_MAX_TOKENS * FDM_MAX_K * sizeof(int)));
  FDM_HIP(hipMalloc(&w.b_pair_of, (size_t)FDM_MAX_TOKENS * FDM_MAX_K * sizeof(int)));
  FDM_HIP(hipMalloc(&w.b_distinct, FDM_N_EXPERTS * sizeof(int)));
  FDM_HIP(hipMalloc(&w.b_ndistinct, sizeof(int)));
  FDM_HIP(hipMalloc(&w.layer_tagged, kLayerTagged * sizeof(uint64_t)));
  FDM_HIP(hipMemset(w.layer_tagged, 0, kLayerTagged * sizeof(uint64_t)));
  FDM_HIP(hipMalloc(&w.stage_x, FDM_HIDDEN * sizeof(float)));
  FDM_HIP(hipMalloc(&w.stage_y, FDM_HIDDEN * sizeof(float)));
  FDM_HIP(hipMalloc(&w.stage_idx, FDM_MAX_K * sizeof(int)));
  FDM_HIP(hipMalloc(&w.stage_w, FDM_MAX_K * sizeof(float)));
  FDM_HIP(hipMalloc(&w.dense_act, kDenseMaxFfn * sizeof(float)));
  FDM_HIP(hipMalloc(&w.q_chunks, kQMaxChunks * sizeof(int4)));
  FDM_HIP(hipMalloc(&w.q_nchunks, sizeof(int)));
  return FDM_OK;
}

// The workspace of the calls on stream s.  Calls on one stream run in stream
// order and share its workspace; calls on different streams use different
// workspaces and may overlap.  The null stream's workspace is made by
// fdm_init, any other stream's at its first call (kept until
// fdm_stream_release or fdm_shutdown).
constexpr size_t kMaxStreamWorkspaces = 64;

int stream_workspace(hipStream_t s, Workspace** out) {
  if (!s) {
    *out = &g.ws;
    return FDM_OK;
  }
  std::lock_guard<std::mutex> lock(g.ws_mu);
  for (auto& e : g.stream_ws)
    if (e.first == s) {
      *out = e.second.get();
      return FDM_OK;
    }
  if (g.stream_ws.size() >= kMaxStreamWorkspaces)
    return fail(FDM_E_STATE, "more than %zu streams hold workspaces; fdm_stream_release the unused ones",
                kMaxStreamWorkspaces);
  auto w = std::make_unique<Workspace>();
  if (int rc = alloc_workspace(*w)) {
    free_workspace(*w);
    return rc;
  }
  *out = w.get();
  g.stream_ws.emplace_back(s, std::move(w));
  return FDM_OK;
}

// The workspace of stream s if it has one.
Workspace* find_workspace(hipStream_t s) {
  if (!s) return &g.ws;
  std::lock_guard<std::mutex> lock(g.ws_mu);
  for (auto& e : g.stream_ws)
    if (e.first == s) return e.second.get();
  return nullptr;
}

void release_dense(DenseLayer& d) {
  for (uint16_t* p : {d.gate, d.up, d.down})
    if (p) (void)hipFree(p);
  d = DenseLayer();
}

// Buffers of a dense layer under construction; freed unless committed.
struct DenseBuffers {
  uint16_t* m[3] = {};  // gate, up, down
  ~DenseBuffers() {
    for (uint16_t* p : m)
      if (p) (void)hipFree(p);
  }
  int alloc(int inter, int L) {
    const size_t n = (size_t)inter * FDM_HIDDEN * sizeof(uint16_t);
    for (uint16_t*& p : m)
      if (hipMalloc(&p, n) != hipSuccess) return fail(FDM_E_NOMEM, "cannot allocate 3 x %zu bytes for dense layer %d", n, L);
    return FDM_OK;
  }
  void commit(int L, int inter) {
    release_dense(g.dense[L]);
    g.dense[L].gate = m[0];
    g.dense[L].up = m[1];
    g.dense[L].down = m[2];
    g.dense[L].inter = inter;
    m[0] = m[1] = m[2] = nullptr;
  }
};

int check_dense(int L, int inter) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS) return fail(FDM_E_INVAL, "layer %d out of range", L);
  if (inter < 512 || inter > kDenseMaxFfn || inter % 512)
    return fail(FDM_E_INVAL, "dense inter dim %d: must be a multiple of 512 in [512, %d]", inter, kDenseMaxFfn);
  return FDM_OK;
}

void release_layer(Layer& L) {
  if (L.resident) {
    (void)hipFree(const_cast<uint8_t*>(L.experts));
    if (L.shared) (void)hipFree(const_cast<uint8_t*>(L.shared));
    if (L.owned) {
      (void)hipFree(const_cast<float*>(L.Wg));
      if (L.bias) (void)hipFree(const_cast<float*>(L.bias));
    }
  }
  L = Layer();
}

// Packed expert blobs (the 256 experts at src + e * src_stride, and the
// shared one) -> freshly allocated buffers in the resident expert layout.
// Synchronous.  On failure nothing stays allocated.
int make_resident_experts(const uint8_t* src, size_t src_stride, const uint8_t* src_shared, size_t es, bool q6,
                          int L, uint8_t** rel, uint8_t** rel_shared) {
  *rel = nullptr;
  *rel_shared = nullptr;
  // the source may still be written by work queued on any stream
  FDM_HIP(hipDeviceSynchronize());
  void *e = nullptr, *sh = nullptr;
  const size_t eb = es * FDM_N_EXPERTS;
  if (hipMalloc(&e, eb) != hipSuccess || (src_shared && hipMalloc(&sh, es) != hipSuccess)) {
    if (e) (void)hipFree(e);
    return fail(FDM_E_NOMEM, "cannot allocate %zu bytes for the experts of layer %d", eb + es, L);
  }
  hipError_t r = launch_rel_pack(src, src_stride, static_cast<uint8_t*>(e), es, FDM_N_EXPERTS, q6, nullptr);
  if (r == hipSuccess && src_shared)
    r = launch_rel_pack(src_shared, es, static_cast<uint8_t*>(sh), es, 1, q6, nullptr);
  if (r == hipSuccess) r = hipStreamSynchronize(nullptr);
  if (r != hipSuccess) {
    (void)hipFree(e);
    if (sh) (void)hipFree(sh);
    return hip_fail(r, "repacking the experts of a layer");
  }
  *rel = static_cast<uint8_t*>(e);
  *rel_shared = static_cast<uint8_t*>(sh);
  return FDM_OK;
}

int get_layer(int L, Layer** out) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS) return fail(FDM_E_INVAL, "layer %d out of range", L);
  if (!g.layers[L].resident) return fail(FDM_E_STATE, "layer %d is not resident", L);
  *out = &g.layers[L];
  return FDM_OK;
}

int check_K(int K) {
  if (K < 1 || K > FDM_MAX_K) return fail(FDM_E_INVAL, "K=%d outside 1..%d", K, FDM_MAX_K);
  return FDM_OK;
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

void prof_clear_stats() {
  Prof& p = g.prof;
  for (int i = 0; i < FDM_PROF_PHASES; ++i) {
    p.count[i] = 0;
    p.total[i] = 0.0;
    p.mn[i] = 1e300;
    p.mx[i] = 0.0;
  }
}

// Fold every recorded pair into the statistics (synchronises on them).
int prof_drain() {
  Prof& p = g.prof;
  for (int i = 0; i < p.pending; ++i) {
    FDM_HIP(hipEventSynchronize(p.stop[i]));
    float ms = 0.0f;
    FDM_HIP(hipEventElapsedTime(&ms, p.start[i], p.stop[i]));
    const int ph = p.phase[i];
    p.count[ph] += 1;
    p.total[ph] += ms;
    if (ms < p.mn[ph]) p.mn[ph] = ms;
    if (ms > p.mx[ph]) p.mx[ph] = ms;
  }
  p.pending = 0;
  return FDM_OK;
}

// Brackets one launch with events when profiling is on.
// Scopes on several host threads take turns (the pool's lock is held from
// the start event to the stop event).
struct ProfScope {
  int slot = -1;
  hipStream_t s;
  std::unique_lock<std::recursive_mutex> lock;
  ProfScope(int phase, hipStream_t st) : s(st) {
    Prof& p = g.prof;
    if (!p.on) return;
    lock = std::unique_lock<std::recursive_mutex>(p.mu);
    if (p.pending == Prof::kPool && prof_drain() != FDM_OK) return;
    slot = p.pending;
    p.phase[slot] = phase;
    if (hipEventRecord(p.start[slot], s) != hipSuccess) slot = -1;
  }
  ~ProfScope() {
    if (slot < 0) return;
    if (hipEventRecord(g.prof.stop[slot], s) == hipSuccess) g.prof.pending = slot + 1;
  }
};

SlotTable slots_for(const Layer& L, const int* idx, const float* w, int K, bool with_shared) {
  SlotTable t;
  t.experts = L.experts;
  t.expert_size = L.expert_size;
  t.n_experts = L.n_experts;
  t.shared = with_shared ? L.shared : nullptr;
  t.idx = idx;
  t.w = w;
  t.K = K;
  t.n_slots = K + ((with_shared && L.shared) ? 1 : 0);
  t.rel = true;
  return t;
}

// ---- ingest helpers -------------------------------------------------------------------

// Host -> device copies through a ring of pinned staging buffers: each
// chunk is read from its file (pread) into the next free buffer and its
// copy queued on a private stream, so the file reads overlap the PCIe
// copies of the chunks before.
class Uploader {
 public:
  static constexpr size_t kChunk = 16u << 20;
  static constexpr int kBufs = 3;
  ~Uploader() {
    if (stream_) (void)hipStreamSynchronize(stream_);
    for (int i = 0; i < kBufs; ++i) {
      if (ev_[i]) (void)hipEventDestroy(ev_[i]);
      if (buf_[i]) (void)hipHostFree(buf_[i]);
    }
    if (stream_) (void)hipStreamDestroy(stream_);
  }
  int init() {
    FDM_HIP(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
    for (int i = 0; i < kBufs; ++i) {
      FDM_HIP(hipHostMalloc(&buf_[i], kChunk, hipHostMallocDefault));
      FDM_HIP(hipEventCreateWithFlags(&ev_[i], hipEventDisableTiming));
    }
    return FDM_OK;
  }
  // n bytes produced by read(host_dst, bytes, offset) -> dev
  template <typename Read>
  int copy(void* dev, uint64_t n, Read&& read) {
    for (uint64_t off = 0; off < n; off += kChunk) {
      const size_t m = (size_t)(n - off < kChunk ? n - off : kChunk);
      const int i = next_++ % kBufs;
      if (used_[i]) FDM_HIP(hipEventSynchronize(ev_[i]));
      if (int rc = read(buf_[i], (uint64_t)m, off)) return rc;
      FDM_HIP(hipMemcpyAsync(static_cast<uint8_t*>(dev) + off, buf_[i], m, hipMemcpyHostToDevice,
                             stream_));
      FDM_HIP(hipEventRecord(ev_[i], stream_));
      used_[i] = true;
      bytes_ += m;
    }
    return FDM_OK;
  }
  int finish() {
    FDM_HIP(hipStreamSynchronize(stream_));
    return FDM_OK;
  }

 private:
  hipStream_t stream_ = nullptr;
  void* buf_[kBufs] = {};
  hipEvent_t ev_[kBufs] = {};
  bool used_[kBufs] = {};
  int next_ = 0;
  uint64_t bytes_ = 0;
};

// IEEE half -> float by integer construction (every finite, infinite and
// NaN pattern; subnormals normalised).
float half_bits_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1Fu, f = h & 0x3FFu;
  uint32_t bits;
  if (e == 0x1Fu) {
    bits = sign | 0x7F800000u | (f << 13);
  } else if (e) {
    bits = sign | ((e + 112u) << 23) | (f << 13);
  } else if (!f) {
    bits = sign;
  } else {
    const uint32_t p = 31u - (uint32_t)__builtin_clz(f), shift = 10u - p;
    bits = sign | ((113u - shift) << 23) | (((f << shift) & 0x3FFu) << 13);
  }
  float v;
  memcpy(&v, &bits, 4);
  return v;
}

// A GGUF tensor with the expected type set and shape.
int expect_tensor(const GgufManifest& m, const char* name, const GgufTensor** out,
                  std::initializer_list<uint32_t> types, std::initializer_list<uint64_t> dims) {
  const GgufTensor* t = m.find(name);
  if (!t) return fail(FDM_E_FORMAT, "tensor %s not in the GGUF", name);
  bool type_ok = false;
  for (uint32_t ty : types) type_ok = type_ok || t->type == ty;
  if (!type_ok) return fail(FDM_E_FORMAT, "tensor %s has ggml type %u", name, t->type);
  if (t->n_dims != dims.size()) return fail(FDM_E_FORMAT, "tensor %s has %u dims", name, t->n_dims);
  int d = 0;
  for (uint64_t want : dims) {
    if (t->dims[d] != want)
      return fail(FDM_E_FORMAT, "tensor %s: ne[%d] = %llu, expected %llu", name, d,
                  (unsigned long long)t->dims[d], (unsigned long long)want);
    ++d;
  }
  *out = t;
  return FDM_OK;
}

// An F32 / F16 / BF16 tensor of n elements, widened to fp32 on the host.
int read_f32(const GgufManifest& m, const GgufTensor& t, std::vector<float>& out) {
  const uint64_t n = t.nbytes / (t.type == FDM_GGML_F32 ? 4 : 2);
  out.resize(n);
  if (t.type == FDM_GGML_F32) return m.read(t, out.data(), t.nbytes, 0);
  std::vector<uint16_t> raw(n);
  if (int rc = m.read(t, raw.data(), t.nbytes, 0)) return rc;
  for (uint64_t i = 0; i < n; ++i) {
    if (t.type == FDM_GGML_F16) {
      out[i] = half_bits_to_float(raw[i]);
    } else {
      const uint32_t b = (uint32_t)raw[i] << 16;
      memcpy(&out[i], &b, 4);
    }
  }
  return FDM_OK;
}

// Router weights, bias and (optionally) the shared expert's three tensors of
// layer L, checked against the R1 shapes; the shared down type must be q6.
struct LayerTensors {
  const GgufTensor *router = nullptr, *bias = nullptr;
  const GgufTensor *sgate = nullptr, *sup = nullptr, *sdown = nullptr;
};
int find_layer_common(const GgufManifest& m, int L, bool with_shared, bool q6, LayerTensors* lt) {
  char name[128];
  const std::initializer_list<uint32_t> fp = {FDM_GGML_F32, FDM_GGML_F16, FDM_GGML_BF16};
  snprintf(name, sizeof name, "blk.%d.ffn_gate_inp.weight", L);
  if (int rc = expect_tensor(m, name, &lt->router, fp, {FDM_HIDDEN, FDM_N_EXPERTS})) return rc;
  // the correction bias is optional (route() then adds nothing); .bias or .weight
  snprintf(name, sizeof name, "blk.%d.exp_probs_b.bias", L);
  if (!m.find(name)) snprintf(name, sizeof name, "blk.%d.exp_probs_b.weight", L);
  if (m.find(name))
    if (int rc = expect_tensor(m, name, &lt->bias, fp, {FDM_N_EXPERTS})) return rc;
  if (!with_shared) return FDM_OK;
  snprintf(name, sizeof name, "blk.%d.ffn_gate_shexp.weight", L);
  if (int rc = expect_tensor(m, name, &lt->sgate, {FDM_GGML_Q4_K}, {FDM_HIDDEN, FDM_MOE_FFN})) return rc;
  snprintf(name, sizeof name, "blk.%d.ffn_up_shexp.weight", L);
  if (int rc = expect_tensor(m, name, &lt->sup, {FDM_GGML_Q4_K}, {FDM_HIDDEN, FDM_MOE_FFN})) return rc;
  snprintf(name, sizeof name, "blk.%d.ffn_down_shexp.weight", L);
  if (int rc = expect_tensor(m, name, &lt->sdown, {FDM_GGML_Q4_K, FDM_GGML_Q6_K}, {FDM_MOE_FFN, FDM_HIDDEN}))
    return rc;
  if ((lt->sdown->type == FDM_GGML_Q6_K) != q6)
    return fail(FDM_E_FORMAT, "layer %d: the shared expert's down type differs from the routed experts'", L);
  return FDM_OK;
}

// Device buffers of one layer under construction; freed unless committed.
struct LayerBuffers {
  void *experts = nullptr, *Wg = nullptr, *bias = nullptr, *shared = nullptr;
  ~LayerBuffers() {
    for (void* p : {experts, Wg, bias, shared})
      if (p) (void)hipFree(p);
  }
  int alloc(size_t es, bool bias_, bool shared_, int L) {
    const size_t eb = es * FDM_N_EXPERTS, wb = (size_t)FDM_N_EXPERTS * FDM_HIDDEN * sizeof(float);
    if (hipMalloc(&experts, eb) != hipSuccess || hipMalloc(&Wg, wb) != hipSuccess ||
        (bias_ && hipMalloc(&bias, FDM_N_EXPERTS * sizeof(float)) != hipSuccess) ||
        (shared_ && hipMalloc(&shared, es) != hipSuccess))
      return fail(FDM_E_NOMEM, "cannot allocate %zu bytes for layer %d", eb + wb + es, L);
    return FDM_OK;
  }
};

// Router, bias and shared expert of a layer under construction.
int upload_layer_common(const GgufManifest& m, const LayerTensors& lt, LayerBuffers& b, Uploader& up,
                        size_t down_bytes) {
  std::vector<float> v;
  if (int rc = read_f32(m, *lt.router, v)) return rc;
  FDM_HIP(hipMemcpy(b.Wg, v.data(), v.size() * sizeof(float), hipMemcpyHostToDevice));
  if (lt.bias) {
    if (int rc = read_f32(m, *lt.bias, v)) return rc;
    FDM_HIP(hipMemcpy(b.bias, v.data(), v.size() * sizeof(float), hipMemcpyHostToDevice));
  }
  if (lt.sgate) {
    const GgufTensor* parts[3] = {lt.sgate, lt.sup, lt.sdown};
    const uint64_t at[3] = {0, (uint64_t)kGateBytes, 2ull * kGateBytes};
    for (int p = 0; p < 3; ++p) {
      const uint64_t n = p < 2 ? (uint64_t)kGateBytes : down_bytes;
      if (int rc = up.copy(static_cast<uint8_t*>(b.shared) + at[p], n,
                           [&](void* dst, uint64_t k, uint64_t off) { return m.read(*parts[p], dst, k, off); }))
        return rc;
    }
  }
  return FDM_OK;
}

int commit_layer(int L, LayerBuffers& b, size_t es, bool q6) {
  uint8_t *rel = nullptr, *rel_shared = nullptr;
  if (int rc = make_resident_experts(static_cast<const uint8_t*>(b.experts), es,
                                     static_cast<const uint8_t*>(b.shared), es, q6, L, &rel, &rel_shared))
    return rc;
  release_layer(g.layers[L]);
  g.streamed[L].reset();
  Layer& y = g.layers[L];
  y.resident = true;
  y.owned = true;
  y.experts = rel;
  y.expert_size = es;
  y.n_experts = FDM_N_EXPERTS;
  y.down_q6 = q6;
  y.Wg = static_cast<const float*>(b.Wg);
  y.bias = static_cast<const float*>(b.bias);
  y.shared = rel_shared;
  b.Wg = nullptr;  // moved to the layer table; the packed staging copies are freed with b
  b.bias = nullptr;
  return FDM_OK;
}

}  // namespace

void set_last_error(const char* msg) {
  snprintf(t_err, sizeof t_err, "%s", msg);
}

}  // namespace fdm

using namespace fdm;

extern "C" {

int fdm_init(int device) {
  if (g.ready) {
    if (device == g.device) return FDM_OK;
    return fail(FDM_E_STATE, "already initialised on device %d", g.device);
  }
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) return fail(FDM_E_NODEV, "no HIP device available");
  if (device < 0 || device >= n) return fail(FDM_E_INVAL, "device %d of %d", device, n);
  FDM_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  FDM_HIP(hipGetDeviceProperties(&prop, device));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(FDM_E_NODEV, "device %d is %s; this build targets gfx950", device,
                prop.gcnArchName);
  g_num_cus = prop.multiProcessorCount;
  if (int rc = bind_scratch(device)) return rc;
  if (int rc = alloc_workspace(g.ws)) {
    free_workspace(g.ws);
    return rc;
  }
  g.device = device;
  g.ready = true;
  return FDM_OK;
}

int fdm_shutdown(void) {
  if (!g.ready) return FDM_OK;
  (void)hipDeviceSynchronize();
  for (auto& L : g.layers) release_layer(L);
  for (auto& d : g.dense) release_dense(d);
  for (auto& st : g.streamed) st.reset();
  for (auto& a : g.attn) a.reset();
  release_stream_pool();
  for (auto& e : g.stream_ws) free_workspace(*e.second);
  g.stream_ws.clear();
  free_workspace(g.ws);
  for (int i = 0; i < g.prof.created; ++i) {
    (void)hipEventDestroy(g.prof.start[i]);
    (void)hipEventDestroy(g.prof.stop[i]);
  }
  g.prof.created = 0;
  g.prof.pending = 0;
  g.prof.on = false;
  g.ready = false;
  g.device = -1;
  return FDM_OK;
}

int fdm_available(void) { return g.ready ? 1 : 0; }

const char* fdm_strerror(int code) {
  switch (code) {
    case FDM_OK: return "ok";
    case FDM_E_INVAL: return "invalid argument";
    case FDM_E_NODEV: return "no usable gfx950 device";
    case FDM_E_HIP: return "HIP runtime error";
    case FDM_E_STATE: return "not initialised or layer not resident";
    case FDM_E_NOMEM: return "device allocation failed";
    case FDM_E_SIZE: return "expert size matches neither R1 layout";
    case FDM_E_IO: return "file error";
    case FDM_E_FORMAT: return "malformed model file";
    default: return "unknown error";
  }
}

const char* fdm_last_error(void) { return t_err; }

int fdm_device_cus(void) { return g.ready ? g_num_cus : 0; }

int fdm_malloc(void** d_ptr, size_t bytes) {
  if (!d_ptr) return fail(FDM_E_INVAL, "null out pointer");
  if (int rc = check_ready()) return rc;
  hipError_t e = hipMalloc(d_ptr, bytes);
  if (e != hipSuccess) return fail(FDM_E_NOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
  return FDM_OK;
}

int fdm_free(void* d_ptr) {
  if (int rc = check_ready()) return rc;
  FDM_HIP(hipFree(d_ptr));
  return FDM_OK;
}

int fdm_memcpy_h2d(void* d_dst, const void* h_src, size_t bytes, void* stream) {
  if (int rc = check_ready()) return rc;
  FDM_HIP(hipMemcpyAsync(d_dst, h_src, bytes, hipMemcpyHostToDevice, as_stream(stream)));
  return FDM_OK;
}

int fdm_memcpy_d2h(void* h_dst, const void* d_src, size_t bytes, void* stream) {
  if (int rc = check_ready()) return rc;
  FDM_HIP(hipMemcpyAsync(h_dst, d_src, bytes, hipMemcpyDeviceToHost, as_stream(stream)));
  return FDM_OK;
}

int fdm_stream_sync(void* stream) {
  if (int rc = check_ready()) return rc;
  hipStream_t s = as_stream(stream);
  FDM_HIP(hipStreamSynchronize(s));
  Workspace* w = find_workspace(s);
  if (w && w->epochs.epoch != 0) {
    // the layer kernel records the epoch of a call whose waits timed out
    unsigned err = 0;
    FDM_HIP(hipMemcpy(&err, w->layer_flags + kLayerFlagErr * kLayerStride, sizeof(err),
                      hipMemcpyDeviceToHost));
    if (w->epochs.new_error(err))
      return fail(FDM_E_STATE,
                  "a bounded wait inside a one-launch kernel (batch-1 layer, expert FFN or matvec) gave up "
                  "in the call of epoch %u on this stream",
                  err);
  }
  return FDM_OK;
}

int fdm_stream_release(void* stream) {
  if (int rc = check_ready()) return rc;
  hipStream_t s = as_stream(stream);
  if (!s) return FDM_OK;  // the null stream keeps its workspace until fdm_shutdown
  std::unique_ptr<Workspace> w;
  {
    std::lock_guard<std::mutex> lock(g.ws_mu);
    for (size_t i = 0; i < g.stream_ws.size(); ++i)
      if (g.stream_ws[i].first == s) {
        w = std::move(g.stream_ws[i].second);
        g.stream_ws.erase(g.stream_ws.begin() + i);
        break;
      }
  }
  if (!w) return FDM_OK;
  FDM_HIP(hipDeviceSynchronize());  // the stream itself may already be destroyed
  free_workspace(*w);
  return FDM_OK;
}

// ---- quant.h twins --------------------------------------------------------
int fdm_fp16_to_fp32(const uint16_t* d_src, float* d_dst, size_t n, void* stream) {
  if (int rc = check_ready()) return rc;
  if (!d_src || !d_dst) return fail(FDM_E_INVAL, "null pointer");
  if (n == 0) return FDM_OK;
  FDM_HIP(launch_fp16_to_fp32(d_src, d_dst, n, as_stream(stream)));
  return FDM_OK;
}

int fdm_dequant_q4k(const void* d_src, float* d_dst, size_t n, void* stream) {
  if (int rc = check_ready()) return rc;
  if (!d_src || !d_dst) return fail(FDM_E_INVAL, "null pointer");
  if (n % FDM_QK_K) return fail(FDM_E_INVAL, "n=%zu is not a multiple of 256", n);
  if (!aligned(d_src, 4) || !aligned(d_dst, 8))
    return fail(FDM_E_INVAL, "Q4_K source must be 4-byte and output 8-byte aligned");
  if (n == 0) return FDM_OK;
  FDM_HIP(launch_dequant_q4k(static_cast<const uint8_t*>(d_src), d_dst, n / FDM_QK_K,
                             as_stream(stream)));
  return FDM_OK;
}

int fdm_dequant_q6k(const void* d_src, float* d_dst, size_t n, void* stream) {
  if (int rc = check_ready()) return rc;
  if (!d_src || !d_dst) return fail(FDM_E_INVAL, "null pointer");
  if (n % FDM_QK_K) return fail(FDM_E_INVAL, "n=%zu is not a multiple of 256", n);
  if (!aligned(d_dst, 4)) return fail(FDM_E_INVAL, "output must be 4-byte aligned");
  if (n == 0) return FDM_OK;
  FDM_HIP(launch_dequant_q6k(static_cast<const uint8_t*>(d_src), d_dst, n / FDM_QK_K,
                             as_stream(stream)));
  return FDM_OK;
}

// ---- matvec -----------------------------------------------------------------
static int matvec_common(const void* d_W, const float* d_x, float* d_y, uint32_t out_dim,
                         uint32_t in_dim, size_t w_align) {
  if (int rc = check_ready()) return rc;
  if (!d_W || !d_x || !d_y) return fail(FDM_E_INVAL, "null pointer");
  if (in_dim == 0 || in_dim % FDM_QK_K || in_dim > 4u * FDM_HIDDEN)
    return fail(FDM_E_INVAL, "in_dim=%u must be a positive multiple of 256 <= %d", in_dim,
                4 * FDM_HIDDEN);
  if (out_dim == 0 || out_dim > (1u << 24)) return fail(FDM_E_INVAL, "out_dim=%u", out_dim);
  if (!aligned(d_W, w_align) || !aligned(d_x, 4) || !aligned(d_y, 4))
    return fail(FDM_E_INVAL, "misaligned pointer (W needs %zu bytes)", w_align);
  return FDM_OK;
}

}  // extern "C"

namespace fdm {
namespace {
// The layer kernel's share of a stream workspace: the digit records, the
// tagged hand-off words, counters, flags and a fresh epoch.
void layer_workspace_args(LayerArgs& a, Workspace* ws) {
  a.xd = ws->xd;
  uint64_t* tg = ws->layer_tagged;
  a.scores = tg;
  a.prov = tg + 256;
  a.route_w = tg + 256 + 16;
  a.route_perm = tg + 256 + 32;
  a.act = tg + 256 + 48;
  a.eo = a.act + (size_t)kLayerMaxSlots * FDM_MOE_FFN;
  a.act_xd = a.eo + (size_t)kLayerMaxSlots * kLayerMaxParts * FDM_HIDDEN;
  a.norm_inv = tg + kLayerTagged - 16;  // its own 128-byte line
  a.counters = ws->layer_cnt;
  a.flags = ws->layer_flags;
  a.epoch = ws->epochs.next();
  a.spin_limit = g_layer_spin_limit;
}

// One launch (digit items, then row items) where the kernel supports in_dim;
// otherwise the digits and the matvec as two launches.
int run_matvec(bool q6, const void* d_W, const float* d_x, float* d_y, uint32_t out_dim, uint32_t in_dim,
               void* stream) {
  hipStream_t s = as_stream(stream);
  Workspace* w = nullptr;
  if (int rc = stream_workspace(s, &w)) return rc;
  const uint8_t* W = static_cast<const uint8_t*>(d_W);
  // the layer kernel's tagged expert-output words hold the partial sums
  const size_t part_words = (size_t)kLayerMaxSlots * kLayerMaxParts * FDM_HIDDEN;
  if (!q6 && matvec3_supported((int)in_dim)) {
    ProfScope p(FDM_PROF_MATVEC, s);
    FDM_HIP(launch_matvec3_q4k(W, d_x, d_y, (int)out_dim, (int)in_dim, s));
    return FDM_OK;
  }
  if (!q6 && matvec2_supported((int)in_dim, (int)out_dim, part_words)) {
    Matvec2Args a;
    a.W = W;
    a.x = d_x;
    a.y = d_y;
    a.rows = (int)out_dim;
    a.part = w->layer_tagged + 256 + 48 + (size_t)kLayerMaxSlots * FDM_MOE_FFN;
    a.err = w->layer_flags + kLayerFlagErr * kLayerStride;
    a.epoch = w->epochs.next();
    a.spin_limit = g_layer_spin_limit;
    ProfScope p(FDM_PROF_MATVEC, s);
    FDM_HIP(launch_matvec2_q4k(a, (int)in_dim, s));
    return FDM_OK;
  }
  if (matvec1_supported(q6, (int)in_dim)) {
    MatvecArgs a;
    a.W = W;
    a.x = d_x;
    a.y = d_y;
    a.rows = (int)out_dim;
    a.gr = (int)in_dim / 64;
    a.xd = w->xd;
    a.counter = w->layer_cnt;  // the layer kernel's digit counter and flag: calls on a stream never overlap
    a.flag = w->layer_flags;
    a.err = w->layer_flags + kLayerFlagErr * kLayerStride;
    a.epoch = w->epochs.next();
    a.spin_limit = g_layer_spin_limit;
    ProfScope p(FDM_PROF_MATVEC, s);
    FDM_HIP(launch_matvec1(a, q6, s));
    return FDM_OK;
  }
  {
    ProfScope p(FDM_PROF_XDIGITS, s);
    FDM_HIP(launch_xdigits(d_x, in_dim / 64, w->xd, s));
  }
  {
    ProfScope p(FDM_PROF_MATVEC, s);
    if (q6)
      FDM_HIP(launch_matvec_q6k(W, w->xd, d_y, (int)out_dim, (int)in_dim, s));
    else
      FDM_HIP(launch_matvec_q4k(W, w->xd, d_y, (int)out_dim, (int)in_dim, s));
  }
  return FDM_OK;
}
}  // namespace
}  // namespace fdm

extern "C" {

int fdm_matvec_q4k(const void* d_W, const float* d_x, float* d_y, uint32_t out_dim,
                   uint32_t in_dim, void* stream) {
  if (int rc = matvec_common(d_W, d_x, d_y, out_dim, in_dim, 4)) return rc;
  return run_matvec(false, d_W, d_x, d_y, out_dim, in_dim, stream);
}

int fdm_matvec_q6k(const void* d_W, const float* d_x, float* d_y, uint32_t out_dim,
                   uint32_t in_dim, void* stream) {
  if (int rc = matvec_common(d_W, d_x, d_y, out_dim, in_dim, 2)) return rc;
  return run_matvec(true, d_W, d_x, d_y, out_dim, in_dim, stream);
}

// ---- one expert -----------------------------------------------------------
int fdm_expert_ffn(const void* d_blob, size_t expert_size, const float* d_x, float* d_out,
                   float* d_act, void* stream) {
  if (int rc = check_ready()) return rc;
  if (!d_blob || !d_x || !d_out) return fail(FDM_E_INVAL, "null pointer");
  bool q6 = false;
  if (int rc = down_type(expert_size, &q6)) return rc;
  if (!aligned(d_blob, 4) || !aligned(d_x, 16))
    return fail(FDM_E_INVAL, "blob must be 4-byte and x 16-byte aligned");
  if (d_act && !aligned(d_act, 4)) return fail(FDM_E_INVAL, "act must be 4-byte aligned");
  hipStream_t s = as_stream(stream);
  // one launch of the fp32 expert kernel (expert_kernels.hip) on the
  // caller's packed blob, Q4_K or Q6_K down
  Workspace* ws = nullptr;
  if (int rc = stream_workspace(s, &ws)) return rc;
  LayerArgs a;
  a.Wg = nullptr;
  a.bias = nullptr;
  a.h = d_x;
  a.h_in = nullptr;
  a.out = d_out;
  a.moe_out = nullptr;
  a.experts = nullptr;
  a.expert_size = expert_size;
  a.n_experts = 0;
  a.shared = static_cast<const uint8_t*>(d_blob);
  a.down_q6 = q6 ? 1 : 0;
  a.K = 0;
  a.n_slots = 1;
  a.idx = ws->idx;
  a.w = ws->w;
  layer_workspace_args(a, ws);
  a.act_out = d_act;
  {
    ProfScope p(FDM_PROF_GATEUP, s);
    // the fp32 expert kernel (gate/up items, one activation hand-off, down items)
    FDM_HIP(launch_expert_f32(a, s));
  }
  return FDM_OK;
}

// ---- router -----------------------------------------------------------------
int fdm_router_logits(const float* d_Wg, const float* d_x, int n_exp, int dim, int T,
                      float* d_logits, void* stream) {
  if (int rc = check_ready()) return rc;
  if (!d_Wg || !d_x || !d_logits) return fail(FDM_E_INVAL, "null pointer");
  if (n_exp <= 0 || n_exp > 65535 || dim <= 0 || dim % 4 || T <= 0 || T > 65535 * 8)
    return fail(FDM_E_INVAL, "n_exp=%d dim=%d T=%d", n_exp, dim, T);
  if (!aligned(d_Wg, 16) || !aligned(d_x, 16))
    return fail(FDM_E_INVAL, "Wg and x must be 16-byte aligned");
  FDM_HIP(launch_router_logits(d_Wg, d_x, n_exp, dim, T, d_logits, as_stream(stream)));
  return FDM_OK;
}

int fdm_route(const float* d_logits, const float* d_bias, int T, int K, int* d_idx, float* d_w,
              void* stream) {
  if (int rc = check_ready()) return rc;
  if (!d_logits || !d_idx || !d_w) return fail(FDM_E_INVAL, "null pointer");
  if (int rc = check_K(K)) return rc;
  if (T <= 0 || T > (1 << 24)) return fail(FDM_E_INVAL, "T=%d", T);
  FDM_HIP(launch_route(d_logits, d_bias, T, K, d_idx, d_w, as_stream(stream)));
  return FDM_OK;
}

// ---- resident layers ------------------------------------------------------------
int fdm_layer_attach(int L, const void* d_experts, size_t expert_size, int n_experts,
                     const float* d_Wg, const float* d_bias, const void* d_shared) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS) return fail(FDM_E_INVAL, "layer %d out of range", L);
  if (!d_experts || !d_Wg) return fail(FDM_E_INVAL, "null experts or router weights");
  if (n_experts != FDM_N_EXPERTS)
    return fail(FDM_E_INVAL, "n_experts=%d: the router is the R1 256-expert router", n_experts);
  bool q6 = false;
  if (int rc = down_type(expert_size, &q6)) return rc;
  if (!aligned(d_experts, 16) || !aligned(d_Wg, 16) || (d_shared && !aligned(d_shared, 16)))
    return fail(FDM_E_INVAL, "layer buffers must be 16-byte aligned");
  uint8_t *rel = nullptr, *rel_shared = nullptr;
  if (int rc = make_resident_experts(static_cast<const uint8_t*>(d_experts), expert_size,
                                     static_cast<const uint8_t*>(d_shared), expert_size, q6, L, &rel,
                                     &rel_shared))
    return rc;
  release_layer(g.layers[L]);
  g.streamed[L].reset();
  Layer& y = g.layers[L];
  y.resident = true;
  y.owned = false;
  y.experts = rel;
  y.expert_size = expert_size;
  y.n_experts = n_experts;
  y.down_q6 = q6;
  y.Wg = d_Wg;
  y.bias = d_bias;
  y.shared = rel_shared;
  return FDM_OK;
}

int fdm_layer_upload(int L, const void* h_experts, size_t expert_size, int n_experts,
                     const float* h_Wg, const float* h_bias, const void* h_shared) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS) return fail(FDM_E_INVAL, "layer %d out of range", L);
  if (!h_experts || !h_Wg) return fail(FDM_E_INVAL, "null experts or router weights");
  if (n_experts != FDM_N_EXPERTS)
    return fail(FDM_E_INVAL, "n_experts=%d: the router is the R1 256-expert router", n_experts);
  bool q6 = false;
  if (int rc = down_type(expert_size, &q6)) return rc;
  const size_t eb = expert_size * (size_t)n_experts;
  const size_t wb = (size_t)FDM_N_EXPERTS * FDM_HIDDEN * sizeof(float);
  void *de = nullptr, *dw = nullptr, *db = nullptr, *ds = nullptr;
  auto cleanup = [&]() {
    if (de) (void)hipFree(de);
    if (dw) (void)hipFree(dw);
    if (db) (void)hipFree(db);
    if (ds) (void)hipFree(ds);
  };
  if (hipMalloc(&de, eb) != hipSuccess || hipMalloc(&dw, wb) != hipSuccess ||
      (h_bias && hipMalloc(&db, FDM_N_EXPERTS * sizeof(float)) != hipSuccess) ||
      (h_shared && hipMalloc(&ds, expert_size) != hipSuccess)) {
    cleanup();
    return fail(FDM_E_NOMEM, "cannot allocate %zu bytes for layer %d", eb + wb + expert_size, L);
  }
  hipError_t e = hipMemcpy(de, h_experts, eb, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(dw, h_Wg, wb, hipMemcpyHostToDevice);
  if (e == hipSuccess && h_bias)
    e = hipMemcpy(db, h_bias, FDM_N_EXPERTS * sizeof(float), hipMemcpyHostToDevice);
  if (e == hipSuccess && h_shared) e = hipMemcpy(ds, h_shared, expert_size, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    cleanup();
    return hip_fail(e, "layer upload");
  }
  uint8_t *rel = nullptr, *rel_shared = nullptr;
  if (int rc = make_resident_experts(static_cast<const uint8_t*>(de), expert_size,
                                     static_cast<const uint8_t*>(ds), expert_size, q6, L, &rel, &rel_shared)) {
    cleanup();
    return rc;
  }
  (void)hipFree(de);  // the packed staging copies
  if (ds) (void)hipFree(ds);
  release_layer(g.layers[L]);
  g.streamed[L].reset();
  Layer& y = g.layers[L];
  y.resident = true;
  y.owned = true;
  y.experts = rel;
  y.expert_size = expert_size;
  y.n_experts = n_experts;
  y.down_q6 = q6;
  y.Wg = static_cast<const float*>(dw);
  y.bias = static_cast<const float*>(db);
  y.shared = rel_shared;
  return FDM_OK;
}

int fdm_layer_load_gguf(int L, const fdm_gguf* mh, int with_shared, int* down_is_q6) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS) return fail(FDM_E_INVAL, "layer %d out of range", L);
  const GgufManifest* m = gguf_manifest(mh);
  if (!m) return fail(FDM_E_INVAL, "null manifest");
  char name[128];
  const GgufTensor *tg = nullptr, *tu = nullptr, *td = nullptr;
  snprintf(name, sizeof name, "blk.%d.ffn_gate_exps.weight", L);
  if (int rc = expect_tensor(*m, name, &tg, {FDM_GGML_Q4_K}, {FDM_HIDDEN, FDM_MOE_FFN, FDM_N_EXPERTS}))
    return rc;
  snprintf(name, sizeof name, "blk.%d.ffn_up_exps.weight", L);
  if (int rc = expect_tensor(*m, name, &tu, {FDM_GGML_Q4_K}, {FDM_HIDDEN, FDM_MOE_FFN, FDM_N_EXPERTS}))
    return rc;
  snprintf(name, sizeof name, "blk.%d.ffn_down_exps.weight", L);
  if (int rc = expect_tensor(*m, name, &td, {FDM_GGML_Q4_K, FDM_GGML_Q6_K},
                             {FDM_MOE_FFN, FDM_HIDDEN, FDM_N_EXPERTS}))
    return rc;
  const bool q6 = td->type == FDM_GGML_Q6_K;
  const size_t down_bytes = td->nbytes / FDM_N_EXPERTS;
  const size_t es = 2 * (size_t)kGateBytes + down_bytes;
  LayerTensors lt;
  if (int rc = find_layer_common(*m, L, with_shared != 0, q6, &lt)) return rc;
  LayerBuffers b;
  if (int rc = b.alloc(es, lt.bias != nullptr, with_shared != 0, L)) return rc;
  Uploader up;
  if (int rc = up.init()) return rc;
  // expert e of each stacked tensor is one contiguous slice: scatter them
  // into the packed blobs [gate | up | down] at e * expert_size
  const GgufTensor* parts[3] = {tg, tu, td};
  const uint64_t sz[3] = {(uint64_t)kGateBytes, (uint64_t)kGateBytes, down_bytes};
  const uint64_t at[3] = {0, (uint64_t)kGateBytes, 2ull * kGateBytes};
  for (int e = 0; e < FDM_N_EXPERTS; ++e)
    for (int p = 0; p < 3; ++p) {
      const uint64_t src = (uint64_t)e * sz[p];
      if (int rc = up.copy(static_cast<uint8_t*>(b.experts) + (size_t)e * es + at[p], sz[p],
                           [&](void* dst, uint64_t k, uint64_t off) { return m->read(*parts[p], dst, k, src + off); }))
        return rc;
    }
  if (int rc = upload_layer_common(*m, lt, b, up, down_bytes)) return rc;
  if (int rc = up.finish()) return rc;
  if (down_is_q6) *down_is_q6 = q6 ? 1 : 0;
  return commit_layer(L, b, es, q6);
}

int fdm_layer_load_packed(int L, const char* layer_file, const fdm_gguf* mh, int with_shared,
                          int* down_is_q6) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS) return fail(FDM_E_INVAL, "layer %d out of range", L);
  const GgufManifest* m = gguf_manifest(mh);
  if (!m || !layer_file) return fail(FDM_E_INVAL, "null manifest or layer file");
  const int fd = open(layer_file, O_RDONLY);
  if (fd < 0) return fail(FDM_E_IO, "open %s: %s", layer_file, strerror(errno));
  struct FdCloser {
    int fd;
    ~FdCloser() { close(fd); }
  } closer{fd};
  struct stat st;
  if (fstat(fd, &st) != 0) return fail(FDM_E_IO, "fstat %s: %s", layer_file, strerror(errno));
  // 256 blobs; the expert size, hence the down type, from the file size
  if (st.st_size <= 0 || st.st_size % FDM_N_EXPERTS)
    return fail(FDM_E_SIZE, "%s: %lld bytes is not 256 expert blobs", layer_file, (long long)st.st_size);
  const size_t es = (size_t)st.st_size / FDM_N_EXPERTS;
  bool q6 = false;
  if (int rc = down_type(es, &q6)) return rc;
  LayerTensors lt;
  if (int rc = find_layer_common(*m, L, with_shared != 0, q6, &lt)) return rc;
  LayerBuffers b;
  if (int rc = b.alloc(es, lt.bias != nullptr, with_shared != 0, L)) return rc;
  Uploader up;
  if (int rc = up.init()) return rc;
  // the packed layout is the library's: one contiguous copy
  if (int rc = up.copy(b.experts, (uint64_t)st.st_size, [&](void* dst, uint64_t k, uint64_t off) {
        uint64_t got = 0;
        while (got < k) {
          const ssize_t r = pread(fd, static_cast<uint8_t*>(dst) + got, k - got, (off_t)(off + got));
          if (r < 0 && errno == EINTR) continue;
          if (r <= 0) return fail(FDM_E_IO, "read of %s: %s", layer_file, r < 0 ? strerror(errno) : "end of file");
          got += (uint64_t)r;
        }
        return (int)FDM_OK;
      }))
    return rc;
  if (int rc = upload_layer_common(*m, lt, b, up, es - 2 * (size_t)kGateBytes)) return rc;
  if (int rc = up.finish()) return rc;
  if (down_is_q6) *down_is_q6 = q6 ? 1 : 0;
  return commit_layer(L, b, es, q6);
}

int fdm_layer_release(int L) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS) return fail(FDM_E_INVAL, "layer %d out of range", L);
  (void)hipDeviceSynchronize();
  release_layer(g.layers[L]);
  g.streamed[L].reset();
  return FDM_OK;
}

int fdm_layer_query(int L, size_t* expert_size, int* down_is_q6, int* n_experts) {
  Layer* y = nullptr;
  if (int rc = get_layer(L, &y)) return rc;
  if (expert_size) *expert_size = y->expert_size;
  if (down_is_q6) *down_is_q6 = y->down_q6 ? 1 : 0;
  if (n_experts) *n_experts = y->n_experts;
  return FDM_OK;
}

// ---- MoE ---------------------------------------------------------------------------
int fdm_moe_forward(int L, const float* d_h_post, const int* d_idx, const float* d_w, int K,
                    float* d_moe_out, void* stream) {
  Layer* y = nullptr;
  if (int rc = get_layer(L, &y)) return rc;
  if (int rc = check_K(K)) return rc;
  if (!d_h_post || !d_idx || !d_w || !d_moe_out) return fail(FDM_E_INVAL, "null pointer");
  hipStream_t s = as_stream(stream);
  const SlotTable t = slots_for(*y, d_idx, d_w, K, false);
  Workspace* w = nullptr;
  if (int rc = stream_workspace(s, &w)) return rc;
  {
    ProfScope p(FDM_PROF_XDIGITS, s);
    FDM_HIP(launch_xdigits(d_h_post, FDM_HIDDEN / 64, w->xd, s));
  }
  {
    ProfScope p(FDM_PROF_GATEUP, s);
    FDM_HIP(launch_gateup(t, w->xd, w->act, w->act_xd, w->gu_count, s));
  }
  {
    ProfScope p(FDM_PROF_DOWN, s);
    FDM_HIP(launch_down_combine(t, y->down_q6, w->act_xd, nullptr, d_moe_out, nullptr, w->eo, w->dn_count,
                                s));
  }
  return FDM_OK;
}

int fdm_moe_forward_host(int L, const float* h_post, const int* exp_idx, const float* exp_w,
                         int K, float* moe_out) {
  Layer* y = nullptr;
  if (int rc = get_layer(L, &y)) return rc;
  if (int rc = check_K(K)) return rc;
  if (!h_post || !exp_idx || !exp_w || !moe_out) return fail(FDM_E_INVAL, "null pointer");
  // the null stream's staging buffers: host callers take turns
  static std::mutex host_mu;
  std::lock_guard<std::mutex> lock(host_mu);
  Workspace& w = g.ws;
  FDM_HIP(hipMemcpy(w.stage_x, h_post, FDM_HIDDEN * sizeof(float), hipMemcpyHostToDevice));
  FDM_HIP(hipMemcpy(w.stage_idx, exp_idx, K * sizeof(int), hipMemcpyHostToDevice));
  FDM_HIP(hipMemcpy(w.stage_w, exp_w, K * sizeof(float), hipMemcpyHostToDevice));
  if (int rc = fdm_moe_forward(L, w.stage_x, w.stage_idx, w.stage_w, K, w.stage_y, nullptr))
    return rc;
  FDM_HIP(hipMemcpy(moe_out, w.stage_y, FDM_HIDDEN * sizeof(float), hipMemcpyDeviceToHost));
  return FDM_OK;
}

}  // extern "C"

namespace fdm {
namespace {
// One launch of the batch-1 layer kernel.  h: h_post, or with norm_w the
// hidden state whose rms_norm the kernel computes.
int run_layer(int L, const float* h, const float* norm_w, float* h_post_out, const float* h_in, int K,
              float* hidden, int* idx, float* w, void* stream) {
  Layer* y = nullptr;
  if (int rc = get_layer(L, &y)) return rc;
  if (int rc = check_K(K)) return rc;
  if (!h || !hidden) return fail(FDM_E_INVAL, "null pointer");
  if (!aligned(h, 16)) return fail(FDM_E_INVAL, "h / h_post must be 16-byte aligned");
  if (norm_w && !aligned(norm_w, 16)) return fail(FDM_E_INVAL, "norm_w must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  LayerArgs a;
  a.Wg = y->Wg;
  a.bias = y->bias;
  a.h = h;
  a.norm_w = norm_w;
  a.h_post_out = h_post_out;
  a.h_in = h_in;
  a.out = hidden;
  a.moe_out = nullptr;
  a.experts = y->experts;
  a.expert_size = y->expert_size;
  a.n_experts = y->n_experts;
  a.shared = y->shared;
  a.down_q6 = y->down_q6 ? 1 : 0;
  a.K = K;
  a.n_slots = K + (y->shared ? 1 : 0);
  Workspace* ws = nullptr;
  if (int rc = stream_workspace(s, &ws)) return rc;
  a.idx = idx ? idx : ws->idx;
  a.w = w ? w : ws->w;
  layer_workspace_args(a, ws);
  {
    ProfScope p(FDM_PROF_LAYER, s);
    FDM_HIP(launch_layer(a, s));
  }
  return FDM_OK;
}
}  // namespace
}  // namespace fdm

extern "C" {

int fdm_moe_layer(int L, const float* d_h_post, const float* d_h_in, int K, float* d_hidden,
                  int* d_idx, float* d_w, void* stream) {
  return run_layer(L, d_h_post, nullptr, nullptr, d_h_in, K, d_hidden, d_idx, d_w, stream);
}

int fdm_moe_layer_norm(int L, const float* d_h, const float* d_norm_w, int K, float* d_hidden,
                       float* d_h_post, int* d_idx, float* d_w, void* stream) {
  if (!d_norm_w) return fail(FDM_E_INVAL, "null norm weight");
  // the norm item writes h_post while router rows and digit items may still
  // read h: an h_post that overlaps h would feed them normalised values
  if (d_h_post && d_h && d_h_post < d_h + FDM_HIDDEN && d_h < d_h_post + FDM_HIDDEN)
    return fail(FDM_E_INVAL, "h_post must not overlap h");
  return run_layer(L, d_h, d_norm_w, d_h_post, d_h, K, d_hidden, d_idx, d_w, stream);
}

// ---- the streaming ceiling of a batch-1 layer's bytes (measurement only) --------------------
int fdm_layer_read_ceiling(int L, const int* d_idx, int K, const float* d_h_post, const float* d_h_in,
                           uint32_t* d_sink, void* stream) {
  Layer* y = nullptr;
  if (int rc = get_layer(L, &y)) return rc;
  if (int rc = check_K(K)) return rc;
  if (!d_idx || !d_h_post || !d_sink) return fail(FDM_E_INVAL, "null pointer");
  if (!aligned(d_h_post, 16) || (d_h_in && !aligned(d_h_in, 16)))
    return fail(FDM_E_INVAL, "h_post / h_in must be 16-byte aligned");
  ReadCeilArgs a{};
  int n = 0, tiles = 0;
  auto add = [&](const void* p, size_t b) {
    a.seg[n] = static_cast<const uint8_t*>(p);
    a.bytes[n] = b;
    a.tile0[n] = tiles;
    tiles += read_ceiling_tiles(b);
    ++n;
  };
  add(y->Wg, (size_t)FDM_N_EXPERTS * FDM_HIDDEN * sizeof(float));
  if (y->bias) add(y->bias, FDM_N_EXPERTS * sizeof(float));
  a.first_routed = n;
  for (int k = 0; k < K; ++k) add(nullptr, y->expert_size);
  if (y->shared) add(y->shared, y->expert_size);
  add(d_h_post, FDM_HIDDEN * sizeof(float));
  if (d_h_in) add(d_h_in, FDM_HIDDEN * sizeof(float));
  a.tile0[n] = tiles;
  if (tiles > FDM_HIDDEN)
    return fail(FDM_E_INVAL, "K=%d: %d tiles exceed the %d-word sink", K, tiles, FDM_HIDDEN);
  a.n_seg = n;
  a.K = K;
  a.n_tiles = tiles;
  a.experts = y->experts;
  a.expert_size = y->expert_size;
  a.n_experts = y->n_experts;
  a.idx = d_idx;
  a.sink = d_sink;
  hipStream_t s = as_stream(stream);
  {
    ProfScope p(FDM_PROF_CEILING, s);
    FDM_HIP(launch_read_ceiling(a, s));
  }
  return FDM_OK;
}

// ---- batched decode ---------------------------------------------------------------------
}  // extern "C"

namespace fdm {
namespace {
// Per-row buffers of the batched path, grown (never shrunk) to `rows`.
// Callers synchronise with earlier work on the stream before a reallocation.
int ensure_batch_rows(Workspace& w, size_t rows, hipStream_t s) {
  if (rows <= w.b_rows) return FDM_OK;
  FDM_HIP(hipStreamSynchronize(s));
  if (w.b_act) (void)hipFree(w.b_act);
  if (w.b_act_xd) (void)hipFree(w.b_act_xd);
  if (w.b_eo) (void)hipFree(w.b_eo);
  w.b_act = nullptr;
  w.b_act_xd = nullptr;
  w.b_eo = nullptr;
  w.b_rows = 0;
  FDM_HIP(hipMalloc(&w.b_act, rows * FDM_MOE_FFN * sizeof(float)));
  FDM_HIP(hipMalloc(&w.b_act_xd, rows * (FDM_MOE_FFN / 64) * sizeof(XGroup)));
  FDM_HIP(hipMalloc(&w.b_eo, rows * FDM_HIDDEN * sizeof(float)));
  w.b_rows = rows;
  return FDM_OK;
}
}  // namespace
}  // namespace fdm

namespace fdm {
namespace {
// The rms_norm output of prefill for T tokens (grown on demand).
int ensure_prefill(Workspace& w, int T, hipStream_t s) {
  if (T > w.p_tokens) {
    FDM_HIP(hipStreamSynchronize(s));
    if (w.p_hpost) (void)hipFree(w.p_hpost);
    w.p_hpost = nullptr;
    w.p_tokens = 0;
    FDM_HIP(hipMalloc(&w.p_hpost, (size_t)T * FDM_HIDDEN * sizeof(float)));
    w.p_tokens = T;
  }
  return FDM_OK;
}

// Activation planes for the grouped GEMMs of T tokens and `rows` expert
// rows: the larger of the token inputs (T x 7168) and the SwiGLU rows
// (rows x 2048), three planes (grown on demand).
int ensure_planes(Workspace& w, int T, size_t rows, hipStream_t s) {
  const size_t elems = std::max((size_t)T * FDM_HIDDEN, rows * FDM_MOE_FFN);
  const size_t nrows = std::max((size_t)T, rows);
  if (elems <= w.q_elems && nrows <= w.q_rows) return FDM_OK;
  FDM_HIP(hipStreamSynchronize(s));
  for (void* q : {(void*)w.q_planes, (void*)w.q_xs, (void*)w.q_xe})
    if (q) (void)hipFree(q);
  w.q_planes = nullptr;
  w.q_xs = nullptr;
  w.q_xe = nullptr;
  w.q_elems = w.q_rows = 0;
  FDM_HIP(hipMalloc(&w.q_planes, 3 * elems * sizeof(_Float16)));
  FDM_HIP(hipMalloc(&w.q_xs, elems / 32 * sizeof(float)));
  FDM_HIP(hipMalloc(&w.q_xe, nrows * sizeof(float)));
  w.q_elems = elems;
  w.q_rows = nrows;
  return FDM_OK;
}

// Upper bound of the chunk list of T tokens, K slots (+ shared).
int max_chunks(int T, int K, int ch) {
  return std::min(256, T * K) + (T * K + ch - 1) / ch + (T + ch - 1) / ch;
}

// Buffers of the grouped GEMMs: activation planes ([3][elems] fp16), their
// sub-block sums and row scales, and the chunk list.
struct QScratch {
  _Float16* planes;
  float* xs;
  float* xe;
  int4* chunks;
  int* n_chunks;
};

QScratch workspace_q(const Workspace& w) {
  return QScratch{w.q_planes, w.q_xs, w.q_xe, w.q_chunks, w.q_nchunks};
}

// The expert half of one step on the grouped GEMMs, after the dispatch:
// chunk list, planes of the token rows (unless x_planes_ready: the caller
// has written them), gate/up + SwiGLU into b.act, then a Q4_K down on the
// GEMM (planes of b.act first) or a Q6_K down on the dot4 kernels, into
// b.eo.  x: the fp32 token rows [T][7168].
int run_qgemm_experts(const Layer* y, const BatchArgs& b0, const float* x, int planes, const QScratch& w,
                      hipStream_t s, bool x_planes_ready = false) {
  BatchArgs b = b0;
  const int T = b.T, K = b.K;
  const size_t rows = (size_t)T * K + (y->shared ? T : 0);
  const int ch = qgemm_chunk_tokens(planes);
  const int mc = max_chunks(T, K, ch);
  if (mc > kQMaxChunks) return fail(FDM_E_INVAL, "chunk list of %d entries exceeds %d", mc, kQMaxChunks);
  b.ch = ch;
  b.chunks = w.chunks;
  b.n_chunks = w.n_chunks;
  FDM_HIP(launch_dispatch(b, s));  // with the chunk list
  if (!x_planes_ready) FDM_HIP(launch_xplanes(x, FDM_HIDDEN, (size_t)T, planes, w.planes, w.xs, w.xe, s));
  QGemmArgs q;
  q.T = T;
  q.K = K;
  q.experts = y->experts;
  q.expert_size = y->expert_size;
  q.shared = y->shared;
  q.xp = w.planes;
  q.plane = (size_t)T * FDM_HIDDEN;
  q.xs = w.xs;
  q.xe = w.xe;
  q.pair_tok = b.pair_tok;
  q.chunks = w.chunks;
  q.n_chunks = w.n_chunks;
  q.out = b.act;
  FDM_HIP(launch_qgemm(q, planes, false, mc, s));
  if (y->down_q6) {
    FDM_HIP(launch_batched_down(b, true, s));
    return FDM_OK;
  }
  FDM_HIP(launch_xplanes(b.act, FDM_MOE_FFN, rows, planes, w.planes, w.xs, w.xe, s));
  q.plane = rows * FDM_MOE_FFN;
  q.out = b.eo;
  FDM_HIP(launch_qgemm(q, planes, true, mc, s));
  return FDM_OK;
}
}  // namespace
}  // namespace fdm

extern "C" {

int fdm_rms_norm(const float* d_x, const float* d_w, float* d_o, int T, int d, void* stream) {
  if (int rc = check_ready()) return rc;
  if (!d_x || !d_o) return fail(FDM_E_INVAL, "null pointer");
  if (T < 1 || d < 1 || d > FDM_HIDDEN) return fail(FDM_E_INVAL, "T=%d d=%d (d <= %d)", T, d, FDM_HIDDEN);
  FDM_HIP(launch_rms_norm(d_x, d_w, d_o, T, d, as_stream(stream)));
  return FDM_OK;
}

int fdm_moe_prefill(const int* layers, int n_layers, float* d_H, int T, int K,
                    const float* const* d_norm_w, int* d_idx, void* stream) {
  if (int rc = check_ready()) return rc;
  if (int rc = check_K(K)) return rc;
  if (!layers || !d_H || n_layers < 1) return fail(FDM_E_INVAL, "no layers or null H");
  if (T < 1 || T > FDM_MAX_TOKENS) return fail(FDM_E_INVAL, "T=%d outside 1..%d", T, FDM_MAX_TOKENS);
  if (!aligned(d_H, 16)) return fail(FDM_E_INVAL, "H must be 16-byte aligned");
  for (int l = 0; l < n_layers; ++l) {
    Layer* y = nullptr;
    if (int rc = get_layer(layers[l], &y)) return rc;
  }
  hipStream_t s = as_stream(stream);
  Workspace* ws = nullptr;
  if (int rc = stream_workspace(s, &ws)) return rc;
  Workspace& w = *ws;
  const size_t rows = (size_t)T * K + T;
  if (int rc = ensure_prefill(w, T, s)) return rc;
  if (int rc = ensure_batch_rows(w, rows, s)) return rc;
  if (int rc = ensure_planes(w, T, rows, s)) return rc;
  ProfScope prof(FDM_PROF_PREFILL, s);
  for (int l = 0; l < n_layers; ++l) {
    Layer* y = nullptr;
    (void)get_layer(layers[l], &y);
    int* idx = d_idx ? d_idx + (size_t)l * T * K : w.idx;
    // the normalised tokens and their one fp16 plane for the expert GEMMs
    FDM_HIP(launch_rms_norm_planes(d_H, d_norm_w ? d_norm_w[l] : nullptr, w.p_hpost, T, w.q_planes, w.q_xs,
                                   w.q_xe, s));
    FDM_HIP(launch_router_logits(y->Wg, w.p_hpost, FDM_N_EXPERTS, FDM_HIDDEN, T, w.logits, s));
    FDM_HIP(launch_route(w.logits, y->bias, T, K, idx, w.w, s));
    BatchArgs b{};
    b.T = T;
    b.K = K;
    b.experts = y->experts;
    b.expert_size = y->expert_size;
    b.shared = y->shared;
    b.h_in = d_H;
    b.out = d_H;  // residual in place
    b.idx = idx;
    b.w = w.w;
    b.act = w.b_act;
    b.act_xd = w.b_act_xd;
    b.eo = w.b_eo;
    b.seg_start = w.b_seg;
    b.pair_tok = w.b_pair_tok;
    b.pair_of = w.b_pair_of;
    b.distinct = w.b_distinct;
    b.n_distinct = w.b_ndistinct;
    // prefill precision: one fp16 plane of the activations (the bar is 1e-2)
    if (int rc = run_qgemm_experts(y, b, w.p_hpost, 1, workspace_q(w), s, true)) return rc;
    FDM_HIP(launch_combine(b, s));
  }
  return FDM_OK;
}

}  // extern "C"

namespace fdm {
namespace {
// Every buffer one batched step uses besides its inputs and outputs.
struct BatchScratch {
  XGroup* xd;       // [T][112] digits of the tokens (dot4 path)
  float* logits;    // [T][256]
  int* idx;         // [T][K] routing when the caller passes none
  float* w;         // [T][K]
  int* seg;         // [257]
  int* pair_tok;    // [T*K]
  int* pair_of;     // [T*K]
  int* distinct;    // [256]
  int* n_distinct;  // [1] when the caller passes none
  float* act;       // [rows][2048]
  XGroup* act_xd;   // [rows][32]
  float* eo;        // [rows][7168]
  QScratch q;       // grouped GEMM buffers (MFMA path)
};

bool batch_uses_mfma(int T) {
  return g_batch_mode == FDM_BATCH_MFMA || (g_batch_mode == FDM_BATCH_AUTO && T >= FDM_BATCH_MFMA_MIN_T);
}

// One batched step (the body of fdm_moe_forward_batched and of its
// no-allocation variant) on buffers the caller has sized for T, K.
int batched_step(const Layer* y, const float* d_X, const float* d_H_in, int T, int K, float* d_hidden,
                 int* d_idx, float* d_w, int* d_n_distinct, const BatchScratch& sc, hipStream_t s) {
  int* idx = d_idx ? d_idx : sc.idx;
  float* w = d_w ? d_w : sc.w;
  ProfScope p(FDM_PROF_BATCH, s);
  FDM_HIP(launch_router_logits(y->Wg, d_X, FDM_N_EXPERTS, FDM_HIDDEN, T, sc.logits, s));
  FDM_HIP(launch_route(sc.logits, y->bias, T, K, idx, w, s));
  BatchArgs b;
  b.T = T;
  b.K = K;
  b.experts = y->experts;
  b.expert_size = y->expert_size;
  b.shared = y->shared;
  b.x = d_X;
  b.h_in = d_H_in;
  b.out = d_hidden;
  b.idx = idx;
  b.w = w;
  b.xd = sc.xd;
  b.act = sc.act;
  b.act_xd = sc.act_xd;
  b.eo = sc.eo;
  b.seg_start = sc.seg;
  b.pair_tok = sc.pair_tok;
  b.pair_of = sc.pair_of;
  b.distinct = sc.distinct;
  b.n_distinct = d_n_distinct ? d_n_distinct : sc.n_distinct;
  if (!batch_uses_mfma(T)) {
    FDM_HIP(launch_batched_experts(b, y->down_q6, s));
    return FDM_OK;
  }
  // grouped MFMA GEMMs at fp32 grade (three fp16 planes of the activations)
  if (int rc = run_qgemm_experts(y, b, d_X, 3, sc.q, s)) return rc;
  FDM_HIP(launch_combine(b, s));
  return FDM_OK;
}

int check_batched_args(int L, const float* d_X, int T, int K, float* d_hidden, Layer** y) {
  if (int rc = get_layer(L, y)) return rc;
  if (int rc = check_K(K)) return rc;
  if (T < 1 || T > FDM_MAX_TOKENS) return fail(FDM_E_INVAL, "T=%d outside 1..%d", T, FDM_MAX_TOKENS);
  if (!d_X || !d_hidden) return fail(FDM_E_INVAL, "null pointer");
  if (!aligned(d_X, 16)) return fail(FDM_E_INVAL, "X must be 16-byte aligned");
  return FDM_OK;
}

BatchScratch noalloc_scratch(unsigned char* base) {
  auto at = [base](NaPart part) { return static_cast<void*>(base + na_offset(part)); };
  BatchScratch sc;
  sc.xd = static_cast<XGroup*>(at(kNaXd));
  sc.logits = static_cast<float*>(at(kNaLogits));
  sc.idx = static_cast<int*>(at(kNaIdx));
  sc.w = static_cast<float*>(at(kNaW));
  sc.seg = static_cast<int*>(at(kNaSeg));
  sc.pair_tok = static_cast<int*>(at(kNaPairTok));
  sc.pair_of = static_cast<int*>(at(kNaPairOf));
  sc.distinct = static_cast<int*>(at(kNaDistinct));
  sc.n_distinct = static_cast<int*>(at(kNaNDistinct));
  sc.act = static_cast<float*>(at(kNaAct));
  sc.act_xd = static_cast<XGroup*>(at(kNaActXd));
  sc.eo = static_cast<float*>(at(kNaEo));
  sc.q = QScratch{static_cast<_Float16*>(at(kNaPlanes)), static_cast<float*>(at(kNaXs)),
                  static_cast<float*>(at(kNaXe)), static_cast<int4*>(at(kNaChunks)),
                  static_cast<int*>(at(kNaNChunks))};
  return sc;
}
}  // namespace
}  // namespace fdm

extern "C" {

int fdm_moe_forward_batched(int L, const float* d_X, const float* d_H_in, int T, int K,
                            float* d_hidden, int* d_idx, float* d_w, int* d_n_distinct,
                            void* stream) {
  Layer* y = nullptr;
  if (int rc = check_batched_args(L, d_X, T, K, d_hidden, &y)) return rc;
  hipStream_t s = as_stream(stream);
  Workspace* ws = nullptr;
  if (int rc = stream_workspace(s, &ws)) return rc;
  Workspace& w = *ws;
  const size_t rows = (size_t)T * K + (y->shared ? T : 0);
  if (int rc = ensure_batch_rows(w, rows, s)) return rc;
  if (batch_uses_mfma(T)) {
    if (int rc = ensure_planes(w, T, rows, s)) return rc;
  }
  const BatchScratch sc{w.xd,         w.logits,   w.idx,      w.w,        w.b_seg,
                        w.b_pair_tok, w.b_pair_of, w.b_distinct, w.b_ndistinct, w.b_act,
                        w.b_act_xd,   w.b_eo,      workspace_q(w)};
  return batched_step(y, d_X, d_H_in, T, K, d_hidden, d_idx, d_w, d_n_distinct, sc, s);
}

int fdm_moe_forward_batched_noalloc(int L, const float* d_X, const float* d_H_in, int T, int K,
                                    float* d_hidden, int* d_idx, float* d_w, int* d_n_distinct,
                                    void* stream) {
  Layer* y = nullptr;
  if (int rc = check_batched_args(L, d_X, T, K, d_hidden, &y)) return rc;
  if (T > FDM_NOALLOC_MAX_T || T * K > FDM_NOALLOC_MAX_PAIRS)
    return fail(FDM_E_INVAL, "T=%d, K=%d exceed the no-allocation scratch (T <= %d, T*K <= %d)", T, K,
                FDM_NOALLOC_MAX_T, FDM_NOALLOC_MAX_PAIRS);
  unsigned char* base = g_scratch_ptr[g.device];
  if (!base) return fail(FDM_E_STATE, "no-allocation scratch not bound on device %d", g.device);
  return batched_step(y, d_X, d_H_in, T, K, d_hidden, d_idx, d_w, d_n_distinct, noalloc_scratch(base),
                      as_stream(stream));
}

int fdm_set_layer_spin_limit(unsigned polls, unsigned* prev) {
  if (int rc = check_ready()) return rc;
  if (prev) *prev = g_layer_spin_limit;
  g_layer_spin_limit = polls ? polls : kLayerSpinLimit;
  return FDM_OK;
}

int fdm_set_batch_kernel(int mode, int* prev) {
  if (int rc = check_ready()) return rc;
  if (mode != FDM_BATCH_AUTO && mode != FDM_BATCH_DOT4 && mode != FDM_BATCH_MFMA)
    return fail(FDM_E_INVAL, "batch kernel mode %d", mode);
  if (prev) *prev = g_batch_mode;
  g_batch_mode = mode;
  return FDM_OK;
}

// ---- per-kernel timing ----------------------------------------------------------------
int fdm_prof_enable(int on) {
  if (int rc = check_ready()) return rc;
  Prof& p = g.prof;
  std::lock_guard<std::recursive_mutex> lock(p.mu);
  if (on && p.created == 0) {
    for (int i = 0; i < Prof::kPool; ++i) {
      FDM_HIP(hipEventCreate(&p.start[i]));
      FDM_HIP(hipEventCreate(&p.stop[i]));
      p.created = i + 1;
    }
    prof_clear_stats();
  }
  if (!on && p.on) {
    if (int rc = prof_drain()) return rc;
  }
  p.on = on != 0;
  return FDM_OK;
}

int fdm_prof_reset(void) {
  if (int rc = check_ready()) return rc;
  std::lock_guard<std::recursive_mutex> lock(g.prof.mu);
  if (g.prof.created == 0) return FDM_OK;
  if (int rc = prof_drain()) return rc;
  prof_clear_stats();
  return FDM_OK;
}

int fdm_prof_read(int phase, int* count, double* total_ms, double* min_ms, double* max_ms) {
  if (int rc = check_ready()) return rc;
  if (phase < 0 || phase >= FDM_PROF_PHASES) return fail(FDM_E_INVAL, "phase %d", phase);
  Prof& p = g.prof;
  std::lock_guard<std::recursive_mutex> lock(p.mu);
  if (p.created == 0) {
    if (count) *count = 0;
    if (total_ms) *total_ms = 0.0;
    if (min_ms) *min_ms = 0.0;
    if (max_ms) *max_ms = 0.0;
    return FDM_OK;
  }
  if (int rc = prof_drain()) return rc;
  if (count) *count = p.count[phase];
  if (total_ms) *total_ms = p.total[phase];
  if (min_ms) *min_ms = p.count[phase] ? p.mn[phase] : 0.0;
  if (max_ms) *max_ms = p.mx[phase];
  return FDM_OK;
}

// ---- synthetic data ------------------------------------------------------------------
// ---- streamed layers (experts read from the layer file on demand) -------------------
int fdm_layer_stream_open(int L, const char* layer_file, size_t expert_size, int n_experts,
                          const float* d_Wg, const float* d_bias, const void* d_shared, int n_cache,
                          int n_threads) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS) return fail(FDM_E_INVAL, "layer %d out of range", L);
  if (!layer_file || !d_Wg) return fail(FDM_E_INVAL, "null layer file or router weights");
  if (n_experts != FDM_N_EXPERTS)
    return fail(FDM_E_INVAL, "n_experts=%d: the router is the R1 256-expert router", n_experts);
  bool q6 = false;
  if (int rc = down_type(expert_size, &q6)) return rc;
  if (n_cache < 1 || n_cache > n_experts) return fail(FDM_E_INVAL, "n_cache=%d: 1 .. n_experts", n_cache);
  if (n_threads < 0 || n_threads > 64) return fail(FDM_E_INVAL, "n_threads=%d: 0 (default 8) .. 64", n_threads);
  if (!aligned(d_Wg, 16) || (d_shared && !aligned(d_shared, 16)))
    return fail(FDM_E_INVAL, "router weights and shared expert must be 16-byte aligned");
  auto st = std::make_unique<StreamedLayer>();
  FDM_HIP(hipEventCreateWithFlags(&st->done, hipEventDisableTiming));
  FDM_HIP(hipEventRecord(st->done, nullptr));
  std::string err;
  if (int rc = st->es.open(layer_file, expert_size, n_experts, n_cache, n_threads ? n_threads : 8, g.device, &err))
    return fail(rc, "layer %d: %s", L, err.c_str());
  if (d_shared) {
    if (hipMalloc(&st->shared, expert_size) != hipSuccess) return fail(FDM_E_NOMEM, "cannot allocate the shared expert");
    FDM_HIP(hipMemcpy(st->shared, d_shared, expert_size, hipMemcpyDeviceToDevice));
  }
  st->Wg = d_Wg;
  st->bias = d_bias;
  st->expert_size = expert_size;
  st->q6 = q6;
  (void)hipDeviceSynchronize();
  release_layer(g.layers[L]);
  g.streamed[L] = std::move(st);
  return FDM_OK;
}

int fdm_moe_layer_streamed(int L, const float* d_h_post, const float* d_h_in, int K, float* d_hidden,
                           int* d_idx, float* d_w, void* stream) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS || !g.streamed[L]) return fail(FDM_E_STATE, "layer %d is not streamed", L);
  if (int rc = check_K(K)) return rc;
  if (!d_h_post || !d_hidden) return fail(FDM_E_INVAL, "null pointer");
  if (!aligned(d_h_post, 16)) return fail(FDM_E_INVAL, "h_post must be 16-byte aligned");
  StreamedLayer& y = *g.streamed[L];
  if (K > y.es.n_cache()) return fail(FDM_E_INVAL, "K=%d exceeds the layer's %d cache slots", K, y.es.n_cache());
  hipStream_t s = as_stream(stream);
  Workspace* ws = nullptr;
  if (int rc = stream_workspace(s, &ws)) return rc;
  Workspace& w = *ws;
  if (!w.ids_h) {
    FDM_HIP(hipHostMalloc(reinterpret_cast<void**>(&w.ids_h), FDM_MAX_K * sizeof(int), hipHostMallocDefault));
    FDM_HIP(hipHostMalloc(reinterpret_cast<void**>(&w.slots_h), FDM_MAX_K * sizeof(int), hipHostMallocDefault));
  }
  // route on the device (infer.m:1881-1883), then the ids to the host
  FDM_HIP(launch_router_logits(y.Wg, d_h_post, FDM_N_EXPERTS, FDM_HIDDEN, 1, w.logits, s));
  FDM_HIP(launch_route(w.logits, y.bias, 1, K, w.idx, w.w, s));
  FDM_HIP(hipMemcpyAsync(w.ids_h, w.idx, K * sizeof(int), hipMemcpyDeviceToHost, s));
  FDM_HIP(hipStreamSynchronize(s));
  std::lock_guard<std::mutex> lock(y.mu);
  FDM_HIP(hipEventSynchronize(y.done));  // the previous call's kernels have read the cache
  std::string err;
  bool miss[FDM_MAX_K];
  if (int rc = y.es.plan(w.ids_h, K, w.slots_h, miss, &err)) return fail(rc, "layer %d: %s", L, err.c_str());
  FDM_HIP(hipMemcpyAsync(w.stage_idx, w.slots_h, K * sizeof(int), hipMemcpyHostToDevice, s));
  SlotTable t;
  t.experts = y.es.cache();
  t.expert_size = y.expert_size;
  t.n_experts = y.es.n_cache();
  t.shared = y.shared;
  t.idx = w.stage_idx;
  t.w = w.w;
  t.K = K;
  t.n_slots = K + (y.shared ? 1 : 0);
  t.rel = false;
  FDM_HIP(launch_xdigits(d_h_post, FDM_HIDDEN / 64, w.xd, s));
  // the shared expert and the cache hits at once, in one launch pair ...
  SlotTable now = t;
  for (int k = 0; k < K; ++k)
    if (miss[k]) now.skip |= 1u << k;
  if (now.skip != (1u << t.n_slots) - 1) {
    FDM_HIP(launch_gateup(now, w.xd, w.act, w.act_xd, w.gu_count, s));
    FDM_HIP(launch_down_combine(now, y.q6, w.act_xd, d_h_in, d_hidden, nullptr, w.eo, w.dn_count, s));
  }
  // ... and each miss as soon as its copies land, while the others are read
  // (whichever launch completes a row tile's last slot combines it, in slot
  // order: the same bits as one launch)
  auto ready = [&](int k) -> int {
    if (launch_gateup(t, w.xd, w.act, w.act_xd, w.gu_count, s, k, 1) != hipSuccess ||
        launch_down_combine(t, y.q6, w.act_xd, d_h_in, d_hidden, nullptr, w.eo, w.dn_count, s, k, 1) != hipSuccess)
      return FDM_E_HIP;
    return FDM_OK;
  };
  const int read_rc = y.es.read(s, ready, &err);
  if (read_rc != FDM_OK) {
    (void)hipEventRecord(y.done, s);
    return fail(read_rc, "layer %d: %s", L, err.c_str());
  }
  FDM_HIP(hipEventRecord(y.done, s));
  if (d_idx) FDM_HIP(hipMemcpyAsync(d_idx, w.idx, K * sizeof(int), hipMemcpyDeviceToDevice, s));
  if (d_w) FDM_HIP(hipMemcpyAsync(d_w, w.w, K * sizeof(float), hipMemcpyDeviceToDevice, s));
  return FDM_OK;
}

int fdm_stream_stats(int L, uint64_t* hits, uint64_t* misses, uint64_t* bytes_read) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS || !g.streamed[L]) return fail(FDM_E_STATE, "layer %d is not streamed", L);
  const ExpertStream& es = g.streamed[L]->es;
  if (hits) *hits = es.hits();
  if (misses) *misses = es.misses();
  if (bytes_read) *bytes_read = es.bytes_read();
  return FDM_OK;
}

static int tensor_to_f16(const GgufManifest& m, const GgufTensor& t, Uploader& up, uint16_t* dst, size_t n);

// ---- MLA attention layers ---------------------------------------------------------------
// yarn_freq(i) of infer.m:586-624 (YaRN correction range of the 64 rope
// dims, base 10000, original context 4096, factor 40), in float as there.
static void yarn_table(float* f) {
  const int dim = 64;
  const float base = 10000.0f, orig = 4096.0f, twopi = 2.0f * (float)M_PI;
  const float lo_f = ((float)dim * logf(orig / (32.0f * twopi))) / (2.0f * logf(base));
  const float hi_f = ((float)dim * logf(orig / (1.0f * twopi))) / (2.0f * logf(base));
  int lo = (int)floorf(lo_f), hi = (int)ceilf(hi_f);
  if (lo < 0) lo = 0;
  if (hi > dim / 2 - 1) hi = dim / 2 - 1;
  if (hi <= lo) hi = lo + 1;
  for (int i = 0; i < dim / 2; ++i) {
    const float freq_extra = 1.0f / powf(base, (float)(2 * i) / (float)dim);
    const float freq_inter = freq_extra / 40.0f;
    float denom = (float)(hi - lo);
    if (denom < 1e-3f) denom = 1e-3f;
    float ramp = ((float)i - (float)lo) / denom;
    if (ramp < 0.0f) ramp = 0.0f;
    if (ramp > 1.0f) ramp = 1.0f;
    const float mask = 1.0f - ramp;
    f[i] = freq_inter * (1.0f - mask) + freq_extra * mask;
  }
}

// The attention scratch of workspace w for a cache of seq positions (grown,
// never shrunk, after the stream's earlier work).
static int ensure_attn(Workspace& w, int seq, hipStream_t s) {
  AttnScratch& ws = w.attn;
  if (ws.seq >= seq) return FDM_OK;
  FDM_HIP(hipStreamSynchronize(s));
  ws.release();
  const size_t H = FDM_HIDDEN, QA = 1536, QB = 128 * 192, KVA = 576, O = 128 * 128;
  const size_t chunks = (size_t)((seq + kMlaChunkPos - 1) / kMlaChunkPos);
  // normed[0]: the attention norm's 1 / rms (the rest of H is spare)
  const size_t n[] = {H, QA + KVA, QB, 128 * 512, 128 * 512, O, chunks * 128 * 512, chunks * 128 * 2};
  float** p[] = {&ws.normed, &ws.q_a, &ws.q, &ws.q_abs, &ws.wc, &ws.attn, &ws.part, &ws.stat};
  for (int i = 0; i < 8; ++i)
    if (hipMalloc(p[i], n[i] * 4) != hipSuccess) {
      ws.release();
      return fail(FDM_E_NOMEM, "cannot allocate the attention scratch");
    }
  ws.kv_a = ws.q_a + QA;  // q_a and kv_a: one [1536 + 576] output
  ws.seq = seq;
  return FDM_OK;
}

int fdm_attn_upload(int L, const fdm_attn_weights* w, int max_seq) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS) return fail(FDM_E_INVAL, "layer %d out of range", L);
  if (!w || !w->attn_norm || !w->q_a || !w->q_a_norm || !w->q_b || !w->kv_a || !w->kv_a_norm || !w->k_b ||
      !w->v_b || !w->o_proj)
    return fail(FDM_E_INVAL, "null attention weight");
  if (max_seq < 1 || max_seq > FDM_ATTN_MAX_SEQ) return fail(FDM_E_INVAL, "max_seq %d: 1 .. %d", max_seq, FDM_ATTN_MAX_SEQ);
  auto a = std::make_unique<AttnLayer>();
  const size_t H = FDM_HIDDEN, QA = 1536, QB = 128 * 192, KVA = 576, KB = 128 * 512 * 128, O = 128 * 128;
  struct M {
    void** dst;
    const void* src;
    size_t bytes;
  } m[] = {{(void**)&a->attn_norm, w->attn_norm, H * 4}, {(void**)&a->q_a_norm, w->q_a_norm, QA * 4},
           {(void**)&a->kv_a_norm, w->kv_a_norm, 512 * 4}, {(void**)&a->q_b, w->q_b, QB * QA * 2},
           {(void**)&a->k_b, w->k_b, KB * 2}, {(void**)&a->v_b, w->v_b, KB * 2}, {(void**)&a->o_proj, w->o_proj, H * O * 2}};
  for (const M& x : m) {
    if (hipMalloc(x.dst, x.bytes) != hipSuccess) return fail(FDM_E_NOMEM, "cannot allocate attention layer %d", L);
    FDM_HIP(hipMemcpy(*x.dst, x.src, x.bytes, hipMemcpyHostToDevice));
  }
  // q_a and kv_a stacked in one allocation ([1536 + 576][7168]): the forward
  // runs both projections, which read the same input, as one matvec
  if (hipMalloc(&a->q_a, (QA + KVA) * H * 2) != hipSuccess)
    return fail(FDM_E_NOMEM, "cannot allocate attention layer %d", L);
  a->kv_a = a->q_a + QA * H;
  FDM_HIP(hipMemcpy(a->q_a, w->q_a, QA * H * 2, hipMemcpyHostToDevice));
  FDM_HIP(hipMemcpy(a->kv_a, w->kv_a, KVA * H * 2, hipMemcpyHostToDevice));
  float freq[32];
  yarn_table(freq);
  if (hipMalloc(&a->freq, sizeof freq) != hipSuccess ||
      hipMalloc(&a->cache_c, (size_t)max_seq * 512 * 4) != hipSuccess ||
      hipMalloc(&a->cache_k, (size_t)max_seq * 64 * 4) != hipSuccess)
    return fail(FDM_E_NOMEM, "cannot allocate the KV cache of layer %d", L);
  FDM_HIP(hipMemcpy(a->freq, freq, sizeof freq, hipMemcpyHostToDevice));
  a->max_seq = max_seq;
  if (int rc = ensure_attn(g.ws, max_seq, nullptr)) return rc;  // the null stream's, made ahead
  (void)hipDeviceSynchronize();
  g.attn[L] = std::move(a);
  return FDM_OK;
}

int fdm_attn_load_gguf(int L, const fdm_gguf* mh, int max_seq) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS) return fail(FDM_E_INVAL, "layer %d out of range", L);
  const GgufManifest* m = gguf_manifest(mh);
  if (!m) return fail(FDM_E_INVAL, "null manifest");
  const std::initializer_list<uint32_t> fp = {FDM_GGML_F32, FDM_GGML_F16, FDM_GGML_BF16};
  const std::initializer_list<uint32_t> any = {FDM_GGML_F32, FDM_GGML_F16, FDM_GGML_BF16, FDM_GGML_Q4_K,
                                               FDM_GGML_Q6_K};
  char name[128];
  auto find = [&](const char* what, const GgufTensor** out, std::initializer_list<uint32_t> types,
                  std::initializer_list<uint64_t> dims) {
    snprintf(name, sizeof name, "blk.%d.%s.weight", L, what);
    return expect_tensor(*m, name, out, types, dims);
  };
  const GgufTensor *tn, *tqan, *tkvn, *tqa, *tqb, *tkva, *to, *tkb = nullptr, *tvb = nullptr, *tkvb = nullptr;
  if (int rc = find("attn_norm", &tn, fp, {FDM_HIDDEN})) return rc;
  if (int rc = find("attn_q_a_norm", &tqan, fp, {1536})) return rc;
  if (int rc = find("attn_kv_a_norm", &tkvn, fp, {512})) return rc;
  if (int rc = find("attn_q_a", &tqa, any, {FDM_HIDDEN, 1536})) return rc;
  if (int rc = find("attn_q_b", &tqb, any, {1536, 128 * 192})) return rc;
  if (int rc = find("attn_kv_a_mqa", &tkva, any, {FDM_HIDDEN, 576})) return rc;
  if (int rc = find("attn_output", &to, any, {128 * 128, FDM_HIDDEN})) return rc;
  // per head k_b [NOPE][KV_LORA] and v_b [V_HEAD][KV_LORA], or kv_b [NOPE + V_HEAD][KV_LORA]
  // (infer.m:1746-1778); the element count is what the reference relies on
  snprintf(name, sizeof name, "blk.%d.attn_k_b.weight", L);
  const bool split = m->find(name) != nullptr;
  if (split) {
    if (int rc = find("attn_k_b", &tkb, any, {512, 128, 128})) return rc;
    if (int rc = find("attn_v_b", &tvb, any, {512, 128, 128})) return rc;
  } else if (int rc = find("attn_kv_b", &tkvb, any, {512, 256 * 128})) {
    return rc;
  }
  std::vector<float> an, qan, kvn;
  if (int rc = read_f32(*m, *tn, an)) return rc;
  if (int rc = read_f32(*m, *tqan, qan)) return rc;
  if (int rc = read_f32(*m, *tkvn, kvn)) return rc;
  // the matrices, converted on the device into host arrays for fdm_attn_upload's copy
  const size_t KB = (size_t)128 * 512 * 128;
  std::vector<uint16_t> hqa((size_t)1536 * FDM_HIDDEN), hqb((size_t)128 * 192 * 1536), hkva((size_t)576 * FDM_HIDDEN),
      hkb(KB), hvb(KB), ho((size_t)FDM_HIDDEN * 128 * 128);
  uint16_t* dev = nullptr;
  const size_t max_n = std::max(ho.size(), (size_t)2 * KB);
  if (hipMalloc(&dev, 2 * max_n * sizeof(uint16_t)) != hipSuccess) return fail(FDM_E_NOMEM, "cannot stage attention weights");
  std::unique_ptr<uint16_t, void (*)(uint16_t*)> keep(dev, [](uint16_t* p) { (void)hipFree(p); });
  uint16_t* tmp = dev + max_n;
  Uploader up;
  if (int rc = up.init()) return rc;
  auto plain = [&](const GgufTensor* t, std::vector<uint16_t>& h) {
    if (int rc = tensor_to_f16(*m, *t, up, dev, h.size())) return rc;
    FDM_HIP(hipMemcpy(h.data(), dev, h.size() * 2, hipMemcpyDeviceToHost));
    return FDM_OK;
  };
  if (int rc = plain(tqa, hqa)) return rc;
  if (int rc = plain(tqb, hqb)) return rc;
  if (int rc = plain(tkva, hkva)) return rc;
  if (int rc = plain(to, ho)) return rc;
  if (split) {
    if (int rc = tensor_to_f16(*m, *tkb, up, tmp, KB)) return rc;
    FDM_HIP(launch_transpose_heads(tmp, (size_t)128 * 512, dev, 128, 128, 512, 0));
    FDM_HIP(hipMemcpy(hkb.data(), dev, KB * 2, hipMemcpyDeviceToHost));
    if (int rc = plain(tvb, hvb)) return rc;
  } else {
    if (int rc = tensor_to_f16(*m, *tkvb, up, tmp, 2 * KB)) return rc;
    FDM_HIP(launch_transpose_heads(tmp, (size_t)256 * 512, dev, 128, 128, 512, 0));
    FDM_HIP(hipMemcpy(hkb.data(), dev, KB * 2, hipMemcpyDeviceToHost));
    FDM_HIP(hipMemcpy2D(hvb.data(), (size_t)128 * 512 * 2, tmp + (size_t)128 * 512, (size_t)256 * 512 * 2,
                        (size_t)128 * 512 * 2, 128, hipMemcpyDeviceToHost));
  }
  fdm_attn_weights w = {an.data(), hqa.data(), qan.data(), hqb.data(), hkva.data(), kvn.data(),
                        hkb.data(), hvb.data(), ho.data()};
  return fdm_attn_upload(L, &w, max_seq);
}

int fdm_attn_reset(int L) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS || !g.attn[L]) return fail(FDM_E_STATE, "attention layer %d not resident", L);
  g.attn[L]->len = 0;
  return FDM_OK;
}

int fdm_attn_len(int L, int* len) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS || !g.attn[L]) return fail(FDM_E_STATE, "attention layer %d not resident", L);
  if (len) *len = g.attn[L]->len;
  return FDM_OK;
}

int fdm_attn_release(int L) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS) return fail(FDM_E_INVAL, "layer %d out of range", L);
  (void)hipDeviceSynchronize();
  g.attn[L].reset();
  return FDM_OK;
}

int fdm_attn_forward(int L, float* d_hidden, int pos, void* stream) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS || !g.attn[L]) return fail(FDM_E_STATE, "attention layer %d not resident", L);
  if (!d_hidden || !aligned(d_hidden, 16)) return fail(FDM_E_INVAL, "hidden must be a 16-byte aligned pointer");
  if (pos < 0) return fail(FDM_E_INVAL, "pos %d", pos);
  AttnLayer& a = *g.attn[L];
  if (a.len >= a.max_seq) return fail(FDM_E_INVAL, "KV cache of layer %d is full (%d)", L, a.max_seq);
  hipStream_t s = as_stream(stream);
  Workspace* w = nullptr;
  if (int rc = stream_workspace(s, &w)) return rc;
  if (int rc = ensure_attn(*w, a.max_seq, s)) return rc;
  AttnScratch& ws = w->attn;
  ProfScope prof(FDM_PROF_ATTN, s);
  // q_a and kv_a (infer.m:781-789) read the same input: one matvec over the
  // stacked [1536 + 576] rows against hidden * attn_norm, the attention
  // norm's 1 / rms computed beside it (ws.normed[0]) and applied by the
  // launches after: q_b with the q_a norm inside it, the latent's norm and
  // k_rope in the prep launch
  FDM_HIP(launch_mv_f16_xw(a.q_a, d_hidden, a.attn_norm, ws.q_a, 1536 + 576, ws.normed, s));
  FDM_HIP(launch_mv_f16_rn(a.q_b, ws.q_a, ws.normed, a.q_a_norm, ws.q, 128 * 192, 1536, s));
  // softmax scale with the YaRN mscale (infer.m:802-815), in float as there
  const float mscale = 0.1f * logf(40.0f) + 1.0f;
  MlaArgs m;
  m.q = ws.q;
  m.kv_a = ws.kv_a;
  m.kv_scale = ws.normed;
  m.kv_a_norm = a.kv_a_norm;
  m.freq = a.freq;
  m.pos = pos;
  m.len = a.len;
  m.cache_c = a.cache_c;
  m.cache_k = a.cache_k;
  m.k_b = a.k_b;
  m.v_b = a.v_b;
  m.q_abs = ws.q_abs;
  m.wc = ws.wc;
  m.attn = ws.attn;
  m.part = ws.part;
  m.stat = ws.stat;
  m.scale = (mscale * mscale) / sqrtf(192.0f);
  FDM_HIP(launch_mla_attend(m, s));
  FDM_HIP(launch_mv_f16(a.o_proj, ws.attn, d_hidden, d_hidden, FDM_HIDDEN, 128 * 128, s));
  ++a.len;
  return FDM_OK;
}

// ---- dense FFN layers ---------------------------------------------------------------
int fdm_f32_to_f16(const float* d_src, uint16_t* d_dst, size_t n, void* stream) {
  if (int rc = check_ready()) return rc;
  if (!d_src || !d_dst) return fail(FDM_E_INVAL, "null pointer");
  if (n == 0) return FDM_OK;
  FDM_HIP(launch_to_f16(d_src, kGgmlF32, d_dst, n, static_cast<hipStream_t>(stream)));
  return FDM_OK;
}

static int dense_copy_in(int L, const uint16_t* gate, const uint16_t* up, const uint16_t* down, int inter,
                         hipMemcpyKind kind) {
  if (int rc = check_dense(L, inter)) return rc;
  if (!gate || !up || !down) return fail(FDM_E_INVAL, "null weight pointer");
  DenseBuffers b;
  if (int rc = b.alloc(inter, L)) return rc;
  const size_t n = (size_t)inter * FDM_HIDDEN * sizeof(uint16_t);
  const uint16_t* src[3] = {gate, up, down};
  for (int i = 0; i < 3; ++i) FDM_HIP(hipMemcpy(b.m[i], src[i], n, kind));
  FDM_HIP(hipDeviceSynchronize());
  b.commit(L, inter);
  return FDM_OK;
}

int fdm_dense_upload(int L, const uint16_t* h_gate, const uint16_t* h_up, const uint16_t* h_down, int inter) {
  return dense_copy_in(L, h_gate, h_up, h_down, inter, hipMemcpyHostToDevice);
}

int fdm_dense_attach(int L, const uint16_t* d_gate, const uint16_t* d_up, const uint16_t* d_down, int inter) {
  return dense_copy_in(L, d_gate, d_up, d_down, inter, hipMemcpyDeviceToDevice);
}

// One GGUF tensor (F32, F16, BF16, Q4_K or Q6_K) -> n F16 values at dst, as
// dequant_tensor_f16 makes them (infer.m:530-538): the type's fp32 values
// (the bit-exact dequant kernels for Q4_K / Q6_K), then (__fp16).
// Synchronous; temporary device buffers are freed before it returns.
static int tensor_to_f16(const GgufManifest& m, const GgufTensor& t, Uploader& up, uint16_t* dst, size_t n) {
  struct Bufs {
    void *raw = nullptr, *wide = nullptr;
    ~Bufs() {
      if (raw) (void)hipFree(raw);
      if (wide) (void)hipFree(wide);
    }
  } b;
  if (hipMalloc(&b.raw, t.nbytes) != hipSuccess) return fail(FDM_E_NOMEM, "cannot stage %s", t.name.c_str());
  if (int rc = up.copy(b.raw, t.nbytes, [&](void* d, uint64_t k, uint64_t off) { return m.read(t, d, k, off); }))
    return rc;
  if (int rc = up.finish()) return rc;
  if (t.type == FDM_GGML_Q4_K || t.type == FDM_GGML_Q6_K) {
    if (hipMalloc(&b.wide, n * sizeof(float)) != hipSuccess) return fail(FDM_E_NOMEM, "cannot widen %s", t.name.c_str());
    if (t.type == FDM_GGML_Q4_K)
      FDM_HIP(launch_dequant_q4k(static_cast<const uint8_t*>(b.raw), static_cast<float*>(b.wide), n / FDM_QK_K, 0));
    else
      FDM_HIP(launch_dequant_q6k(static_cast<const uint8_t*>(b.raw), static_cast<float*>(b.wide), n / FDM_QK_K, 0));
    FDM_HIP(launch_to_f16(b.wide, kGgmlF32, dst, n, 0));
  } else {
    FDM_HIP(launch_to_f16(b.raw, (int)t.type, dst, n, 0));
  }
  FDM_HIP(hipDeviceSynchronize());
  return FDM_OK;
}

int fdm_dense_load_gguf(int L, const fdm_gguf* mh, int* inter_out) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS) return fail(FDM_E_INVAL, "layer %d out of range", L);
  const GgufManifest* m = gguf_manifest(mh);
  if (!m) return fail(FDM_E_INVAL, "null manifest");
  char name[128];
  snprintf(name, sizeof name, "blk.%d.ffn_gate.weight", L);
  const GgufTensor* t0 = m->find(name);
  if (!t0) return fail(FDM_E_FORMAT, "tensor %s not in the GGUF", name);
  if (t0->n_dims != 2 || t0->dims[0] != FDM_HIDDEN)
    return fail(FDM_E_FORMAT, "tensor %s: expected [%d, inter]", name, FDM_HIDDEN);
  const int inter = (int)t0->dims[1];
  if (int rc = check_dense(L, inter)) return rc;
  const std::initializer_list<uint32_t> types = {FDM_GGML_F32, FDM_GGML_F16, FDM_GGML_BF16, FDM_GGML_Q4_K,
                                                 FDM_GGML_Q6_K};
  const char* which[3] = {"gate", "up", "down"};
  const GgufTensor* t[3] = {};
  for (int i = 0; i < 3; ++i) {
    snprintf(name, sizeof name, "blk.%d.ffn_%s.weight", L, which[i]);
    if (i < 2) {
      if (int rc = expect_tensor(*m, name, &t[i], types, {FDM_HIDDEN, (uint64_t)inter})) return rc;
    } else if (int rc = expect_tensor(*m, name, &t[i], types, {(uint64_t)inter, FDM_HIDDEN})) {
      return rc;
    }
  }
  DenseBuffers b;
  if (int rc = b.alloc(inter, L)) return rc;
  const size_t n = (size_t)inter * FDM_HIDDEN;
  Uploader up;
  if (int rc = up.init()) return rc;
  for (int i = 0; i < 3; ++i)
    if (int rc = tensor_to_f16(*m, *t[i], up, b.m[i], n)) return rc;
  b.commit(L, inter);
  if (inter_out) *inter_out = inter;
  return FDM_OK;
}

int fdm_dense_release(int L) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS) return fail(FDM_E_INVAL, "layer %d out of range", L);
  (void)hipDeviceSynchronize();
  release_dense(g.dense[L]);
  return FDM_OK;
}

int fdm_dense_query(int L, int* inter) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS) return fail(FDM_E_INVAL, "layer %d out of range", L);
  if (!g.dense[L].inter) return fail(FDM_E_STATE, "dense layer %d not resident", L);
  if (inter) *inter = g.dense[L].inter;
  return FDM_OK;
}

int fdm_dense_ffn(int L, const float* d_h_post, const float* d_h_in, float* d_hidden, void* stream) {
  if (int rc = check_ready()) return rc;
  if (L < 0 || L >= FDM_MAX_LAYERS) return fail(FDM_E_INVAL, "layer %d out of range", L);
  const DenseLayer& d = g.dense[L];
  if (!d.inter) return fail(FDM_E_STATE, "dense layer %d not resident", L);
  if (!d_h_post || !d_hidden) return fail(FDM_E_INVAL, "null pointer");
  if (!aligned(d_h_post, 16)) return fail(FDM_E_INVAL, "h_post must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  Workspace* w = nullptr;
  if (int rc = stream_workspace(s, &w)) return rc;
  ProfScope prof(FDM_PROF_DENSE, s);
  DenseArgs a;
  a.gate = d.gate;
  a.up = d.up;
  a.down = d.down;
  a.x = d_h_post;
  a.h_in = d_h_in;
  a.act = w->dense_act;
  a.out = d_hidden;
  a.inter = d.inter;
  a.n_cus = g_num_cus;
  FDM_HIP(launch_dense_ffn(a, s));
  return FDM_OK;
}

int fdm_synth_q4k(void* d_dst, size_t n_blocks, uint64_t seed, void* stream) {
  if (int rc = check_ready()) return rc;
  if (!d_dst || !aligned(d_dst, 8)) return fail(FDM_E_INVAL, "destination must be 8-byte aligned");
  if (n_blocks == 0) return FDM_OK;
  FDM_HIP(launch_synth_q4k(static_cast<uint8_t*>(d_dst), n_blocks, seed, as_stream(stream)));
  return FDM_OK;
}

int fdm_synth_q6k(void* d_dst, size_t n_blocks, uint64_t seed, void* stream) {
  if (int rc = check_ready()) return rc;
  if (!d_dst || !aligned(d_dst, 8)) return fail(FDM_E_INVAL, "destination must be 8-byte aligned");
  if (n_blocks == 0) return FDM_OK;
  FDM_HIP(launch_synth_q6k(static_cast<uint8_t*>(d_dst), n_blocks, seed, as_stream(stream)));
  return FDM_OK;
}

int fdm_synth_normal(float* d_dst, size_t n, float mean, float std_dev, uint64_t seed,
                     void* stream) {
  if (int rc = check_ready()) return rc;
  if (!d_dst) return fail(FDM_E_INVAL, "null pointer");
  if (n == 0) return FDM_OK;
  FDM_HIP(launch_synth_normal(d_dst, n, mean, std_dev, seed, as_stream(stream)));
  return FDM_OK;
}

}  // extern "C"
