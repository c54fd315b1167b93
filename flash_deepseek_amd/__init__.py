"""flash_deepseek_amd -- MI355X (gfx950) MoE expert hot path of flash_deepseek.

The Python layer is a thin host-side mirror of the reference's C operators
for this path, over the C ABI of libfdm.so (include/fdm.h):

  reference (infer.m / quant.c)            here
  ---------------------------------------  ----------------------------------
  metal_init(model_path)        :1276      init(device)
  dequantize_row_q4_K / _q6_K   quant.c    dequantize_row_q4_K / _q6_K (device)
  fp16_to_fp32                  quant.c:4  fp16_to_fp32 (device, vectorised)
  enc_matvec_q + dequant_matvec_q4k/q6k    matvec_q4k / matvec_q6k
  encode_expert                 :1559      expert_ffn
  mv(gate_inp) + route()        :1881-1883 router_logits + route
  load_layer_weights (MoE part) :1794      attach_layer / upload_layer
  metal_moe_forward             :1604      moe_forward / moe_forward_host
  layer_forward MoE branch      :1878-1922 moe_layer
  expert streaming (flash)      :1478-1602 stream_layer / moe_layer_streamed
  mla_forward                   :766-903   attn_upload / attn_forward
  layer_forward dense branch    :1852-1868 dense_ffn (weights: upload_dense /
                                           attach_dense / load_dense_gguf)

Tensors are torch tensors on the GPU (torch provides device memory and the
current stream; all compute is the library's own HIP kernels).  Every call
is asynchronous on torch's current stream unless noted.
"""
import ctypes

from . import _lib
from ._lib import (DENSE_FFN, EXPERT_Q4K_BYTES, EXPERT_Q6K_BYTES, HIDDEN, MAX_K, MAX_LAYERS, MAX_TOKENS,
                   MOE_FFN, N_EXPERTS, Q4K_BLOCK_SIZE, Q6K_BLOCK_SIZE, QK_K, FdmError)

__all__ = [
    "init", "shutdown", "sync", "set_layer_spin_limit", "available", "dequantize_row_q4_K", "dequantize_row_q6_K",
    "fp16_to_fp32", "matvec_q4k", "matvec_q6k", "expert_ffn", "router_logits", "route",
    "attach_layer", "upload_layer", "release_layer", "layer_info", "moe_forward",
    "moe_forward_host", "moe_layer", "f32_to_f16", "upload_dense", "attach_dense", "load_dense_gguf",
    "release_dense", "dense_info", "dense_ffn", "DENSE_FFN", "stream_layer", "moe_layer_streamed",
    "stream_stats", "attn_upload", "attn_load_gguf", "attn_forward", "attn_reset", "attn_len", "attn_release", "set_batch_kernel", "BATCH_AUTO", "BATCH_DOT4", "BATCH_MFMA", "prof_enable", "prof_reset", "prof_read", "synth_q4k", "synth_q6k", "synth_normal", "FdmError",
    "QK_K", "Q4K_BLOCK_SIZE", "Q6K_BLOCK_SIZE", "HIDDEN", "MOE_FFN", "N_EXPERTS", "MAX_K",
    "MAX_LAYERS", "MAX_TOKENS", "EXPERT_Q4K_BYTES", "EXPERT_Q6K_BYTES",
]

call = _lib.call
lib = _lib.lib


def _p(t):
    """Device address of a tensor (or None / an int address)."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream=None):
    if stream is not None:
        return stream if isinstance(stream, int) else stream.cuda_stream
    import torch
    return torch.cuda.current_stream().cuda_stream


# ---- lifecycle -----------------------------------------------------------------
def init(device=0):
    """Select the device and allocate the workspace (metal_init).  Raises
    FdmError when no gfx950 device is usable."""
    call("fdm_init", int(device))


def shutdown():
    call("fdm_shutdown")


def sync(stream=None):
    """Wait for the stream's work and report what the kernels could only
    record: raises FdmError (FDM_E_STATE) when a wait inside an earlier
    moe_layer launch gave up, i.e. that call's result is not valid."""
    call("fdm_stream_sync", _stream(stream))


def stream_release(stream):
    """Free the workspace the library holds for `stream` (made at the stream's
    first call; each stream has its own, so host threads on their own streams
    may call concurrently).  No effect on the null stream's."""
    call("fdm_stream_release", _stream(stream))


def set_layer_spin_limit(polls):
    """Polls one wait inside moe_layer's kernel makes before giving up (0:
    the default).  Returns the previous limit."""
    prev = ctypes.c_uint32(0)
    call("fdm_set_layer_spin_limit", polls, ctypes.byref(prev))
    return prev.value


def available():
    """1 when initialised, 0 otherwise (metal_init's return convention)."""
    return lib.fdm_available()


# ---- quant.h twins ---------------------------------------------------------------
def fp16_to_fp32(src, dst, n=None, stream=None):
    n = src.numel() if n is None else n
    call("fdm_fp16_to_fp32", _p(src), _p(dst), n, _stream(stream))


def dequantize_row_q4_K(src, dst, n, stream=None):
    """quant.c:36-61 on the device: n weights (multiple of 256)."""
    call("fdm_dequant_q4k", _p(src), _p(dst), n, _stream(stream))


def dequantize_row_q6_K(src, dst, n, stream=None):
    """quant.c:63-92 on the device."""
    call("fdm_dequant_q6k", _p(src), _p(dst), n, _stream(stream))


# ---- matvec / expert -------------------------------------------------------------
def matvec_q4k(W, x, y, out_dim, in_dim, stream=None):
    call("fdm_matvec_q4k", _p(W), _p(x), _p(y), out_dim, in_dim, _stream(stream))


def matvec_q6k(W, x, y, out_dim, in_dim, stream=None):
    call("fdm_matvec_q6k", _p(W), _p(x), _p(y), out_dim, in_dim, _stream(stream))


def expert_ffn(blob, expert_size, x, out, act=None, stream=None):
    call("fdm_expert_ffn", _p(blob), expert_size, _p(x), _p(out), _p(act), _stream(stream))


# ---- router ----------------------------------------------------------------------
def router_logits(Wg, x, logits, T=1, stream=None):
    n_exp, dim = Wg.shape
    call("fdm_router_logits", _p(Wg), _p(x), n_exp, dim, T, _p(logits), _stream(stream))


def route(logits, bias, K, idx, w, T=1, stream=None):
    call("fdm_route", _p(logits), _p(bias), T, K, _p(idx), _p(w), _stream(stream))


# ---- resident layers ---------------------------------------------------------------
def attach_layer(L, experts, expert_size, Wg, bias, shared=None, n_experts=N_EXPERTS):
    """Register device-resident buffers as layer L (caller keeps ownership)."""
    call("fdm_layer_attach", L, _p(experts), expert_size, n_experts, _p(Wg), _p(bias),
         _p(shared))


def upload_layer(L, experts_host, expert_size, Wg_host, bias_host, shared_host=None,
                 n_experts=N_EXPERTS):
    """Copy host arrays (numpy) to HBM as layer L (library-owned)."""
    def hp(a):
        return None if a is None else a.ctypes.data
    call("fdm_layer_upload", L, hp(experts_host), expert_size, n_experts, hp(Wg_host),
         hp(bias_host), hp(shared_host))


def release_layer(L):
    call("fdm_layer_release", L)


def layer_info(L):
    es, q6, ne = ctypes.c_size_t(), ctypes.c_int(), ctypes.c_int()
    call("fdm_layer_query", L, ctypes.byref(es), ctypes.byref(q6), ctypes.byref(ne))
    return es.value, bool(q6.value), ne.value


# ---- MoE ---------------------------------------------------------------------------
def moe_forward(L, h_post, exp_idx, exp_w, K, moe_out, stream=None):
    """metal_moe_forward with device tensors: moe_out = sum_k w_k E_k(h_post)."""
    call("fdm_moe_forward", L, _p(h_post), _p(exp_idx), _p(exp_w), K, _p(moe_out),
         _stream(stream))


def moe_forward_host(L, h_post, exp_idx, exp_w, K, moe_out):
    """metal_moe_forward's exact convention: numpy host arrays, synchronous."""
    call("fdm_moe_forward_host", L, h_post.ctypes.data, exp_idx.ctypes.data,
         exp_w.ctypes.data, K, moe_out.ctypes.data)


BATCH_AUTO, BATCH_DOT4, BATCH_MFMA = 0, 1, 2
BATCH_MFMA_MIN_T = 12
NOALLOC_MAX_T = 32  # FDM_NOALLOC_MAX_T
NOALLOC_MAX_PAIRS = 256  # FDM_NOALLOC_MAX_PAIRS


def set_batch_kernel(mode):
    """Expert kernels behind moe_forward_batched: BATCH_DOT4 (per-token int8
    digit dot products), BATCH_MFMA (grouped GEMMs on MFMA, three fp16 planes
    of the activations) or BATCH_AUTO (MFMA from BATCH_MFMA_MIN_T tokens).
    Returns the previous mode."""
    prev = ctypes.c_int(-1)
    call("fdm_set_batch_kernel", mode, ctypes.byref(prev))
    return prev.value


def moe_layer(L, h_post, h_in, K, hidden, idx=None, w=None, stream=None):
    """MoE branch of layer_forward: hidden = h_in + routed + shared."""
    call("fdm_moe_layer", L, _p(h_post), _p(h_in), K, _p(hidden), _p(idx), _p(w),
         _stream(stream))


def moe_layer_norm(L, h, norm_w, K, hidden, h_post=None, idx=None, w=None, stream=None):
    """The MoE branch with its rms_norm fused in: hidden = h + routed(h_post)
    + shared(h_post), h_post = rms_norm(h, norm_w) (written to h_post if
    given).  hidden may be h itself."""
    call("fdm_moe_layer_norm", L, _p(h), _p(norm_w), K, _p(hidden), _p(h_post), _p(idx), _p(w),
         _stream(stream))


def layer_read_ceiling(L, idx, K, h_post, h_in, sink, stream=None):
    """Measurement only: read exactly the bytes one moe_layer launch on layer
    L reads (router, the K routed experts idx (device int32), the shared
    expert, h_post, h_in) with the layer kernel's load policy, and nothing
    else; sink (7168 int32/uint32) receives words whose sum (mod 2^32) is the
    sum of every byte read."""
    call("fdm_layer_read_ceiling", L, _p(idx), K, _p(h_post), _p(h_in), _p(sink), _stream(stream))


def moe_forward_batched(L, X, H_in, T, K, hidden, idx=None, w=None, n_distinct=None,
                        stream=None):
    """T tokens through the MoE branch of layer L in one step, each selected
    expert's weights read once: hidden[t] = H_in[t] + routed + shared."""
    call("fdm_moe_forward_batched", L, _p(X), _p(H_in), T, K, _p(hidden), _p(idx), _p(w),
         _p(n_distinct), _stream(stream))


def moe_forward_batched_noalloc(L, X, H_in, T, K, hidden, idx=None, w=None, n_distinct=None,
                                stream=None):
    """moe_forward_batched on the library's fixed device scratch: allocates
    nothing (T <= NOALLOC_MAX_T, T*K <= NOALLOC_MAX_PAIRS).  Calls that
    overlap on one device share that scratch and race."""
    call("fdm_moe_forward_batched_noalloc", L, _p(X), _p(H_in), T, K, _p(hidden), _p(idx), _p(w),
         _p(n_distinct), _stream(stream))


def rms_norm(x, w, out, T, d=HIDDEN, stream=None):
    """out[t] = rms_norm(x[t], w) on the device (infer.m:369-374), bit-exact."""
    call("fdm_rms_norm", _p(x), _p(w), _p(out), T, d, _stream(stream))


def moe_prefill(layers, H, T, K, norm_w, idx=None, stream=None):
    """In place on H [T][7168]: for each layer l, H += MoE_l(rms_norm(H, norm_w[l]))."""
    n = len(layers)
    lay = (ctypes.c_int * n)(*layers)
    nw = (ctypes.c_void_p * n)(*[_p(w) for w in norm_w]) if norm_w is not None else None
    call("fdm_moe_prefill", ctypes.cast(lay, ctypes.c_void_p),  n, _p(H), T, K,
         ctypes.cast(nw, ctypes.c_void_p) if nw is not None else None, _p(idx), _stream(stream))


# ---- streamed layers (experts read from the packed layer file on demand) --------------
def stream_layer(L, layer_file, expert_size, Wg, bias, shared=None, n_cache=N_EXPERTS, n_threads=0,
                 n_experts=N_EXPERTS):
    """Open layer L as a streamed layer: routed experts stay in layer_file
    (repack_experts.c layout) and are read into an HBM cache of n_cache
    slots on demand; Wg / bias stay caller-owned device tensors."""
    call("fdm_layer_stream_open", L, str(layer_file).encode(), expert_size, n_experts, _p(Wg), _p(bias),
         _p(shared), n_cache, n_threads)


def moe_layer_streamed(L, h_post, h_in, K, hidden, idx=None, w=None, stream=None):
    """moe_layer for a streamed layer (reads the routed experts it lacks)."""
    call("fdm_moe_layer_streamed", L, _p(h_post), _p(h_in), K, _p(hidden), _p(idx), _p(w), _stream(stream))


def stream_stats(L):
    """(hits, misses, bytes read) of a streamed layer since it was opened."""
    h, m, b = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
    call("fdm_stream_stats", L, ctypes.byref(h), ctypes.byref(m), ctypes.byref(b))
    return h.value, m.value, b.value


# ---- MLA attention (mla_forward) ------------------------------------------------------
ATTN_FIELDS = ("attn_norm", "q_a", "q_a_norm", "q_b", "kv_a", "kv_a_norm", "k_b", "v_b", "o_proj")


def attn_upload(L, weights, max_seq=_lib.ATTN_MAX_SEQ):
    """Copy one layer's attention weights to HBM: weights maps the
    fdm_attn_weights field names to contiguous host arrays (norms float32,
    matrices F16 as uint16 or float16) in LayerAttnDense's layout."""
    w = _lib.AttnWeights(*[weights[n].ctypes.data for n in ATTN_FIELDS])
    call("fdm_attn_upload", L, ctypes.byref(w), max_seq)


def attn_load_gguf(L, gguf, max_seq=_lib.ATTN_MAX_SEQ):
    """One layer's attention weights from an open GGUF (see gguf.GGUF),
    converted as load_layer_weights does."""
    call("fdm_attn_load_gguf", L, gguf.handle, max_seq)


def attn_forward(L, hidden, pos, stream=None):
    """hidden += W_o . MLA(rms_norm(hidden), pos), appending to the layer's KV cache."""
    call("fdm_attn_forward", L, _p(hidden), pos, _stream(stream))


def attn_reset(L):
    call("fdm_attn_reset", L)


def attn_len(L):
    n = ctypes.c_int()
    call("fdm_attn_len", L, ctypes.byref(n))
    return n.value


def attn_release(L):
    call("fdm_attn_release", L)


# ---- dense FFN layers (layer_forward's branch for L < 3) ------------------------------
def f32_to_f16(src, dst, n=None, stream=None):
    """(__fp16) cast of f32_to_f16_alloc on the device: fp32 -> F16 bits."""
    n = src.numel() if n is None else n
    call("fdm_f32_to_f16", _p(src), _p(dst), n, _stream(stream))


def upload_dense(L, gate, up, down):
    """Copy F16 weights (numpy uint16 or float16 arrays on the host; gate and
    up [inter][7168], down [7168][inter]) to HBM as dense layer L."""
    inter = gate.shape[0]
    call("fdm_dense_upload", L, gate.ctypes.data, up.ctypes.data, down.ctypes.data, inter)


def attach_dense(L, gate, up, down, inter):
    """Copy F16 weights from device memory (the library keeps its own copy)."""
    call("fdm_dense_attach", L, _p(gate), _p(up), _p(down), inter)


def load_dense_gguf(L, gguf):
    """blk.L.ffn_{gate,up,down}.weight of an open GGUF (see gguf.GGUF),
    converted to F16 as dequant_tensor_f16.  Returns the intermediate size."""
    inter = ctypes.c_int()
    call("fdm_dense_load_gguf", L, gguf.handle, ctypes.byref(inter))
    return inter.value


def release_dense(L):
    call("fdm_dense_release", L)


def dense_info(L):
    inter = ctypes.c_int()
    call("fdm_dense_query", L, ctypes.byref(inter))
    return inter.value


def dense_ffn(L, h_post, h_in, hidden, stream=None):
    """hidden = h_in + W_down . (silu(W_gate . h_post) * (W_up . h_post))."""
    call("fdm_dense_ffn", L, _p(h_post), _p(h_in), _p(hidden), _stream(stream))


# ---- per-kernel GPU timing (HIP events; the moe_prof_t counterpart) --------------------
PHASES = {"router": _lib.PROF_ROUTER, "gateup": _lib.PROF_GATEUP, "down": _lib.PROF_DOWN,
          "xdigits": _lib.PROF_XDIGITS, "matvec": _lib.PROF_MATVEC, "layer": _lib.PROF_LAYER,
          "batch": _lib.PROF_BATCH, "prefill": _lib.PROF_PREFILL, "dense": _lib.PROF_DENSE,
          "attn": _lib.PROF_ATTN, "ceiling": _lib.PROF_CEILING}


def prof_enable(on=True):
    call("fdm_prof_enable", 1 if on else 0)


def prof_reset():
    call("fdm_prof_reset")


def prof_read(phase):
    """(count, total_ms, min_ms, max_ms) of one phase since the last reset."""
    n, tot, mn, mx = ctypes.c_int(), ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
    call("fdm_prof_read", PHASES.get(phase, phase), ctypes.byref(n), ctypes.byref(tot),
         ctypes.byref(mn), ctypes.byref(mx))
    return n.value, tot.value, mn.value, mx.value


# ---- synthetic data ------------------------------------------------------------------
def synth_q4k(dst, n_blocks, seed, stream=None):
    call("fdm_synth_q4k", _p(dst), n_blocks, seed, _stream(stream))


def synth_q6k(dst, n_blocks, seed, stream=None):
    call("fdm_synth_q6k", _p(dst), n_blocks, seed, _stream(stream))


def synth_normal(dst, n, mean, std, seed, stream=None):
    call("fdm_synth_normal", _p(dst), n, mean, std, seed, _stream(stream))
