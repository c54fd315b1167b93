"""ctypes binding of the C restatement (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, where it is the checker.  The shipped package
(flash_deepseek_amd) never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libquant_ref.so")
REF_DUMP = os.path.join(HERE, "_ref", "ref_dump")

HIDDEN, FFN, N_EXPERTS, MAX_K = 7168, 2048, 256, 16
Q4K_BLOCK, Q6K_BLOCK, QK_K = 144, 210, 256
GATE_BYTES = 57344 * Q4K_BLOCK
DOWN_Q4K_BYTES = 57344 * Q4K_BLOCK
DOWN_Q6K_BYTES = 57344 * Q6K_BLOCK
EXPERT_Q4K = 2 * GATE_BYTES + DOWN_Q4K_BYTES
EXPERT_Q6K = 2 * GATE_BYTES + DOWN_Q6K_BYTES

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_vp = ctypes.c_void_p


def build():
    """Compile liboracle.so (and _ref when the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    sig = {
        "orc_fp16_to_fp32": (ctypes.c_float, [ctypes.c_uint16]),
        "orc_fp16_to_fp32_array": (None, [_vp, _f32p, ctypes.c_size_t]),
        "orc_dequantize_row_q4_K": (None, [_vp, _f32p, ctypes.c_size_t]),
        "orc_dequantize_row_q6_K": (None, [_vp, _f32p, ctypes.c_size_t]),
        "orc_expf": (ctypes.c_float, [ctypes.c_float]),
        "orc_sigmoidf": (ctypes.c_float, [ctypes.c_float]),
        "orc_silu_mul": (None, [_f32p, _f32p, _f32p, ctypes.c_int]),
        "orc_rms_norm": (None, [_f32p, _vp, _f32p, ctypes.c_int]),
        "orc_matvec_q4k": (None, [_vp, _f32p, _f32p, ctypes.c_int, ctypes.c_int]),
        "orc_matvec_q6k": (None, [_vp, _f32p, _f32p, ctypes.c_int, ctypes.c_int]),
        "orc_matvec_q4k_f32": (None, [_vp, _f32p, _f32p, ctypes.c_int, ctypes.c_int]),
        "orc_matvec_q6k_f32": (None, [_vp, _f32p, _f32p, ctypes.c_int, ctypes.c_int]),
        "orc_expert_ffn": (None, [_vp, ctypes.c_int, _f32p, _f32p, _vp, _vp, _vp]),
        "orc_fp32_to_fp16": (ctypes.c_uint16, [ctypes.c_float]),
        "orc_fp32_to_fp16_array": (None, [_f32p, _vp, ctypes.c_size_t]),
        "orc_dense_ffn": (None, [_vp, _vp, _vp, ctypes.c_int, _f32p, _vp, _f32p, _vp]),
        "orc_yarn_freq": (None, [_f32p]),
        "orc_mla_scale": (ctypes.c_float, []),
        "orc_mla_forward": (None, [_vp] * 9 + [_f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int]),
        "orc_mla_append": (None, [_vp] * 3 + [_f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int]),
        "orc_router_logits": (None, [_f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int]),
        "orc_route_ex": (None, [_f32p, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                ctypes.c_int, ctypes.c_float, _i32p, _f32p]),
        "orc_moe_forward": (None, [_vp, ctypes.c_size_t, _f32p, _i32p, _f32p, ctypes.c_int,
                                   _f32p]),
        "orc_moe_layer": (None, [_vp, ctypes.c_size_t, _f32p, _f32p, _vp, _f32p, _vp,
                                 ctypes.c_int, _f32p, _i32p, _f32p, _f32p, _f32p]),
        "orc_rand_u64": (ctypes.c_uint64, [ctypes.c_uint64, ctypes.c_uint64]),
        "orc_synth_bytes": (None, [_u8p, ctypes.c_size_t, ctypes.c_uint64]),
        "orc_synth_normal": (None, [_f32p, ctypes.c_size_t, ctypes.c_float, ctypes.c_float,
                                    ctypes.c_uint64]),
        "orc_synth_q4k": (None, [_u8p, ctypes.c_size_t, ctypes.c_uint64]),
        "orc_synth_q6k": (None, [_u8p, ctypes.c_size_t, ctypes.c_uint64]),
        "orc_cpu_expert_baseline": (ctypes.c_double, [ctypes.POINTER(_vp), ctypes.c_int,
                                                      ctypes.c_int, _f32p, _f32p, _f32p,
                                                      ctypes.c_int, ctypes.c_int]),
        "orc_cpu_layer_baseline": (ctypes.c_double, [ctypes.POINTER(_vp), ctypes.c_int,
                                                     ctypes.c_int, _f32p, _f32p, _f32p, _f32p,
                                                     _f32p, ctypes.c_int]),
        "orc_cpu_layer_tuned": (ctypes.c_double, [ctypes.POINTER(_vp), ctypes.c_int, ctypes.c_int,
                                                  _f32p, _f32p, _f32p, _f32p, _f32p, ctypes.c_int,
                                                  ctypes.c_int, ctypes.POINTER(ctypes.c_int)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


L = _load()


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


# ---- quant codec ----------------------------------------------------------
def fp16_to_fp32(h):
    """Scalar conversion (returned as a Python float: NaNs come back quiet)."""
    return L.orc_fp16_to_fp32(int(h))


def fp16_to_fp32_array(bits):
    """Bit-exact conversion of an array of half bit patterns."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.size, dtype=np.float32)
    L.orc_fp16_to_fp32_array(_ptr(bits), out, bits.size)
    return out


def dequant_q4k(raw, n=None):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    n = n if n is not None else raw.size // Q4K_BLOCK * QK_K
    out = np.empty(n, dtype=np.float32)
    L.orc_dequantize_row_q4_K(_ptr(raw), out, n)
    return out


def dequant_q6k(raw, n=None):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    n = n if n is not None else raw.size // Q6K_BLOCK * QK_K
    out = np.empty(n, dtype=np.float32)
    L.orc_dequantize_row_q6_K(_ptr(raw), out, n)
    return out


# ---- dense helpers ----------------------------------------------------------
def expf(x):
    return L.orc_expf(float(x))


def sigmoidf(x):
    return L.orc_sigmoidf(float(x))


def rms_norm(x, w=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    o = np.empty_like(x)
    wp = None if w is None else _ptr(np.ascontiguousarray(w, dtype=np.float32))
    L.orc_rms_norm(x, wp, o, x.size)
    return o


def matvec(raw, x, rows, cols, qtype="q4k", f32=False):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, dtype=np.float32)
    fn = {("q4k", False): L.orc_matvec_q4k, ("q6k", False): L.orc_matvec_q6k,
          ("q4k", True): L.orc_matvec_q4k_f32, ("q6k", True): L.orc_matvec_q6k_f32}[(qtype, f32)]
    fn(_ptr(raw), x, y, rows, cols)
    return y


def expert_ffn(blob, down_is_q6, x, with_intermediates=False):
    blob = np.ascontiguousarray(blob, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(HIDDEN, dtype=np.float32)
    if with_intermediates:
        g, u, a = (np.empty(FFN, dtype=np.float32) for _ in range(3))
        L.orc_expert_ffn(_ptr(blob), int(down_is_q6), x, out, _ptr(g), _ptr(u), _ptr(a))
        return out, g, u, a
    L.orc_expert_ffn(_ptr(blob), int(down_is_q6), x, out, None, None, None)
    return out


def expert_ffn_f32(blob, down_is_q6, x):
    """expert_worker (infer.m:1069-1091) in the reference's own precision:
    fp32 dequant, fp32 dot products summed in index order, silu_mul in fp32
    (infer.m:378-383).  The yardstick for "fp32 grade" errors."""
    blob = np.ascontiguousarray(blob, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = matvec(blob[:GATE_BYTES], x, FFN, HIDDEN, "q4k", f32=True)
    u = matvec(blob[GATE_BYTES:2 * GATE_BYTES], x, FFN, HIDDEN, "q4k", f32=True)
    a = np.empty(FFN, dtype=np.float32)
    L.orc_silu_mul(g, u, a, FFN)
    return matvec(blob[2 * GATE_BYTES:], a, HIDDEN, FFN, "q6k" if down_is_q6 else "q4k", f32=True)


def fp32_to_fp16(x):
    """(__fp16)x elementwise (infer.m:521-528): uint16 bits."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    L.orc_fp32_to_fp16_array(x.ravel(), _ptr(out), x.size)
    return out


def dense_ffn(gate, up, down, h_post, h_in=None, with_act=False):
    """Dense branch of layer_forward (infer.m:1852-1868) on F16 bit arrays:
    gate, up [inter][7168], down [7168][inter]; float64 accumulation."""
    gate, up, down = (np.ascontiguousarray(a).view(np.uint16) for a in (gate, up, down))
    inter = gate.shape[0]
    assert gate.shape == (inter, HIDDEN) and up.shape == gate.shape and down.shape == (HIDDEN, inter)
    h_post = np.ascontiguousarray(h_post, dtype=np.float32)
    hp = None if h_in is None else _ptr(np.ascontiguousarray(h_in, dtype=np.float32))
    out = np.empty(HIDDEN, dtype=np.float32)
    act = np.empty(inter, dtype=np.float32) if with_act else None
    L.orc_dense_ffn(_ptr(gate), _ptr(up), _ptr(down), inter, h_post, hp, out,
                    None if act is None else _ptr(act))
    return (out, act) if with_act else out


ATTN_FIELDS = ("attn_norm", "q_a", "q_a_norm", "q_b", "kv_a", "kv_a_norm", "k_b", "v_b", "o_proj")


def yarn_freq():
    f = np.empty(32, dtype=np.float32)
    L.orc_yarn_freq(f)
    return f


def mla_scale():
    return L.orc_mla_scale()


class MlaCache:
    """The latent KV cache of one layer (c_kv [n][512], k_rope [n][64], fp32)."""

    def __init__(self, max_seq):
        self.c = np.zeros((max_seq, 512), np.float32)
        self.k = np.zeros((max_seq, 64), np.float32)
        self.len = 0


def mla_forward(w, hidden, cache, pos):
    """mla_forward (infer.m:766-903): returns the new hidden; appends to cache.
    w maps ATTN_FIELDS to arrays (norms float32, matrices F16 bits)."""
    h = np.ascontiguousarray(hidden, dtype=np.float32).copy()
    args = [_ptr(np.ascontiguousarray(w[n])) for n in ATTN_FIELDS]
    L.orc_mla_forward(*args, h, cache.c, cache.k, cache.len, pos)
    cache.len += 1
    return h


def mla_append(w, hidden, cache, pos):
    """Only the cache append of mla_forward (the token's c_kv and rotated
    k_rope as row cache.len), for filling long caches cheaply."""
    h = np.ascontiguousarray(hidden, dtype=np.float32)
    args = [_ptr(np.ascontiguousarray(w[n])) for n in ("attn_norm", "kv_a", "kv_a_norm")]
    L.orc_mla_append(*args, h, cache.c, cache.k, cache.len, pos)
    cache.len += 1


# ---- router -------------------------------------------------------------------
def router_logits(Wg, x):
    Wg = np.ascontiguousarray(Wg, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    n_exp, dim = Wg.shape
    out = np.empty(n_exp, dtype=np.float32)
    L.orc_router_logits(Wg, x, out, n_exp, dim)
    return out


def route(logits, bias, K=8, n_group=8, topk_group=4, scale=2.5):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    idx = np.empty(K, dtype=np.int32)
    w = np.empty(K, dtype=np.float32)
    bp = None if bias is None else _ptr(np.ascontiguousarray(bias, dtype=np.float32))
    L.orc_route_ex(logits, bp, logits.size, n_group, topk_group, K, scale, idx, w)
    return idx, w


# ---- MoE layer ----------------------------------------------------------------
def moe_forward(experts, expert_size, h_post, idx, w):
    h_post = np.ascontiguousarray(h_post, dtype=np.float32)
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty(HIDDEN, dtype=np.float32)
    L.orc_moe_forward(_ptr(experts), expert_size, h_post, idx, w, idx.size, out)
    return out


def moe_layer(experts, expert_size, Wg, bias, shared, h_post, h_in=None, K=8):
    """Returns (hidden_out, idx, w, moe_out, shared_out)."""
    Wg = np.ascontiguousarray(Wg, dtype=np.float32)
    bias = np.ascontiguousarray(bias, dtype=np.float32)
    h_post = np.ascontiguousarray(h_post, dtype=np.float32)
    hid = np.empty(HIDDEN, dtype=np.float32)
    moe = np.empty(HIDDEN, dtype=np.float32)
    sd = np.empty(HIDDEN, dtype=np.float32)
    idx = np.empty(K, dtype=np.int32)
    w = np.empty(K, dtype=np.float32)
    hin = None if h_in is None else _ptr(np.ascontiguousarray(h_in, dtype=np.float32))
    sh = None if shared is None else _ptr(shared)
    L.orc_moe_layer(_ptr(experts), expert_size, Wg, bias, sh, h_post, hin, K, hid, idx, w,
                    moe, sd)
    return hid, idx, w, moe, sd


# ---- synthetic data -----------------------------------------------------------
def rand_u64(seed, i):
    return L.orc_rand_u64(seed, i)


def synth_bytes(n, seed):
    out = np.empty(n, dtype=np.uint8)
    L.orc_synth_bytes(out, n, seed)
    return out


def synth_normal(n, mean, std, seed):
    out = np.empty(n, dtype=np.float32)
    L.orc_synth_normal(out, n, mean, std, seed)
    return out


def synth_q4k(n_blocks, seed):
    out = np.empty(n_blocks * Q4K_BLOCK, dtype=np.uint8)
    L.orc_synth_q4k(out, n_blocks, seed)
    return out


def synth_q6k(n_blocks, seed):
    out = np.empty(n_blocks * Q6K_BLOCK, dtype=np.uint8)
    L.orc_synth_q6k(out, n_blocks, seed)
    return out


def synth_expert(seed, down_is_q6=False):
    """One packed expert blob [gate | up | down] (infer.m:71-78 layout)."""
    g = synth_q4k(57344, seed * 3 + 1)
    u = synth_q4k(57344, seed * 3 + 2)
    d = synth_q6k(57344, seed * 3 + 3) if down_is_q6 else synth_q4k(57344, seed * 3 + 3)
    return np.concatenate([g, u, d])


def cpu_expert_baseline(blobs, down_is_q6, x, w, reps, n_threads=0):
    """Median microseconds of the reference-shaped CPU expert path."""
    arr = (ctypes.c_void_p * len(blobs))(*[b.ctypes.data for b in blobs])
    out = np.empty(HIDDEN, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    us = L.orc_cpu_expert_baseline(arr, len(blobs), int(down_is_q6), x, w, out, reps,
                                   n_threads)
    return us, out


def cpu_layer_baseline(blobs, down_is_q6, Wg, bias, x, h_in, reps):
    """Median microseconds per token of the reference-shaped CPU MoE layer
    (blobs: K routed experts then the shared one)."""
    arr = (ctypes.c_void_p * len(blobs))(*[b.ctypes.data for b in blobs])
    out = np.empty(HIDDEN, dtype=np.float32)
    us = L.orc_cpu_layer_baseline(arr, len(blobs) - 1, int(down_is_q6),
                                  np.ascontiguousarray(Wg, np.float32),
                                  np.ascontiguousarray(bias, np.float32),
                                  np.ascontiguousarray(x, np.float32),
                                  np.ascontiguousarray(h_in, np.float32), out, reps)
    return us, out


def cpu_layer_tuned(blobs, down_is_q6, Wg, bias, x, h_in, reps, n_threads=0):
    """Median microseconds per token of the tuned CPU MoE layer (fused
    row dequant-dot over every host core); returns (us, out, threads)."""
    arr = (ctypes.c_void_p * len(blobs))(*[b.ctypes.data for b in blobs])
    out = np.empty(HIDDEN, dtype=np.float32)
    used = ctypes.c_int(0)
    us = L.orc_cpu_layer_tuned(arr, len(blobs) - 1, int(down_is_q6),
                               np.ascontiguousarray(Wg, np.float32), np.ascontiguousarray(bias, np.float32),
                               np.ascontiguousarray(x, np.float32), np.ascontiguousarray(h_in, np.float32),
                               out, reps, n_threads, ctypes.byref(used))
    return us, out, used.value


# ---- the reference's own quant.c, compiled under _ref -------------------------
def load_ref():
    """ctypes handle of the reference quant.c built by `make ref`, or None."""
    if not os.path.exists(REF_PATH):
        return None
    lib = ctypes.CDLL(REF_PATH)
    lib.fp16_to_fp32.restype = ctypes.c_float
    lib.fp16_to_fp32.argtypes = [ctypes.c_uint16]
    lib.dequantize_row_q4_K.restype = None
    lib.dequantize_row_q4_K.argtypes = [_vp, _f32p, ctypes.c_size_t]
    lib.dequantize_row_q6_K.restype = None
    lib.dequantize_row_q6_K.argtypes = [_vp, _f32p, ctypes.c_size_t]
    return lib
