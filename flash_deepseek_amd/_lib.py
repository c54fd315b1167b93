"""ctypes binding of libfdm.so, the C ABI declared in include/fdm.h.

Loading fails loudly when the library has not been built: there is no CPU
fallback for any entry point.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfdm.so")

FDM_OK = 0
FDM_E_INVAL = -1
FDM_E_NODEV = -2
FDM_E_HIP = -3
FDM_E_STATE = -4
FDM_E_NOMEM = -5
FDM_E_SIZE = -6
FDM_E_IO = -7
FDM_E_FORMAT = -8

(PROF_ROUTER, PROF_GATEUP, PROF_DOWN, PROF_XDIGITS, PROF_MATVEC, PROF_LAYER, PROF_BATCH,
 PROF_PREFILL, PROF_DENSE, PROF_ATTN, PROF_CEILING) = range(11)

QK_K = 256
Q4K_BLOCK_SIZE = 144
Q6K_BLOCK_SIZE = 210
HIDDEN = 7168
MOE_FFN = 2048
N_EXPERTS = 256
MAX_K = 16
MAX_LAYERS = 61
MAX_TOKENS = 512
DENSE_FFN = 18432
ATTN_MAX_SEQ = 16384


class AttnWeights(ctypes.Structure):
    """struct fdm_attn_weights (host pointers)."""
    _fields_ = [(n, ctypes.c_void_p) for n in
                ("attn_norm", "q_a", "q_a_norm", "q_b", "kv_a", "kv_a_norm", "k_b", "v_b", "o_proj")]
EXPERT_Q4K_BYTES = 24772608
EXPERT_Q6K_BYTES = 28557312

_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t
_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64
_f = ctypes.c_float

# name -> argtypes (all functions return int unless listed in _RESTYPES)
SIGNATURES = {
    "fdm_init": [_i],
    "fdm_shutdown": [],
    "fdm_available": [],
    "fdm_strerror": [_i],
    "fdm_last_error": [],
    "fdm_device_cus": [],
    "fdm_set_batch_kernel": [_i, ctypes.POINTER(ctypes.c_int)],
    "fdm_set_layer_spin_limit": [_u32, ctypes.POINTER(_u32)],
    "fdm_malloc": [ctypes.POINTER(_vp), _sz],
    "fdm_free": [_vp],
    "fdm_memcpy_h2d": [_vp, _vp, _sz, _vp],
    "fdm_memcpy_d2h": [_vp, _vp, _sz, _vp],
    "fdm_stream_sync": [_vp],
    "fdm_stream_release": [_vp],
    "fdm_fp16_to_fp32": [_vp, _vp, _sz, _vp],
    "fdm_f32_to_f16": [_vp, _vp, _sz, _vp],
    "fdm_dense_upload": [_i, _vp, _vp, _vp, _i],
    "fdm_dense_attach": [_i, _vp, _vp, _vp, _i],
    "fdm_dense_load_gguf": [_i, _vp, ctypes.POINTER(_i)],
    "fdm_dense_release": [_i],
    "fdm_dense_query": [_i, ctypes.POINTER(_i)],
    "fdm_dense_ffn": [_i, _vp, _vp, _vp, _vp],
    "fdm_layer_stream_open": [_i, ctypes.c_char_p, _sz, _i, _vp, _vp, _vp, _i, _i],
    "fdm_moe_layer_streamed": [_i, _vp, _vp, _i, _vp, _vp, _vp, _vp],
    "fdm_stream_stats": [_i, ctypes.POINTER(_u64), ctypes.POINTER(_u64), ctypes.POINTER(_u64)],
    "fdm_attn_upload": [_i, ctypes.POINTER(AttnWeights), _i],
    "fdm_attn_forward": [_i, _vp, _i, _vp],
    "fdm_attn_load_gguf": [_i, _vp, _i],
    "fdm_attn_reset": [_i],
    "fdm_attn_len": [_i, ctypes.POINTER(_i)],
    "fdm_attn_release": [_i],
    "fdm_dequant_q4k": [_vp, _vp, _sz, _vp],
    "fdm_dequant_q6k": [_vp, _vp, _sz, _vp],
    "fdm_matvec_q4k": [_vp, _vp, _vp, _u32, _u32, _vp],
    "fdm_matvec_q6k": [_vp, _vp, _vp, _u32, _u32, _vp],
    "fdm_expert_ffn": [_vp, _sz, _vp, _vp, _vp, _vp],
    "fdm_router_logits": [_vp, _vp, _i, _i, _i, _vp, _vp],
    "fdm_route": [_vp, _vp, _i, _i, _vp, _vp, _vp],
    "fdm_layer_attach": [_i, _vp, _sz, _i, _vp, _vp, _vp],
    "fdm_layer_upload": [_i, _vp, _sz, _i, _vp, _vp, _vp],
    "fdm_layer_release": [_i],
    "fdm_layer_query": [_i, ctypes.POINTER(_sz), ctypes.POINTER(_i), ctypes.POINTER(_i)],
    "fdm_moe_forward": [_i, _vp, _vp, _vp, _i, _vp, _vp],
    "fdm_moe_forward_host": [_i, _vp, _vp, _vp, _i, _vp],
    "fdm_moe_layer": [_i, _vp, _vp, _i, _vp, _vp, _vp, _vp],
    "fdm_moe_layer_norm": [_i, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp],
    "fdm_layer_read_ceiling": [_i, _vp, _i, _vp, _vp, _vp, _vp],
    "fdm_moe_forward_batched": [_i, _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp],
    "fdm_moe_forward_batched_noalloc": [_i, _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp],
    "fdm_rms_norm": [_vp, _vp, _vp, _i, _i, _vp],
    "fdm_moe_prefill": [_vp, _i, _vp, _i, _i, _vp, _vp, _vp],
    "fdm_prof_enable": [_i],
    "fdm_prof_reset": [],
    "fdm_prof_read": [_i, ctypes.POINTER(_i), ctypes.POINTER(ctypes.c_double),
                      ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)],
    "fdm_synth_q4k": [_vp, _sz, _u64, _vp],
    "fdm_synth_q6k": [_vp, _sz, _u64, _vp],
    "fdm_synth_normal": [_vp, _sz, _f, _f, _u64, _vp],
    "fdm_gguf_open": [ctypes.POINTER(ctypes.c_char_p), _i, ctypes.POINTER(_vp)],
    "fdm_gguf_close": [_vp],
    "fdm_gguf_count": [_vp, ctypes.POINTER(_i), ctypes.POINTER(_u64)],
    "fdm_gguf_shard_info": [_vp, _i, ctypes.POINTER(_u32), ctypes.POINTER(_u64),
                            ctypes.POINTER(_u64), ctypes.POINTER(_u64), ctypes.POINTER(_u64)],
    "fdm_gguf_find": [_vp, ctypes.c_char_p, _vp],
    "fdm_gguf_tensor_at": [_vp, _u64, ctypes.c_char_p, _sz, _vp],
    "fdm_gguf_find_kv": [_vp, _i, ctypes.c_char_p, ctypes.POINTER(_i), ctypes.POINTER(_i),
                         ctypes.POINTER(_u64)],
    "fdm_gguf_kv_int": [_vp, _i, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64)],
    "fdm_gguf_kv_float": [_vp, _i, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)],
    "fdm_gguf_kv_str": [_vp, _i, ctypes.c_char_p, ctypes.c_char_p, _sz],
    "fdm_gguf_read": [_vp, ctypes.c_char_p, _vp, _u64, _u64],
    "fdm_ggml_type_geometry": [_i, ctypes.POINTER(_u64), ctypes.POINTER(_u64)],
    "fdm_layer_load_gguf": [_i, _vp, _i, ctypes.POINTER(_i)],
    "fdm_layer_load_packed": [_i, ctypes.c_char_p, _vp, _i, ctypes.POINTER(_i)],
}
_RESTYPES = {"fdm_strerror": ctypes.c_char_p, "fdm_last_error": ctypes.c_char_p}


class FdmError(RuntimeError):
    def __init__(self, code, fn, detail):
        self.code = code
        super().__init__(f"{fn} failed ({code}): {detail}")


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m flash_deepseek_amd.build` "
            "(hipcc, gfx950). There is no CPU fallback.")
    lib = ctypes.CDLL(LIB_PATH)
    for name, args in SIGNATURES.items():
        try:
            fn = getattr(lib, name)
        except AttributeError as e:
            raise ImportError(f"{LIB_PATH} lacks {name}: it is stale, rebuild it with "
                              "`python -m flash_deepseek_amd.build`") from e
        fn.argtypes = args
        fn.restype = _RESTYPES.get(name, _i)
    return lib


class _LazyLib:
    """Loads libfdm.so on first use, so the package (and its build module)
    can be imported before the library exists."""

    _handle = None

    def __getattr__(self, name):
        if _LazyLib._handle is None:
            _LazyLib._handle = _load()
        return getattr(_LazyLib._handle, name)


lib = _LazyLib()


def check(rc, fn="fdm call"):
    if rc != FDM_OK:
        detail = lib.fdm_last_error().decode(errors="replace")
        raise FdmError(rc, fn, detail or lib.fdm_strerror(rc).decode())
    return rc


def call(name, *args):
    """Call an fdm_* entry point and raise FdmError on a non-zero code."""
    return check(getattr(lib, name)(*args), name)
