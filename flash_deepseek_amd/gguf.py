"""Python mirror of the library's GGUF ingest (include/fdm.h, "real-weight
ingest"): the manifest of gguf.h:163-192 (open, find, metadata, ranged
reads) and the layer loaders that replace repack_experts.c and the MoE part
of load_layer_weights (infer.m:1794-1823).  Every call goes through
libfdm.so; nothing is parsed in Python."""
import ctypes
import os

import numpy as np

from . import _lib
from ._lib import FDM_E_STATE, FdmError, call, check, lib

# ggml type ids used by the MoE path, and the GGUF metadata value types
GGML_F32, GGML_F16, GGML_Q4_K, GGML_Q6_K, GGML_BF16 = 0, 1, 12, 14, 30
(GGUF_UINT8, GGUF_INT8, GGUF_UINT16, GGUF_INT16, GGUF_UINT32, GGUF_INT32, GGUF_FLOAT32,
 GGUF_BOOL, GGUF_STRING, GGUF_ARRAY, GGUF_UINT64, GGUF_INT64, GGUF_FLOAT64) = range(13)


class TensorInfo(ctypes.Structure):
    """fdm_gguf_tensor_info: type, n_dims, dims (ne[0] innermost), nbytes,
    absolute offset in its shard, shard index."""
    _fields_ = [("type", ctypes.c_int), ("n_dims", ctypes.c_int),
                ("dims", ctypes.c_uint64 * 4), ("nbytes", ctypes.c_uint64),
                ("offset", ctypes.c_uint64), ("shard", ctypes.c_int)]

    @property
    def shape(self):
        return tuple(int(d) for d in self.dims[: self.n_dims])


def type_geometry(ggml_type):
    """(elements, bytes) per block of a ggml type (ggml_blck_size / ggml_type_size)."""
    e, b = ctypes.c_uint64(), ctypes.c_uint64()
    call("fdm_ggml_type_geometry", ggml_type, ctypes.byref(e), ctypes.byref(b))
    return e.value, b.value


class GGUF:
    """A multi-shard GGUF manifest (gguf_load_manifest)."""

    def __init__(self, paths):
        if isinstance(paths, (str, bytes, os.PathLike)):
            paths = [paths]
        arr = (ctypes.c_char_p * len(paths))(*[str(p).encode() for p in paths])
        h = ctypes.c_void_p()
        call("fdm_gguf_open", arr, len(paths), ctypes.byref(h))
        self._h = h

    @property
    def handle(self):
        return self._h

    def close(self):
        if self._h:
            lib.fdm_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def counts(self):
        n, t = ctypes.c_int(), ctypes.c_uint64()
        call("fdm_gguf_count", self._h, ctypes.byref(n), ctypes.byref(t))
        return n.value, t.value

    def shard_info(self, shard):
        v, a, d = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64()
        k, t = ctypes.c_uint64(), ctypes.c_uint64()
        call("fdm_gguf_shard_info", self._h, shard, ctypes.byref(v), ctypes.byref(a),
             ctypes.byref(d), ctypes.byref(k), ctypes.byref(t))
        return {"version": v.value, "alignment": a.value, "data_start": d.value,
                "n_kv": k.value, "n_tensors": t.value}

    def find(self, name):
        """TensorInfo of a tensor, or None (gguf_find)."""
        info = TensorInfo()
        rc = lib.fdm_gguf_find(self._h, name.encode(), ctypes.byref(info))
        if rc == FDM_E_STATE:
            return None
        check(rc, "fdm_gguf_find")
        return info

    def tensors(self):
        """[(name, TensorInfo)] in shard order, then file order."""
        out = []
        for i in range(self.counts()[1]):
            buf = ctypes.create_string_buffer(4096)
            info = TensorInfo()
            call("fdm_gguf_tensor_at", self._h, i, buf, 4096, ctypes.byref(info))
            out.append((buf.value.decode(), info))
        return out

    def kv_type(self, key, shard=0):
        """(value type, array element type or -1, array length) or None."""
        t, at, n = ctypes.c_int(), ctypes.c_int(), ctypes.c_uint64()
        rc = lib.fdm_gguf_find_kv(self._h, shard, key.encode(), ctypes.byref(t),
                                  ctypes.byref(at), ctypes.byref(n))
        if rc == FDM_E_STATE:
            return None
        check(rc, "fdm_gguf_find_kv")
        return t.value, at.value, n.value

    def kv_int(self, key, shard=0):
        v = ctypes.c_int64()
        call("fdm_gguf_kv_int", self._h, shard, key.encode(), ctypes.byref(v))
        return v.value

    def kv_float(self, key, shard=0):
        v = ctypes.c_double()
        call("fdm_gguf_kv_float", self._h, shard, key.encode(), ctypes.byref(v))
        return v.value

    def kv_str(self, key, shard=0, cap=1 << 16):
        buf = ctypes.create_string_buffer(cap)
        call("fdm_gguf_kv_str", self._h, shard, key.encode(), buf, cap)
        return buf.value.decode()

    def read(self, name, n=None, rel=0):
        """n bytes of a tensor from `rel` on (gguf_tensor_pread), as uint8."""
        if n is None:
            info = self.find(name)
            if info is None:
                raise FdmError(FDM_E_STATE, "fdm_gguf_read", f"no tensor {name}")
            n = info.nbytes - rel
        out = np.empty(n, dtype=np.uint8)
        call("fdm_gguf_read", self._h, name.encode(), out.ctypes.data, n, rel)
        return out


def load_layer_gguf(L, gguf, with_shared=True):
    """Resident layer L straight from the GGUF's stacked expert tensors.
    Returns True when the layer's down matrices are Q6_K."""
    q6 = ctypes.c_int(-1)
    call("fdm_layer_load_gguf", L, gguf.handle, int(bool(with_shared)), ctypes.byref(q6))
    return bool(q6.value)


def load_layer_packed(L, layer_file, gguf, with_shared=True):
    """Resident layer L from a packed layer file (256 expert blobs, as
    repack_experts.c writes them), router, bias and shared expert from the
    GGUF.  Returns True when the down matrices are Q6_K."""
    q6 = ctypes.c_int(-1)
    call("fdm_layer_load_packed", L, str(layer_file).encode(), gguf.handle,
         int(bool(with_shared)), ctypes.byref(q6))
    return bool(q6.value)


__all__ = ["GGUF", "TensorInfo", "type_geometry", "load_layer_gguf", "load_layer_packed",
           "GGML_F32", "GGML_F16", "GGML_Q4_K", "GGML_Q6_K", "GGML_BF16"]
