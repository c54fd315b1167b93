"""Minimal GGUF v2/v3 writer for the ingest tests, written from the public
format description: "GGUF", u32 version, u64 tensor count, u64 metadata
count, metadata (string key, u32 type, value), tensor infos (string name,
u32 n_dims, u64 dims, u32 ggml type, u64 offset from the data section),
data section aligned to general.alignment (32 by default).  Tensor payloads
may be left out (None): the file is then extended without writing them, so
large layers stay sparse on disk."""
import struct

UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALAR = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i",
           FLOAT32: "<f", BOOL: "<B", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}
# ggml block geometry (elements, bytes) for the types the tests use
GEOM = {0: (1, 4), 1: (1, 2), 12: (256, 144), 14: (256, 210), 30: (1, 2), 8: (32, 34)}
F32, F16, Q4_K, Q6_K, BF16 = 0, 1, 12, 14, 30


def _str(s):
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STRING:
        return _str(v)
    if t == ARRAY:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        for x in items:
            out += _value(et, x)
        return out
    return struct.pack(_SCALAR[t], v)


def nbytes(ggml_type, dims):
    blck, size = GEOM[ggml_type]
    n = 1
    for d in dims:
        n *= d
    assert n % blck == 0
    return n // blck * size


def write_gguf(path, kvs=(), tensors=(), version=3, magic=b"GGUF", alignment=None,
               n_dims_override=None, tensor_type_override=None, offset_override=None,
               truncate_to=None):
    """kvs: [(key, type, value)] (arrays: value = (elem_type, [items]));
    tensors: [(name, ggml_type, dims, payload bytes or None)].
    Returns {name: (absolute data offset, nbytes)}."""
    kvs = list(kvs)
    if alignment is not None:
        kvs.append(("general.alignment", UINT32, alignment))
    align = alignment or 32
    head = magic + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for key, t, v in kvs:
        head += _str(key) + struct.pack("<I", t) + _value(t, v)
    rel, rels = 0, []
    for name, gt, dims, _ in tensors:
        rels.append(rel)
        rel += nbytes(gt, dims)
        rel = (rel + align - 1) // align * align
    for i, (name, gt, dims, _) in enumerate(tensors):
        nd = len(dims) if n_dims_override is None else n_dims_override
        head += _str(name) + struct.pack("<I", nd)
        for d in list(dims)[:max(nd, 0)]:
            head += struct.pack("<Q", d)
        t = gt if tensor_type_override is None else tensor_type_override
        off = rels[i] if offset_override is None else offset_override
        head += struct.pack("<IQ", t, off)
    data_start = (len(head) + align - 1) // align * align
    out = {}
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * (data_start - len(head)))
        end = data_start
        for i, (name, gt, dims, payload) in enumerate(tensors):
            n = nbytes(gt, dims)
            out[name] = (data_start + rels[i], n)
            if payload is not None:
                assert len(payload) == n
                f.seek(data_start + rels[i])
                f.write(payload)
            end = max(end, data_start + rels[i] + n)
        f.truncate(end if truncate_to is None else truncate_to)
    return out


def write_slices(path, offset, pieces):
    """Write (relative offset, bytes) pieces into an existing file at offset."""
    with open(path, "r+b") as f:
        for rel, b in pieces:
            f.seek(offset + rel)
            f.write(b)
