"""GGUF ingest on the host (no GPU): the library's reader (fdm_gguf_*)
against the reference's own gguf.c (compiled where it lies into
oracle/_ref/gguf_ref_dump by oracle/Makefile) on the same synthetic files,
written by tests/gguf_writer.py from the format description.  Without the
reference build the comparisons are skipped; the byte-level checks (reads
against the file, metadata values against what was written) still run."""
import os
import subprocess

import numpy as np
import pytest

from tests import gguf_writer as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.path.join(ROOT, "oracle", "_ref", "gguf_ref_dump")
have_ref = pytest.mark.skipif(not os.path.exists(REF), reason="reference gguf.c not built (oracle/_ref)")


@pytest.fixture(scope="module")
def G():
    from flash_deepseek_amd import gguf
    return gguf


def ref_dump(paths, timeout=20):
    r = subprocess.run([REF, *map(str, paths)], capture_output=True, text=True, timeout=timeout)
    return r.returncode, r.stdout.splitlines()


def ref_tensors(lines):
    out = []
    for ln in lines:
        f = ln.split()
        if f[0] == "tensor":
            nd = int(f[3])
            out.append((f[1], int(f[2]), nd, tuple(int(x) for x in f[4:4 + nd]), int(f[8]), int(f[9]),
                        int(f[10])))
    return out


def our_tensors(m):
    return [(n, i.type, i.n_dims, i.shape, i.nbytes, i.offset, i.shard) for n, i in m.tensors()]


KVS = [("general.architecture", W.STRING, "deepseek2"), ("k.u8", W.UINT8, 200), ("k.i8", W.INT8, -5),
       ("k.u16", W.UINT16, 60000), ("k.i16", W.INT16, -300), ("k.u32", W.UINT32, 4000000000),
       ("k.i32", W.INT32, -7), ("k.f32", W.FLOAT32, 1.5), ("k.bool", W.BOOL, 1),
       ("k.u64", W.UINT64, 2 ** 40 + 3), ("k.i64", W.INT64, -2 ** 40), ("k.f64", W.FLOAT64, 0.1),
       ("k.arr_i32", W.ARRAY, (W.INT32, [1, 2, 3])), ("k.arr_str", W.ARRAY, (W.STRING, ["a", "bc", ""])),
       ("k.arr_empty", W.ARRAY, (W.UINT8, []))]


def rich_tensors(seed=1, prefix=""):
    rng = np.random.default_rng(seed)
    spec = [(prefix + "w.f32", W.F32, (7, 3)), (prefix + "w.f16", W.F16, (16,)),
            (prefix + "blk.0.q4k", W.Q4_K, (512, 3)), (prefix + "blk.0.q6k", W.Q6_K, (256, 2, 2)),
            (prefix + "w.bf16", W.BF16, (4, 2, 3)), (prefix + "x.4d", W.F32, (2, 2, 2, 2))]
    return [(n, t, d, rng.integers(0, 256, W.nbytes(t, d), dtype=np.uint8).tobytes()) for n, t, d in spec]


def test_type_geometry(G):
    for t, (blck, size) in W.GEOM.items():
        assert G.type_geometry(t) == (blck, size)


@have_ref
def test_type_geometry_matches_reference(G):
    from flash_deepseek_amd._lib import FdmError
    f = subprocess.run([REF, "types"], capture_output=True, text=True, check=True).stdout.split()[1:]
    for i in range(0, len(f), 3):
        t, blck, size = int(f[i]), int(f[i + 1]), int(f[i + 2])
        if blck == 0:
            with pytest.raises(FdmError):
                G.type_geometry(t)
        else:
            assert G.type_geometry(t) == (blck, size), t


@pytest.mark.parametrize("version,alignment", [(3, None), (2, None), (3, 64), (3, 4096), (3, 8)])
def test_manifest_and_reads(G, tmp_path, version, alignment):
    path = tmp_path / "a.gguf"
    tens = rich_tensors()
    where = W.write_gguf(path, KVS, tens, version=version, alignment=alignment)
    raw = path.read_bytes()
    with G.GGUF([path]) as m:
        assert m.counts() == (1, len(tens))
        si = m.shard_info(0)
        assert si["version"] == version and si["alignment"] == (alignment or 32)
        assert si["n_kv"] == len(KVS) + (alignment is not None) and si["n_tensors"] == len(tens)
        for name, t, dims, payload in tens:
            info = m.find(name)
            assert info.type == t and info.shape == dims and info.shard == 0
            assert (info.offset, info.nbytes) == where[name]
            assert info.offset % (alignment or 32) == 0
            assert m.read(name).tobytes() == payload
            assert m.read(name, 5, 3).tobytes() == payload[3:8]
            assert raw[info.offset:info.offset + info.nbytes] == payload
        assert m.find("no.such.tensor") is None
        if os.path.exists(REF):
            rc, lines = ref_dump([path])
            assert rc == 0
            assert our_tensors(m) == ref_tensors(lines)
            shard = [ln.split() for ln in lines if ln.startswith("shard ")][0]
            assert [int(x) for x in shard[2:]] == [si["version"], si["alignment"], si["data_start"],
                                                   si["n_kv"], si["n_tensors"]]


def test_metadata_values(G, tmp_path):
    path = tmp_path / "kv.gguf"
    W.write_gguf(path, KVS, rich_tensors())
    with G.GGUF(path) as m:
        assert m.kv_str("general.architecture") == "deepseek2"
        for key, val in [("k.u8", 200), ("k.i8", -5), ("k.u16", 60000), ("k.i16", -300),
                         ("k.u32", 4000000000), ("k.i32", -7), ("k.bool", 1), ("k.u64", 2 ** 40 + 3),
                         ("k.i64", -2 ** 40)]:
            assert m.kv_int(key) == val, key
        assert m.kv_float("k.f32") == 1.5 and m.kv_float("k.f64") == 0.1
        assert m.kv_type("k.arr_i32") == (W.ARRAY, W.INT32, 3)
        assert m.kv_type("k.arr_str") == (W.ARRAY, W.STRING, 3)
        assert m.kv_type("k.arr_empty") == (W.ARRAY, W.UINT8, 0)
        assert m.kv_type("k.f32") == (W.FLOAT32, -1, 0)
        assert m.kv_type("no.such.key") is None
        if os.path.exists(REF):
            rc, lines = ref_dump([path])
            ref = {f[2]: f[3:] for f in (ln.split() for ln in lines if ln.startswith("kv "))}
            for key, t, _ in KVS:
                assert int(ref[key][0]) == t
            assert int(ref["k.u32"][1]) == m.kv_int("k.u32") and int(ref["k.i64"][1]) == m.kv_int("k.i64")
            assert ref["k.arr_str"][1:] == [str(W.STRING), "3"]


def test_read_bounds(G, tmp_path):
    from flash_deepseek_amd._lib import FDM_E_INVAL, FdmError
    path = tmp_path / "b.gguf"
    W.write_gguf(path, [], rich_tensors())
    with G.GGUF(path) as m:
        n = m.find("w.f32").nbytes
        assert len(m.read("w.f32", n, 0)) == n
        for cnt, rel in [(n + 1, 0), (1, n), (2, n - 1)]:
            with pytest.raises(FdmError) as e:
                m.read("w.f32", cnt, rel)
            assert e.value.code == FDM_E_INVAL


def test_multishard(G, tmp_path):
    a, b = tmp_path / "m-00001-of-00002.gguf", tmp_path / "m-00002-of-00002.gguf"
    ta, tb = rich_tensors(1, "a."), rich_tensors(2, "b.")
    W.write_gguf(a, KVS, ta)
    W.write_gguf(b, [("split.no", W.UINT16, 1)], tb, alignment=128)
    with G.GGUF([a, b]) as m:
        assert m.counts() == (2, len(ta) + len(tb))
        assert m.find("a.w.f32").shard == 0 and m.find("b.w.f32").shard == 1
        assert m.read("b.blk.0.q6k").tobytes() == tb[3][3]
        assert m.kv_int("split.no", shard=1) == 1 and m.kv_type("split.no", shard=0) is None
        if os.path.exists(REF):
            rc, lines = ref_dump([a, b])
            assert rc == 0 and our_tensors(m) == ref_tensors(lines)


def _malformed(tmp_path, case):
    p = tmp_path / f"{case}.gguf"
    t = [("t", W.F32, (100,), None)]
    if case == "magic":
        W.write_gguf(p, [], t, magic=b"GGUX")
    elif case == "version1":
        W.write_gguf(p, [], t, version=1)
    elif case == "version4":
        W.write_gguf(p, [], t, version=4)
    elif case == "dims0":
        W.write_gguf(p, [], t, n_dims_override=0)
    elif case == "dims5":
        W.write_gguf(p, [], [("t", W.F32, (2, 2, 2, 2, 2), None)])
    elif case == "not_whole_blocks":
        W.write_gguf(p, [], t, tensor_type_override=W.Q4_K)   # 100 elements of Q4_K
    elif case == "past_eof":
        W.write_gguf(p, [], t, truncate_to=None, offset_override=1 << 20)
    elif case == "unknown_type":
        W.write_gguf(p, [], t, tensor_type_override=4)        # an id ggml removed
    return [p]


@pytest.mark.parametrize("case", ["magic", "version1", "version4", "dims0", "dims5", "not_whole_blocks",
                                  "past_eof", "unknown_type"])
def test_malformed_rejected(G, tmp_path, case):
    from flash_deepseek_amd._lib import FDM_E_FORMAT, FdmError
    paths = _malformed(tmp_path, case)
    with pytest.raises(FdmError) as e:
        G.GGUF(paths)
    assert e.value.code == FDM_E_FORMAT
    if os.path.exists(REF):
        rc, lines = ref_dump(paths)
        assert rc == 1 and lines == ["error"]


def test_duplicate_across_shards(G, tmp_path):
    from flash_deepseek_amd._lib import FDM_E_FORMAT, FdmError
    a, b = tmp_path / "d1.gguf", tmp_path / "d2.gguf"
    W.write_gguf(a, [], rich_tensors(1))
    W.write_gguf(b, [], rich_tensors(2)[:2])
    with pytest.raises(FdmError) as e:
        G.GGUF([a, b])
    assert e.value.code == FDM_E_FORMAT
    if os.path.exists(REF):
        assert ref_dump([a, b])[0] == 1


@pytest.mark.parametrize("cut", [3, 20, 60, 200])
def test_truncated_header(G, tmp_path, cut):
    """A header cut short is an error.  (The reference's reader retries a
    short header buffer up to the file size and, once the buffer is the
    whole file, retries without end: it is not run on these files.)"""
    from flash_deepseek_amd._lib import FDM_E_FORMAT, FdmError
    p = tmp_path / "t.gguf"
    W.write_gguf(p, KVS, rich_tensors())
    with open(p, "r+b") as f:
        f.truncate(cut)
    with pytest.raises(FdmError) as e:
        G.GGUF(p)
    assert e.value.code == FDM_E_FORMAT


def test_missing_file(G, tmp_path):
    from flash_deepseek_amd._lib import FDM_E_IO, FdmError
    with pytest.raises(FdmError) as e:
        G.GGUF(tmp_path / "nope.gguf")
    assert e.value.code == FDM_E_IO
