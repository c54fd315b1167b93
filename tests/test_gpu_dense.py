"""Dense FFN layers (fdm_dense_*; the dense branch of layer_forward,
infer.m:1852-1868) against the oracle: outputs within 1e-3 relative L2 of
the float64 truth on the same F16 weights, the F16 conversion of the
weights (fdm_f32_to_f16 and the GGUF ingest, infer.m:314-355, 521-538) bit
for bit."""
import numpy as np
import pytest

from tests import gguf_writer as W
from tests._helpers import empty_f32, rel_l2, say, to_dev, to_host
from tests.test_oracle_dense import edge_floats

pytestmark = pytest.mark.gpu
TOL = 1e-3
H = 7168


def dense_weights(seed, inter):
    """Seeded F16 weights made on the device (torch), as host bit arrays
    and device tensors: gate, up [inter][7168], down [7168][inter]."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    mats = [(torch.randn((inter, H), generator=g, device="cuda") * H ** -0.5).half(),
            (torch.randn((inter, H), generator=g, device="cuda") * H ** -0.5).half(),
            (torch.randn((H, inter), generator=g, device="cuda") * inter ** -0.5).half()]
    host = [m.cpu().numpy().view(np.uint16) for m in mats]
    return host, mats


@pytest.fixture(scope="module")
def r1_dense(fdm):
    """A dense layer of R1 size (inter 18432) attached as layer 0."""
    import torch
    say("building dense layer L=0 inter=18432")
    host, mats = dense_weights(11, fdm.DENSE_FFN)
    fdm.attach_dense(0, *mats, fdm.DENSE_FFN)
    del mats
    torch.cuda.empty_cache()
    yield host
    fdm.release_dense(0)


def test_f32_to_f16_matches_oracle(fdm, oracle):
    x = edge_floats()
    nan = np.array([0x7FC00000, 0xFFC00000, 0x7FC02000, 0x7F800001, 0xFFA00000, 0x7FBFFFFF],
                   dtype=np.uint32).view(np.float32)  # quiet and signalling NaNs
    x = np.concatenate([x, nan])
    import torch
    out = torch.empty(x.size, dtype=torch.int16, device="cuda")
    say(f"f32_to_f16 n={x.size}")
    fdm.f32_to_f16(to_dev(x), out, x.size)
    assert np.array_equal(to_host(out).view(np.uint16), oracle.fp32_to_fp16(x))


@pytest.mark.parametrize("tok", [0, 1])
def test_dense_ffn_r1(fdm, oracle, r1_dense, tok):
    gate, up, down = r1_dense
    assert fdm.dense_info(0) == fdm.DENSE_FFN
    h = oracle.synth_normal(H, 0.0, 1.0, 300 + tok)
    h_in = oracle.synth_normal(H, 0.0, 1.0, 400 + tok)
    out = empty_f32(H)
    say(f"dense_ffn L=0 tok={tok}")
    fdm.dense_ffn(0, to_dev(h), to_dev(h_in), out)
    got = to_host(out)
    want = oracle.dense_ffn(gate, up, down, h, h_in)
    err = rel_l2(got, want.astype(np.float64))
    err_ffn = rel_l2(got.astype(np.float64) - h_in, want.astype(np.float64) - h_in)
    print(f"rel_l2={err:.3e} (ffn part {err_ffn:.3e})")
    assert err <= TOL and err_ffn <= TOL


def test_dense_ffn_small_upload_no_residual(fdm, oracle):
    rng = np.random.default_rng(5)
    inter = 1536
    mats = [rng.normal(0, H ** -0.5, (inter, H)).astype(np.float16),
            rng.normal(0, H ** -0.5, (inter, H)).astype(np.float16),
            rng.normal(0, inter ** -0.5, (H, inter)).astype(np.float16)]
    bits = [m.view(np.uint16) for m in mats]
    fdm.upload_dense(5, *bits)
    try:
        h = oracle.synth_normal(H, 0.0, 1.0, 77)
        out = empty_f32(H)
        say(f"dense_ffn L=5 inter={inter}")
        fdm.dense_ffn(5, to_dev(h), None, out)
        assert rel_l2(to_host(out), oracle.dense_ffn(*bits, h).astype(np.float64)) <= TOL
    finally:
        fdm.release_dense(5)


def q4k_blocks(rng, n):
    b = rng.integers(0, 256, (n, 144), dtype=np.uint8)
    b[:, 0:4] = np.abs(rng.normal(0, 0.002, (n, 2))).astype(np.float16).view(np.uint8).reshape(n, 4)
    return b.reshape(-1)


def q6k_blocks(rng, n):
    b = rng.integers(0, 256, (n, 210), dtype=np.uint8)
    b[:, 208:210] = np.abs(rng.normal(0, 0.0005, n)).astype(np.float16).view(np.uint8).reshape(n, 2)
    return b.reshape(-1)


def widened(oracle, gt, raw, n):
    """What dequant_tensor_f16 holds: the type's fp32 values, then (__fp16)."""
    if gt == W.Q4_K:
        f = oracle.dequant_q4k(np.frombuffer(raw, np.uint8), n)
    elif gt == W.Q6_K:
        f = oracle.dequant_q6k(np.frombuffer(raw, np.uint8), n)
    elif gt == W.F16:
        return np.frombuffer(raw, np.uint16).copy()
    elif gt == W.BF16:
        f = (np.frombuffer(raw, np.uint16).astype(np.uint32) << 16).view(np.float32)
    else:
        f = np.frombuffer(raw, np.float32)
    return oracle.fp32_to_fp16(f)


def payload(rng, gt, rows, cols):
    n = rows * cols
    if gt == W.Q4_K:
        return q4k_blocks(rng, n // 256).tobytes()
    if gt == W.Q6_K:
        return q6k_blocks(rng, n // 256).tobytes()
    v = rng.normal(0, cols ** -0.5, n).astype(np.float32)
    if gt == W.F32:
        return v.tobytes()
    if gt == W.F16:
        return v.astype(np.float16).tobytes()
    return (v.view(np.uint32) >> 16).astype(np.uint16).tobytes()  # BF16 (truncated)


@pytest.mark.parametrize("L,types", [(1, (W.Q4_K, W.BF16, W.Q6_K)), (2, (W.F16, W.F32, W.Q4_K))],
                         ids=["q4k_bf16_q6k", "f16_f32_q4k"])
def test_dense_load_gguf(fdm, oracle, tmp_path, L, types):
    from flash_deepseek_amd.gguf import GGUF
    rng = np.random.default_rng(40 + L)
    inter = 512
    shapes = [(inter, H), (inter, H), (H, inter)]  # [rows][cols]
    raws = [payload(rng, t, r, c) for t, (r, c) in zip(types, shapes)]
    p = tmp_path / "dense.gguf"
    W.write_gguf(p, [("general.architecture", W.STRING, "deepseek2")], [
        (f"blk.{L}.ffn_{name}.weight", t, (c, r), raw)
        for name, t, (r, c), raw in zip(("gate", "up", "down"), types, shapes, raws)])
    with GGUF([p]) as m:
        say(f"load_dense_gguf L={L} types={types}")
        assert fdm.load_dense_gguf(L, m) == inter
    try:
        bits = [widened(oracle, t, raw, r * c).reshape(r, c) for t, raw, (r, c) in zip(types, raws, shapes)]
        h = oracle.synth_normal(H, 0.0, 1.0, 90 + L)
        h_in = oracle.synth_normal(H, 0.0, 1.0, 91 + L)
        out = empty_f32(H)
        fdm.dense_ffn(L, to_dev(h), to_dev(h_in), out)
        want = oracle.dense_ffn(*bits, h, h_in).astype(np.float64)
        err = rel_l2(to_host(out), want)
        print(f"rel_l2={err:.3e}")
        assert err <= TOL
    finally:
        fdm.release_dense(L)


def test_dense_errors(fdm, tmp_path):
    from flash_deepseek_amd.gguf import GGUF
    x = empty_f32(H)
    with pytest.raises(fdm.FdmError):
        fdm.dense_ffn(7, x, None, empty_f32(H))  # not resident
    with pytest.raises(fdm.FdmError):
        fdm.dense_info(7)
    bad = np.zeros((500, H), np.uint16)  # inter not a multiple of 512
    with pytest.raises(fdm.FdmError):
        fdm.upload_dense(7, bad, bad, np.zeros((H, 500), np.uint16))
    p = tmp_path / "nodown.gguf"
    W.write_gguf(p, [], [("blk.7.ffn_gate.weight", W.F16, (H, 512), None),
                         ("blk.7.ffn_up.weight", W.F16, (H, 512), None)])
    with GGUF([p]) as m:
        with pytest.raises(fdm.FdmError):
            fdm.load_dense_gguf(7, m)
