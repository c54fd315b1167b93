"""MLA attention of decode tokens on the device (fdm_attn_*; mla_forward,
infer.m:766-903) against the oracle over a growing KV cache: hidden after
each token within 1e-3 relative L2 of the float64 truth (attention part and
whole), positions in order and after a jump, the cache length counted, a
reset reproducing the first token bit for bit, and the errors."""
import numpy as np
import pytest

from tests._helpers import rel_l2, say, to_dev, to_host
from tests.mla_case import H, mla_weights

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(scope="module")
def attn_layer(fdm):
    w = mla_weights(903)
    say("attn_upload L=0")
    fdm.attn_upload(0, w, max_seq=64)
    yield w
    fdm.attn_release(0)


def test_attn_tokens_match_oracle(fdm, oracle, attn_layer):
    w = attn_layer
    fdm.attn_reset(0)
    cache = oracle.MlaCache(64)
    rng = np.random.default_rng(5)
    first = None
    for n, pos in enumerate([0, 1, 2, 3, 4, 5, 100]):
        hidden = rng.normal(0, 1, H).astype(np.float32)
        d = to_dev(hidden)
        say(f"attn_forward pos={pos}")
        fdm.attn_forward(0, d, pos)
        got = to_host(d)
        want = oracle.mla_forward(w, hidden, cache, pos)
        err = rel_l2(got, want.astype(np.float64))
        err_attn = rel_l2(got.astype(np.float64) - hidden, want.astype(np.float64) - hidden)
        print(f"pos {pos}: rel_l2 {err:.2e}, attention part {err_attn:.2e}")
        assert err <= TOL and err_attn <= TOL, pos
        assert fdm.attn_len(0) == n + 1
        if first is None:
            first = (hidden, got)
    fdm.attn_reset(0)
    assert fdm.attn_len(0) == 0
    d = to_dev(first[0])
    fdm.attn_forward(0, d, 0)
    assert np.array_equal(to_host(d).view(np.uint32), first[1].view(np.uint32))


def test_attn_long_cache_matches_oracle(fdm, oracle):
    """A cache of up to 2100 positions: the scores, softmax and latent sums
    run over many chunks, merged by the combine (every merge path: a few
    chunks, one batch of chunk loads, and the batched walk of long caches).
    The oracle fills its cache with the append alone and runs the whole
    forward at the checked lengths."""
    w = mla_weights(829)
    say("attn_upload L=5 max_seq=2112")
    fdm.attn_upload(5, w, max_seq=2112)
    try:
        cache = oracle.MlaCache(2112)
        rng = np.random.default_rng(11)
        checks = {69, 599, 1029, 2099}  # token n: cache length n + 1 when it attends
        for n in range(2100):
            hidden = rng.normal(0, 1, H).astype(np.float32)
            d = to_dev(hidden)
            if n in checks or n % 500 == 0:
                say(f"attn_forward L=5 pos={n}")
            fdm.attn_forward(5, d, n)
            if n in checks:
                got = to_host(d)
                want = oracle.mla_forward(w, hidden, cache, n)
                err = rel_l2(got, want.astype(np.float64))
                err_attn = rel_l2(got.astype(np.float64) - hidden, want.astype(np.float64) - hidden)
                print(f"cache {n + 1}: rel_l2 {err:.2e}, attention part {err_attn:.2e}")
                assert err <= TOL and err_attn <= TOL, n
            else:
                oracle.mla_append(w, hidden, cache, n)
        assert fdm.attn_len(5) == 2100
    finally:
        fdm.attn_release(5)


def test_attn_errors(fdm, attn_layer):
    x = to_dev(np.zeros(H, np.float32))
    with pytest.raises(fdm.FdmError):
        fdm.attn_forward(9, x, 0)  # not resident
    with pytest.raises(fdm.FdmError):
        fdm.attn_forward(0, x, -1)
    fdm.attn_upload(9, attn_layer, max_seq=2)
    try:
        fdm.attn_forward(9, x, 0)
        fdm.attn_forward(9, x, 1)
        with pytest.raises(fdm.FdmError):
            fdm.attn_forward(9, x, 2)  # cache full
    finally:
        fdm.attn_release(9)
    with pytest.raises(fdm.FdmError):
        fdm.attn_upload(9, attn_layer, max_seq=0)


def _q4k(rng, n):
    b = rng.integers(0, 256, (n, 144), dtype=np.uint8)
    b[:, 0:4] = np.abs(rng.normal(0, 2e-4, (n, 2))).astype(np.float16).view(np.uint8).reshape(n, 4)
    return b.reshape(-1)


def _q6k(rng, n):
    b = rng.integers(0, 256, (n, 210), dtype=np.uint8)
    b[:, 208:210] = np.abs(rng.normal(0, 1e-4, n)).astype(np.float16).view(np.uint8).reshape(n, 2)
    return b.reshape(-1)


def _tensor(oracle, rng, gt, rows, cols):
    """(payload bytes, F16 bits [rows][cols] as dequant_tensor_f16 makes them)."""
    from tests import gguf_writer as W
    n = rows * cols
    if gt == W.Q4_K:
        raw = _q4k(rng, n // 256)
        return raw.tobytes(), oracle.fp32_to_fp16(oracle.dequant_q4k(raw, n)).reshape(rows, cols)
    if gt == W.Q6_K:
        raw = _q6k(rng, n // 256)
        return raw.tobytes(), oracle.fp32_to_fp16(oracle.dequant_q6k(raw, n)).reshape(rows, cols)
    v = rng.normal(0, cols ** -0.5, n).astype(np.float32)
    if gt == W.F16:
        h = v.astype(np.float16)
        return h.tobytes(), h.view(np.uint16).reshape(rows, cols)
    bf = (v.view(np.uint32) >> 16).astype(np.uint16)  # BF16
    return bf.tobytes(), oracle.fp32_to_fp16((bf.astype(np.uint32) << 16).view(np.float32)).reshape(rows, cols)


@pytest.mark.parametrize("split", [True, False], ids=["k_b_v_b", "kv_b"])
def test_attn_load_gguf_matches_upload(fdm, oracle, tmp_path, split):
    from flash_deepseek_amd.gguf import GGUF
    from tests import gguf_writer as W
    rng = np.random.default_rng(17 + split)
    L = 4
    norms = {"attn_norm": rng.normal(1, 0.1, H).astype(np.float32),
             "q_a_norm": rng.normal(1, 0.1, 1536).astype(np.float32),
             "kv_a_norm": rng.normal(1, 0.1, 512).astype(np.float32)}
    tens = [(f"blk.{L}.attn_norm.weight", W.F32, (H,), norms["attn_norm"].tobytes()),
            (f"blk.{L}.attn_q_a_norm.weight", W.F32, (1536,), norms["q_a_norm"].tobytes()),
            (f"blk.{L}.attn_kv_a_norm.weight", W.F32, (512,), norms["kv_a_norm"].tobytes())]
    w = dict(norms)
    for key, name, gt, rows, cols in [("q_a", "attn_q_a", W.Q4_K, 1536, H), ("q_b", "attn_q_b", W.F16, 128 * 192, 1536),
                                      ("kv_a", "attn_kv_a_mqa", W.BF16, 576, H),
                                      ("o_proj", "attn_output", W.Q4_K, H, 128 * 128)]:
        raw, bits = _tensor(oracle, rng, gt, rows, cols)
        tens.append((f"blk.{L}.{name}.weight", gt, (cols, rows), raw))
        w[key] = bits
    if split:
        raw_k, kb = _tensor(oracle, rng, W.Q6_K, 128 * 128, 512)  # [h][NOPE][KV_LORA]
        raw_v, vb = _tensor(oracle, rng, W.Q4_K, 128 * 128, 512)  # [h][V_HEAD][KV_LORA]
        tens += [(f"blk.{L}.attn_k_b.weight", W.Q6_K, (512, 128, 128), raw_k),
                 (f"blk.{L}.attn_v_b.weight", W.Q4_K, (512, 128, 128), raw_v)]
        w["k_b"] = np.ascontiguousarray(kb.reshape(128, 128, 512).transpose(0, 2, 1))
        w["v_b"] = vb.reshape(128, 128, 512)
    else:
        raw_kv, kvb = _tensor(oracle, rng, W.BF16, 128 * 256, 512)  # [h][NOPE + V_HEAD][KV_LORA]
        tens.append((f"blk.{L}.attn_kv_b.weight", W.BF16, (512, 256 * 128), raw_kv))
        kvb = kvb.reshape(128, 256, 512)
        w["k_b"] = np.ascontiguousarray(kvb[:, :128].transpose(0, 2, 1))
        w["v_b"] = np.ascontiguousarray(kvb[:, 128:])
    p = tmp_path / "attn.gguf"
    W.write_gguf(p, [("general.architecture", W.STRING, "deepseek2")], tens)
    fdm.attn_upload(20, w, max_seq=8)
    try:
        with GGUF([p]) as m:
            say(f"attn_load_gguf split={split}")
            fdm.attn_load_gguf(L, m, max_seq=8)  # reads blk.L.*
        for pos in range(3):
            h = rng.normal(0, 1, H).astype(np.float32)
            a, b = to_dev(h), to_dev(h)
            fdm.attn_forward(20, a, pos)
            fdm.attn_forward(L, b, pos)
            assert np.array_equal(to_host(a).view(np.uint32), to_host(b).view(np.uint32)), pos
    finally:
        fdm.attn_release(20)
        fdm.attn_release(L)
