"""The oracle's MLA attention (infer.m:586-655, 766-903) pinned on the CPU:
the YaRN frequency table against its closed form (correction range (10, 23)
of DeepSeek's 64 rope dims, base 10000, original context 4096, factor 40),
the softmax scale against (0.1 ln 40 + 1)^2 / sqrt(192), and mla_forward
against an independent numpy float64 evaluation (matmuls, vectorised
rotation) over a growing cache."""
import numpy as np

from tests.mla_case import H, KVL, NH, NOPE, QK, ROPE, VH, mla_weights


def test_yarn_table_closed_form(oracle):
    i = np.arange(32, dtype=np.float64)
    extra = 10000.0 ** (-2 * i / 64)
    ramp = np.clip((i - 10) / 13, 0, 1)
    want = extra / 40 * ramp + extra * (1 - ramp)
    assert np.allclose(oracle.yarn_freq(), want, rtol=2e-6, atol=0)


def test_softmax_scale(oracle):
    m = 0.1 * np.log(40.0) + 1.0
    assert abs(oracle.mla_scale() - m * m / np.sqrt(192.0)) < 1e-6


def numpy_mla(w, hidden, c, k, pos, oracle):
    f = lambda a: a.view(np.float16).astype(np.float64)
    x = oracle.rms_norm(hidden, w["attn_norm"]).astype(np.float64)
    qa = oracle.rms_norm((f(w["q_a"]) @ x).astype(np.float32), w["q_a_norm"]).astype(np.float64)
    q = (f(w["q_b"]) @ qa).reshape(NH, QK)
    kva = f(w["kv_a"]) @ x
    ckv = oracle.rms_norm(kva[:KVL].astype(np.float32), w["kv_a_norm"])
    ang = (np.float32(pos) * oracle.yarn_freq()).astype(np.float64)
    cs, sn = np.cos(ang), np.sin(ang)

    def rot(v):  # interleaved pairs
        a, b = v[..., 0::2].copy(), v[..., 1::2].copy()
        out = np.empty_like(v)
        out[..., 0::2] = a * cs - b * sn
        out[..., 1::2] = a * sn + b * cs
        return out

    qr = rot(q[:, NOPE:])
    c = np.vstack([c, ckv[None].astype(np.float32)])
    k = np.vstack([k, rot(kva[KVL:]).astype(np.float32)[None]])
    qabs = np.einsum("hrc,hc->hr", f(w["k_b"]), q[:, :NOPE])
    scale = np.float64(oracle.mla_scale())
    s = scale * (qabs @ c.T.astype(np.float64)) + scale * (qr @ k.T.astype(np.float64))
    p = np.exp(s - s.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    wc = p @ c.astype(np.float64)
    attn = np.einsum("hvr,hr->hv", f(w["v_b"]), wc).ravel()
    return (hidden.astype(np.float64) + f(w["o_proj"]) @ attn).astype(np.float32), c, k


def test_mla_forward_matches_numpy(oracle):
    w = mla_weights(766)
    rng = np.random.default_rng(1)
    cache = oracle.MlaCache(8)
    c = np.zeros((0, KVL), np.float32)
    k = np.zeros((0, ROPE), np.float32)
    for pos in (0, 1, 37):
        hidden = rng.normal(0, 1, H).astype(np.float32)
        got = oracle.mla_forward(w, hidden, cache, pos)
        want, c, k = numpy_mla(w, hidden, c, k, pos, oracle)
        assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want)), pos
        assert np.array_equal(cache.c[:cache.len], c) and np.allclose(cache.k[:cache.len], k, rtol=1e-6, atol=1e-7)


def test_mla_append_is_the_forward_cache_row(oracle):
    """mla_append (the cache append alone) writes the same cache row as
    mla_forward, bit for bit, at in-order and jumped positions."""
    w = mla_weights(767)
    rng = np.random.default_rng(2)
    full, app = oracle.MlaCache(4), oracle.MlaCache(4)
    for pos in (0, 5, 1999):
        hidden = rng.normal(0, 1, H).astype(np.float32)
        oracle.mla_forward(w, hidden, full, pos)
        oracle.mla_append(w, hidden, app, pos)
    assert app.len == full.len == 3
    assert np.array_equal(app.c.view(np.uint32), full.c.view(np.uint32))
    assert np.array_equal(app.k.view(np.uint32), full.k.view(np.uint32))
