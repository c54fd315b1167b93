"""The C restatement of the expert path (oracle/moe_ref.c, cpu_baseline.c),
pinned by composition from independently computed pieces: the pinned
decoders plus numpy float64 linear algebra, SiLU from its definition, the
combine order of infer.m:1689-1695 / 1922, and route() from the pinned
router functions.
"""
import numpy as np
import pytest


def deq_matrix(oracle, raw, rows, cols, q6=False):
    flat = (oracle.dequant_q6k if q6 else oracle.dequant_q4k)(raw, rows * cols)
    return flat.reshape(rows, cols).astype(np.float64)


@pytest.mark.parametrize("q6", [False, True])
def test_matvec_oracle_is_row_major_dot(oracle, q6):
    rows, cols = 48, 1024
    nb = rows * cols // 256
    raw = oracle.synth_q6k(nb, 11) if q6 else oracle.synth_q4k(nb, 11)
    x = oracle.synth_normal(cols, 0.0, 1.0, 12)
    y = oracle.matvec(raw, x, rows, cols, "q6k" if q6 else "q4k")
    ref = deq_matrix(oracle, raw, rows, cols, q6) @ x.astype(np.float64)
    assert np.allclose(y, ref, rtol=1e-6, atol=1e-6 * np.abs(ref).max())
    y32 = oracle.matvec(raw, x, rows, cols, "q6k" if q6 else "q4k", f32=True)
    assert np.linalg.norm(y32 - ref) <= 1e-5 * np.linalg.norm(ref)


def expert_ref(oracle, blob, q6, x):
    G = oracle.GATE_BYTES
    Wg = deq_matrix(oracle, blob[:G], 2048, 7168)
    Wu = deq_matrix(oracle, blob[G:2 * G], 2048, 7168)
    Wd = deq_matrix(oracle, blob[2 * G:], 7168, 2048, q6)
    g = Wg @ x.astype(np.float64)
    u = Wu @ x.astype(np.float64)
    a = g / (1.0 + np.exp(-g)) * u
    return Wd @ a, g, u, a


@pytest.mark.parametrize("q6", [False, True])
def test_expert_ffn_composition(oracle, q6):
    blob = oracle.synth_expert(21, down_is_q6=q6)
    assert blob.size == (oracle.EXPERT_Q6K if q6 else oracle.EXPERT_Q4K)
    x = oracle.synth_normal(7168, 0.0, 1.0, 22)
    out, g, u, a = oracle.expert_ffn(blob, q6, x, with_intermediates=True)
    ref, rg, ru, ra = expert_ref(oracle, blob, q6, x)
    for got, want in ((g, rg), (u, ru), (a, ra), (out, ref)):
        assert np.linalg.norm(got - want) <= 1e-6 * np.linalg.norm(want)


def test_moe_forward_and_layer_composition(oracle):
    K = 8
    E = oracle.EXPERT_Q4K
    # a layer whose router is steered onto experts 0..7, so only those
    # blobs need to exist (the layer oracle indexes experts by id)
    experts = np.concatenate([oracle.synth_expert(100 + e) for e in range(K)])
    shared = oracle.synth_expert(99)
    Wg = oracle.synth_normal(256 * 7168, 0.0, 0.01, 31).reshape(256, 7168)
    bias = oracle.synth_normal(256, 0.0, 0.1, 32)
    bias[:8] += 10.0
    h = oracle.synth_normal(7168, 0.0, 1.0, 33)
    h_in = oracle.synth_normal(7168, 0.0, 1.0, 34)
    hid, idx, w, moe, sd = oracle.moe_layer(experts, E, Wg, bias, shared, h, h_in, K)
    # routing = route(router_logits)
    ridx, rw = oracle.route(oracle.router_logits(Wg, h), bias, K=K)
    assert np.array_equal(idx, ridx) and np.array_equal(w, rw)
    assert sorted(idx) == list(range(8))
    # moe_out = sum_k w_k E_k in slot order (fma), shared added unweighted
    eo = [oracle.expert_ffn(experts[i * E:(i + 1) * E], False, h) for i in idx]
    acc = np.zeros(7168, np.float32)
    for k in range(K):
        acc = (np.float64(w[k]) * eo[k] + acc).astype(np.float32)  # fma rounding
    assert np.array_equal(moe, acc)
    assert np.array_equal(sd, oracle.expert_ffn(shared, False, h))
    assert np.array_equal(hid, (h_in + moe) + sd)
    # metal_moe_forward twin
    mf = oracle.moe_forward(experts, E, h, idx, w)
    assert np.array_equal(mf, moe)


def test_cpu_baseline_computes_the_expert_path(oracle):
    blobs = [oracle.synth_expert(300 + i) for i in range(2)]
    x = oracle.synth_normal(7168, 0.0, 1.0, 301)
    w = np.array([0.7, 1.3], np.float32)
    us, out = oracle.cpu_expert_baseline(blobs, False, x, w, reps=1)
    assert us > 0
    ref = 0.7 * oracle.expert_ffn(blobs[0], False, x) + 1.3 * oracle.expert_ffn(blobs[1], False, x)
    assert np.linalg.norm(out - ref) <= 1e-4 * np.linalg.norm(ref)
