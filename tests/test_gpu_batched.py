"""Batched decode (fdm_moe_forward_batched): T tokens through one resident
R1-shape layer in one step with token -> expert dispatch, against the
oracle applied token by token -- routing bit-exact per token, outputs
within 1e-4 relative L2 of the float64 truth, and the distinct-expert count
equal to the number of distinct routed ids."""
import numpy as np
import pytest

from tests._helpers import empty_f32, rel_l2, say, to_dev, to_host

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(scope="module", params=[False, True], ids=["q4k_down", "q6k_down"])
def layer(request, fdm):
    from flash_deepseek_amd.synthetic import make_layer
    L = 11 if request.param else 10
    say(f"building layer L={L} down_q6={request.param}")
    lay = make_layer(2000 + L, down_q6=request.param)
    fdm.attach_layer(L, lay.experts, lay.expert_size, lay.Wg, lay.bias, lay.shared)
    yield L, lay
    fdm.release_layer(L)


@pytest.fixture(params=["dot4", "mfma"])
def batch_kernel(request, fdm):
    """Runs the test under each expert path behind moe_forward_batched: the
    per-token digit dot products and the grouped MFMA GEMMs (three fp16
    planes of the activations)."""
    mode = fdm.BATCH_DOT4 if request.param == "dot4" else fdm.BATCH_MFMA
    prev = fdm.set_batch_kernel(mode)
    yield request.param
    fdm.set_batch_kernel(prev)


def check_tokens(fdm, oracle, L, lay, T, K, seed, tokens_checked, tol=TOL):
    import torch
    X = np.stack([oracle.synth_normal(7168, 0.0, 1.0, seed + t) for t in range(T)])
    Hin = np.stack([oracle.synth_normal(7168, 0.0, 1.0, seed + 1000 + t) for t in range(T)])
    out = empty_f32(T * 7168)
    idx = torch.empty(T * K, dtype=torch.int32, device="cuda")
    w = empty_f32(T * K)
    nd = torch.zeros(1, dtype=torch.int32, device="cuda")
    say(f"moe_forward_batched L={L} T={T} K={K}")
    fdm.moe_forward_batched(L, to_dev(X.ravel()), to_dev(Hin.ravel()), T, K, out, idx, w, nd)
    got = to_host(out).reshape(T, 7168)
    gi = to_host(idx).reshape(T, K)
    gw = to_host(w).reshape(T, K)
    assert int(to_host(nd)[0]) == len(np.unique(gi))
    Wg, bias = to_host(lay.Wg), to_host(lay.bias)
    cache = {}

    def ffn(e):
        if e not in cache:
            cache[e] = oracle.expert_ffn(lay.expert_bytes(e), lay.down_q6, X_t)
        return cache[e]

    for t in tokens_checked:
        X_t = X[t]
        cache.clear()
        ri, rw = oracle.route(oracle.router_logits(Wg, X_t), bias, K=K)
        assert np.array_equal(gi[t], ri), t
        assert np.array_equal(gw[t].view(np.uint32), rw.view(np.uint32)), t
        moe = np.zeros(7168)
        for k in range(K):
            moe += np.float64(rw[k]) * ffn(int(ri[k]))
        want = Hin[t].astype(np.float64) + moe + ffn(-1)
        err = rel_l2(got[t], want)
        assert err <= tol, (t, err)
    # every token's routing is checked (cheap); outputs on the sampled tokens
    for t in range(T):
        ri, rw = oracle.route(oracle.router_logits(Wg, X[t]), bias, K=K)
        assert np.array_equal(gi[t], ri), t


@pytest.mark.parametrize("T,K", [(1, 8), (16, 8), (5, 3), (70, 8), (64, 8), (256, 8)])
def test_batched_matches_per_token_oracle(fdm, oracle, layer, batch_kernel, T, K):
    """T = 70: several tokens per expert and a shared expert spread over
    several items; T = 64 and 256: the batched-decode workloads (routing
    checked on every token, outputs on four of them)."""
    L, lay = layer
    checked = sorted({0, T // 3, (2 * T) // 3, T - 1})
    check_tokens(fdm, oracle, L, lay, T, K, 9000 + 17 * T, tokens_checked=checked, tol=1e-4)


def activations(kind, n, seed):
    """N(0,1); heavy-tailed (a product of normals, a few huge entries); or one
    outlier of +-1e3 in every 32-element sub-block among N(0,1) values (as
    the matvec fp32-grade test): the fp16 planes of the grouped GEMMs are
    scaled per token row, so an outlier pushes the rest of the row down."""
    rng = np.random.default_rng(seed)
    if kind == "normal":
        return rng.standard_normal(n).astype(np.float32)
    if kind == "heavy":
        x = rng.standard_normal(n) * rng.standard_normal(n) * 300
        x[::97] *= 50
        return x.astype(np.float32)
    x = rng.standard_normal(n)
    x[rng.integers(0, 32, n // 32) + 32 * np.arange(n // 32)] = 1e3 * rng.choice([-1.0, 1.0], n // 32)
    return x.astype(np.float32)


@pytest.mark.parametrize("kind", ["normal", "heavy", "outlier"])
@pytest.mark.parametrize("T", [16, 64, 256])
def test_batched_fp32_grade(fdm, oracle, layer, batch_kernel, T, kind):
    """Both expert paths keep every token at fp32 grade on hard inputs: for
    sampled tokens the relative L2 and the largest per-element error of the
    MoE part (sum_k w_k E_k + S) against float64 stay within 4x of the same
    sum in the reference's fp32 arithmetic; routing of every token is
    bit-exact."""
    import torch
    L, lay = layer
    K = 8
    X = activations(kind, T * 7168, 500 + T).reshape(T, 7168)
    out = empty_f32(T * 7168)
    idx = torch.empty(T * K, dtype=torch.int32, device="cuda")
    w = empty_f32(T * K)
    say(f"moe_forward_batched fp32 grade L={L} T={T} input={kind}")
    fdm.moe_forward_batched(L, to_dev(X.ravel()), None, T, K, out, idx, w)
    got = to_host(out).reshape(T, 7168)
    gi = to_host(idx).reshape(T, K)
    gw = to_host(w).reshape(T, K)
    Wg, bias = to_host(lay.Wg), to_host(lay.bias)
    for t in range(T):
        ri, rw = oracle.route(oracle.router_logits(Wg, X[t]), bias, K=K)
        assert np.array_equal(gi[t], ri), t
        assert np.array_equal(gw[t].view(np.uint32), rw.view(np.uint32)), t
    blobs = {}

    def blob(e):
        if e not in blobs:
            blobs[e] = lay.expert_bytes(e)
        return blobs[e]

    for t in sorted({0, T // 2, T - 1}):
        ri, rw = oracle.route(oracle.router_logits(Wg, X[t]), bias, K=K)
        want = oracle.expert_ffn(blob(-1), lay.down_q6, X[t]).astype(np.float64)
        f32 = oracle.expert_ffn_f32(blob(-1), lay.down_q6, X[t]).astype(np.float32)
        for k in range(K):
            e = int(ri[k])
            want += np.float64(rw[k]) * oracle.expert_ffn(blob(e), lay.down_q6, X[t])
            f32 += rw[k] * oracle.expert_ffn_f32(blob(e), lay.down_q6, X[t])
        g = got[t].astype(np.float64)
        e_got, e_f32 = rel_l2(g, want), rel_l2(f32, want)
        m_got, m_f32 = np.abs(g - want).max(), np.abs(f32.astype(np.float64) - want).max()
        print(f"T={T} {kind} token {t}: rel_l2 {e_got:.3e} (fp32 {e_f32:.3e}), max {m_got:.3e} (fp32 {m_f32:.3e})")
        assert e_got <= 4 * e_f32, (t, e_got, e_f32)
        assert m_got <= 4 * m_f32, (t, m_got, m_f32)


def test_batched_paths_agree(fdm, layer):
    """The two expert paths on the same 96-token step: identical routing,
    outputs within 1e-4 of each other (both carry the activations at fp32
    grade)."""
    import torch
    from flash_deepseek_amd.synthetic import make_tokens
    L, _ = layer
    T, K = 96, 8
    X = make_tokens(T, 4321)
    outs = []
    for mode in (fdm.BATCH_DOT4, fdm.BATCH_MFMA):
        prev = fdm.set_batch_kernel(mode)
        try:
            out = empty_f32(T * 7168)
            idx = torch.empty(T * K, dtype=torch.int32, device="cuda")
            say(f"moe_forward_batched L={L} T={T} mode={mode}")
            fdm.moe_forward_batched(L, X, None, T, K, out, idx, None, None)
            outs.append((to_host(out).reshape(T, 7168), to_host(idx)))
        finally:
            fdm.set_batch_kernel(prev)
    assert np.array_equal(outs[0][1], outs[1][1])
    for t in range(T):
        assert rel_l2(outs[1][0][t], outs[0][0][t].astype(np.float64)) <= 1e-4, t


def test_batched_unaligned_residual_and_output(fdm, layer, batch_kernel):
    """h_in and hidden need no 16-byte alignment: the same step with both
    pointers 4 bytes past an aligned address (the combine's one-value-per-
    thread variant) gives the same bits as with aligned ones (its 16-byte
    vector variant)."""
    import torch
    from flash_deepseek_amd.synthetic import make_tokens
    L, _ = layer
    T, K = 24, 8
    X = make_tokens(T, 5150)
    Hin = make_tokens(T, 5151).reshape(-1)
    n = T * 7168
    out_a = empty_f32(n)
    say(f"moe_forward_batched L={L} T={T} aligned")
    fdm.moe_forward_batched(L, X, Hin, T, K, out_a)
    hbuf = torch.zeros(n + 4, dtype=torch.float32, device="cuda")
    hbuf[1:1 + n].copy_(Hin)
    obuf = torch.zeros(n + 4, dtype=torch.float32, device="cuda")
    h_off, o_off = hbuf[1:1 + n], obuf[1:1 + n]
    assert h_off.data_ptr() % 16 != 0 and o_off.data_ptr() % 16 != 0
    say(f"moe_forward_batched L={L} T={T} unaligned h_in / hidden")
    fdm.moe_forward_batched(L, X, h_off, T, K, o_off)
    assert np.array_equal(to_host(out_a).view(np.uint32), to_host(o_off).view(np.uint32))
    assert float(obuf[0]) == 0.0 and float(obuf[1 + n]) == 0.0  # nothing written outside


def test_batched_equals_single_token_layer(fdm, oracle, layer, batch_kernel):
    """Each token of a batch gets the same routing as fdm_moe_layer and an
    output within 1e-4 of it."""
    import torch
    L, lay = layer
    T, K = 12, 8
    X = np.stack([oracle.synth_normal(7168, 0.0, 1.0, 777 + t) for t in range(T)]).astype(np.float32)
    out = empty_f32(T * 7168)
    idx = torch.empty(T * K, dtype=torch.int32, device="cuda")
    fdm.moe_forward_batched(L, to_dev(X.ravel()), None, T, K, out, idx, None, None)
    got = to_host(out).reshape(T, 7168)
    gi = to_host(idx).reshape(T, K)
    for t in (0, 7, 11):
        one = empty_f32(7168)
        i1 = torch.empty(K, dtype=torch.int32, device="cuda")
        fdm.moe_layer(L, to_dev(X[t]), None, K, one, i1)
        assert np.array_equal(to_host(i1), gi[t])
        assert rel_l2(got[t], to_host(one).astype(np.float64)) <= 1e-4


def test_batched_errors(fdm, layer):
    L, _ = layer
    x = empty_f32(7168)
    with pytest.raises(fdm.FdmError):
        fdm.moe_forward_batched(L, x, None, 0, 8, empty_f32(7168))
    with pytest.raises(fdm.FdmError):
        fdm.moe_forward_batched(L, x, None, 513, 8, empty_f32(7168))
    with pytest.raises(fdm.FdmError):
        fdm.moe_forward_batched(L, x, None, 1, 17, empty_f32(7168))
    with pytest.raises(fdm.FdmError):
        fdm.set_batch_kernel(3)
