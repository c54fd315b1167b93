"""Prefill (fdm_moe_prefill): T tokens through stacked MoE layers (Q4_K and
Q6_K down), h <- h + MoE(rms_norm(h, w)).  The expert GEMMs contract one
fp16 plane of the activations on MFMA, so the bar is 1e-2 relative L2
against the float64 truth; routing (fp32 rms_norm output, same router
kernels) stays bit-exact; rms_norm itself is bit-exact with the reference's
sequential loop."""
import numpy as np
import pytest

from tests._helpers import empty_f32, rel_l2, say, to_dev, to_host

pytestmark = pytest.mark.gpu
TOL = 1e-2


@pytest.fixture(scope="module")
def layers(fdm):
    from flash_deepseek_amd.synthetic import make_layer
    out = []
    for L in (20, 21, 22, 23):
        say(f"building layer L={L}")
        lay = make_layer(3000 + L, down_q6=(L == 22))
        fdm.attach_layer(L, lay.experts, lay.expert_size, lay.Wg, lay.bias, lay.shared)
        out.append((L, lay))
    yield out
    for L, _ in out:
        fdm.release_layer(L)


def test_rms_norm_bit_exact(fdm, oracle):
    T = 5
    x = np.stack([oracle.synth_normal(7168, 0.0, 2.0, 40 + t) for t in range(T)]).astype(np.float32)
    w = oracle.synth_normal(7168, 1.0, 0.1, 49)
    o = empty_f32(T * 7168)
    fdm.rms_norm(to_dev(x.ravel()), to_dev(w), o, T)
    got = to_host(o).reshape(T, 7168)
    for t in range(T):
        want = oracle.rms_norm(x[t], w)
        assert np.array_equal(got[t].view(np.uint32), want.view(np.uint32)), t


def oracle_layer_step(oracle, lay, h, w_norm, K):
    """One layer on the CPU: h + moe + shared with moe over route() of rms_norm(h)."""
    Wg, bias = to_host(lay.Wg), to_host(lay.bias)
    hp = oracle.rms_norm(h.astype(np.float32), w_norm)
    ri, rw = oracle.route(oracle.router_logits(Wg, hp), bias, K=K)
    moe = np.zeros(7168)
    for k in range(K):
        moe += np.float64(rw[k]) * oracle.expert_ffn(lay.expert_bytes(int(ri[k])), lay.down_q6, hp)
    sd = oracle.expert_ffn(lay.expert_bytes(-1), lay.down_q6, hp)
    return ri, h.astype(np.float64) + moe + sd


def test_prefill_each_layer_matches_oracle(fdm, oracle, layers):
    """Every layer on fresh N(0,1) activations.  (Chained through these
    synthetic layers, whose Q4_K weights have a large positive mean, the
    residual stream grows to ~1e10 with a strong common mode, and the next
    layer's SwiGLU outputs are all zero -- a degenerate check; chaining is
    covered by the stack-equals-chain test.)"""
    import torch
    T, K = 6, 8
    norms = [oracle.synth_normal(7168, 1.0, 0.1, 80 + i) for i in range(len(layers))]
    dnorm = [to_dev(w) for w in norms]
    idx = torch.empty(T * K, dtype=torch.int32, device="cuda")
    for i, (L, lay) in enumerate(layers):
        H0 = np.stack([oracle.synth_normal(7168, 0.0, 1.0, 70 + 10 * i + t)
                       for t in range(T)]).astype(np.float32)
        dH = to_dev(H0.ravel())
        h_before = H0
        say(f"prefill layer {L} T={T}")
        fdm.moe_prefill([L], dH, T, K, [dnorm[i]], idx)
        got = to_host(dH).reshape(T, 7168)
        gi = to_host(idx).reshape(T, K)
        for t in range(T):
            ri, want = oracle_layer_step(oracle, lay, h_before[t], norms[i], K)
            assert np.array_equal(gi[t], ri), (L, t)
            err = rel_l2(got[t].astype(np.float64) - h_before[t], want - h_before[t])
            print(f"layer {L} token {t}: rel_l2 of the MoE update {err:.2e}")
            assert err <= TOL, (L, t, err)


def test_prefill_stack_equals_layer_chain(fdm, oracle, layers):
    import torch
    T, K = 9, 8
    H0 = np.stack([oracle.synth_normal(7168, 0.0, 1.0, 170 + t) for t in range(T)]).astype(np.float32)
    norms = [to_dev(oracle.synth_normal(7168, 1.0, 0.1, 180 + i)) for i in range(len(layers))]
    ids = [L for L, _ in layers]
    a = to_dev(H0.ravel())
    fdm.moe_prefill(ids, a, T, K, norms)
    b = to_dev(H0.ravel())
    for i, L in enumerate(ids):
        fdm.moe_prefill([L], b, T, K, [norms[i]])
    assert np.array_equal(to_host(a), to_host(b))


def test_prefill_matches_batched_decode(fdm, oracle, layers):
    """At T = 128: one prefill layer against rms_norm + the (digit-precise)
    batched decode path on the same h_post: same routing, outputs within the
    bf16 bar."""
    import torch
    T, K = 128, 8
    L, lay = layers[0]
    from flash_deepseek_amd.synthetic import make_tokens
    H = make_tokens(T, 4242)
    say(f"prefill vs batched decode L={L} T={T}")
    w = to_dev(oracle.synth_normal(7168, 1.0, 0.1, 4243))
    hp = torch.empty_like(H)
    fdm.rms_norm(H, w, hp, T)
    ref = torch.empty_like(H)
    i_ref = torch.empty(T * K, dtype=torch.int32, device="cuda")
    fdm.moe_forward_batched(L, hp, H, T, K, ref, i_ref)
    got = H.clone()
    i_got = torch.empty(T * K, dtype=torch.int32, device="cuda")
    fdm.moe_prefill([L], got, T, K, [w], i_got)
    torch.cuda.synchronize()
    assert torch.equal(i_got, i_ref)
    upd_got = (got - H).double().cpu().numpy()
    upd_ref = (ref - H).double().cpu().numpy()
    err = rel_l2(upd_got.ravel(), upd_ref.ravel())
    print(f"prefill vs batched decode, T={T}: rel_l2 {err:.2e}")
    assert err <= TOL


@pytest.mark.parametrize("T", [100, 90])
def test_prefill_large_chunks_match_batched_decode(fdm, oracle, layers, T):
    """Every token routed to the same 8 experts (a router bias of +10 on
    four experts of each of two groups): the prefill GEMMs run a 64-token
    chunk per expert and a remainder of 36 (T = 100) or 26 (T = 90) tokens,
    the four-, three- and two-block bodies; against the batched decode path
    (16-token chunks) on the same h_post: identical routing, every token's
    update within the bar."""
    import torch
    from flash_deepseek_amd.synthetic import make_tokens
    K, L = 8, 29
    _, lay = layers[0]
    fav = [1, 5, 9, 13, 100, 104, 108, 112]
    bias = lay.bias.clone()
    bias[fav] += 10.0
    say(f"attaching L={L} with a router bias onto experts {fav}")
    fdm.attach_layer(L, lay.experts, lay.expert_size, lay.Wg, bias, lay.shared)
    try:
        H = make_tokens(T, 4300 + T)
        w = to_dev(oracle.synth_normal(7168, 1.0, 0.1, 4301))
        hp = torch.empty_like(H)
        fdm.rms_norm(H, w, hp, T)
        ref = torch.empty_like(H)
        i_ref = torch.empty(T * K, dtype=torch.int32, device="cuda")
        say(f"batched decode L={L} T={T}")
        fdm.moe_forward_batched(L, hp, H, T, K, ref, i_ref)
        got = H.clone()
        i_got = torch.empty(T * K, dtype=torch.int32, device="cuda")
        say(f"prefill L={L} T={T}")
        fdm.moe_prefill([L], got, T, K, [w], i_got)
        torch.cuda.synchronize()
        assert torch.equal(i_got, i_ref)
        assert sorted(np.unique(to_host(i_got)).tolist()) == fav
        upd_got = (got - H).double().cpu().numpy()
        upd_ref = (ref - H).double().cpu().numpy()
        errs = [rel_l2(upd_got[t], upd_ref[t]) for t in range(T)]
        print(f"T={T}: per-token rel_l2 max {max(errs):.2e}")
        assert max(errs) <= TOL
    finally:
        fdm.release_layer(L)


def test_prefill_512_tokens_4_layers(fdm, oracle, layers):
    """The prefill workload: 512 tokens through the 4-layer stack in one call
    with the routing captured; the same stack layer by layer gives each
    layer's input (and must give the same bits).  Routing of every token of
    every layer against the oracle on that input; the MoE update of sampled
    tokens within 1e-2.  (Through these synthetic layers the residual grows
    by orders of magnitude per layer; rms_norm rescales each layer's input,
    so routing and the updates stay meaningful checks.)"""
    import torch
    from flash_deepseek_amd.synthetic import make_tokens
    T, K = 512, 8
    ids = [L for L, _ in layers]
    norms = [oracle.synth_normal(7168, 1.0, 0.1, 280 + i) for i in range(len(layers))]
    dnorm = [to_dev(w) for w in norms]
    H0 = make_tokens(T, 2424)
    idx = torch.empty(len(ids) * T * K, dtype=torch.int32, device="cuda")
    stack = H0.clone()
    say(f"prefill stack of {len(ids)} layers T={T}")
    fdm.moe_prefill(ids, stack, T, K, dnorm, idx)
    inputs = []
    h = H0.clone()
    for i, L in enumerate(ids):
        inputs.append(to_host(h).reshape(T, 7168).copy())
        say(f"prefill layer {L} alone T={T}")
        fdm.moe_prefill([L], h, T, K, [dnorm[i]])
    assert torch.equal(h, stack)
    gi = to_host(idx).reshape(len(ids), T, K)
    for i, (L, lay) in enumerate(layers):
        Wg, bias = to_host(lay.Wg), to_host(lay.bias)
        H_in = inputs[i]
        out = inputs[i + 1] if i + 1 < len(ids) else to_host(h).reshape(T, 7168)
        for t in range(T):
            hp = oracle.rms_norm(H_in[t], norms[i])
            ri, _ = oracle.route(oracle.router_logits(Wg, hp), bias, K=K)
            assert np.array_equal(gi[i, t], ri), (L, t)
        for t in (0, 171, 342, 511):
            ri, want = oracle_layer_step(oracle, lay, H_in[t], norms[i], K)
            err = rel_l2(out[t].astype(np.float64) - H_in[t], want - H_in[t])
            print(f"layer {L} token {t}: rel_l2 of the MoE update {err:.2e}")
            assert err <= TOL, (L, t, err)


def test_prefill_512_fresh_tokens_each_layer(fdm, oracle, layers):
    """The bench's per-layer workload: each of the 4 layers alone on its own
    512 fresh N(0,1) tokens (~190 distinct experts per layer, every chunk
    body of the grouped GEMMs).  Routing of every token against the oracle,
    and the MoE update of 6 sampled tokens per layer within 1e-2."""
    import torch
    from flash_deepseek_amd.synthetic import make_tokens
    T, K = 512, 8
    for i, (L, lay) in enumerate(layers):
        w_norm = oracle.synth_normal(7168, 1.0, 0.1, 380 + i)
        H0 = make_tokens(T, 9300 + i)
        h = H0.clone()
        idx = torch.empty(T * K, dtype=torch.int32, device="cuda")
        say(f"prefill layer {L} alone on fresh tokens T={T}")
        fdm.moe_prefill([L], h, T, K, [to_dev(w_norm)], idx)
        H_in = to_host(H0).reshape(T, 7168)
        out = to_host(h).reshape(T, 7168)
        gi = to_host(idx).reshape(T, K)
        Wg, bias = to_host(lay.Wg), to_host(lay.bias)
        for t in range(T):
            hp = oracle.rms_norm(H_in[t], w_norm)
            ri, _ = oracle.route(oracle.router_logits(Wg, hp), bias, K=K)
            assert np.array_equal(gi[t], ri), (L, t)
        print(f"layer {L}: {len(np.unique(gi))} distinct experts")
        for t in (0, 97, 200, 301, 420, 511):
            ri, want = oracle_layer_step(oracle, lay, H_in[t], w_norm, K)
            err = rel_l2(out[t].astype(np.float64) - H_in[t], want - H_in[t])
            print(f"layer {L} token {t}: rel_l2 of the MoE update {err:.2e}")
            assert err <= TOL, (L, t, err)


def test_prefill_errors(fdm, layers):
    L, _ = layers[0]
    h = empty_f32(7168)
    with pytest.raises(fdm.FdmError):
        fdm.moe_prefill([L], h, 0, 8, None)
    with pytest.raises(fdm.FdmError):
        fdm.moe_prefill([L], h, 1, 17, None)
