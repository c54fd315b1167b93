"""The full batch-1 MoE layer (fdm_moe_layer) and the metal_moe_forward
twins on a resident, seeded 256-expert layer of R1 shape, against the
oracle: routing bit-exact (indices in slot order and weights), outputs
within 1e-3 relative L2 of the float64 truth."""
import numpy as np
import pytest

from tests._helpers import empty_f32, rel_l2, say, to_dev, to_host

pytestmark = pytest.mark.gpu
TOL = 1e-3


def build(fdm, L, seed, down_q6):
    from flash_deepseek_amd.synthetic import make_layer
    say(f"building layer L={L} seed={seed} down_q6={down_q6}")
    lay = make_layer(seed, down_q6=down_q6)
    fdm.attach_layer(L, lay.experts, lay.expert_size, lay.Wg, lay.bias, lay.shared)
    return lay


@pytest.fixture(scope="module", params=[False, True], ids=["q4k_down", "q6k_down"])
def layer(request, fdm):
    L = 7 if request.param else 3
    lay = build(fdm, L, 1000 + L, request.param)
    yield L, lay
    fdm.release_layer(L)


def oracle_layer(oracle, lay, h, h_in, K, Wg=None, bias=None):
    Wg = to_host(lay.Wg if Wg is None else Wg)
    bias = to_host(lay.bias if bias is None else bias)
    ri, rw = oracle.route(oracle.router_logits(Wg, h), bias, K=K)
    moe = np.zeros(7168)
    for k in range(K):
        moe += np.float64(rw[k]) * oracle.expert_ffn(lay.expert_bytes(int(ri[k])), lay.down_q6, h)
    sd = oracle.expert_ffn(lay.expert_bytes(-1), lay.down_q6, h).astype(np.float64)
    return ri, rw, moe, sd, h_in.astype(np.float64) + moe + sd


def run_layer(fdm, oracle, L, lay, K, tok, Wg=None, bias=None):
    import torch
    h = oracle.synth_normal(7168, 0.0, 1.0, 500 + tok)
    h_in = oracle.synth_normal(7168, 0.0, 1.0, 600 + tok)
    hid = empty_f32(7168)
    idx = torch.empty(K, dtype=torch.int32, device="cuda")
    w = empty_f32(K)
    say(f"moe_layer L={L} K={K} tok={tok}")
    fdm.moe_layer(L, to_dev(h), to_dev(h_in), K, hid, idx, w)
    got, gi, gw = to_host(hid), to_host(idx), to_host(w)
    ri, rw, moe, sd, want = oracle_layer(oracle, lay, h, h_in, K, Wg, bias)
    return h_in, got, gi, gw, ri, rw, moe, sd, want


@pytest.mark.parametrize("K,tok", [(8, 0), (8, 1), (1, 2), (4, 3), (16, 4)])
def test_moe_layer(fdm, oracle, layer, K, tok):
    L, lay = layer
    h_in, got, gi, gw, ri, rw, moe, sd, want = run_layer(fdm, oracle, L, lay, K, tok)
    assert np.array_equal(gi, ri)
    assert np.array_equal(gw.view(np.uint32), rw.view(np.uint32))
    err = rel_l2(got, want)
    err_moe = rel_l2(got.astype(np.float64) - h_in, moe + sd)
    print(f"idx={gi.tolist()} rel_l2={err:.3e} (moe part {err_moe:.3e})")
    assert err <= TOL and err_moe <= TOL


def test_moe_layer_fp32_grade(fdm, oracle, layer):
    """The MoE part of the layer (sum_k w_k E_k + S) against float64: within
    4x the error of the same sum in the reference's fp32 arithmetic."""
    L, lay = layer
    K = 8
    h_in, got, gi, gw, ri, rw, moe, sd, want = run_layer(fdm, oracle, L, lay, K, 5)
    f32 = np.zeros(7168, np.float32)
    for k in range(K):
        f32 += rw[k] * oracle.expert_ffn_f32(lay.expert_bytes(int(ri[k])), lay.down_q6, lay_h(oracle, 5))
    f32 += oracle.expert_ffn_f32(lay.expert_bytes(-1), lay.down_q6, lay_h(oracle, 5))
    e_got = rel_l2(got.astype(np.float64) - h_in, moe + sd)
    e_f32 = rel_l2(f32, moe + sd)
    print(f"moe part rel_l2 {e_got:.3e} (fp32 restatement {e_f32:.3e})")
    assert e_got <= 4 * e_f32


def lay_h(oracle, tok):
    return oracle.synth_normal(7168, 0.0, 1.0, 500 + tok)


@pytest.mark.parametrize("K,nudge", [(5, 0.0), (7, 0.0), (5, 2.0 ** -22), (7, 2.0 ** -22), (8, 2.0 ** -22)])
def test_moe_layer_tied_set(fdm, oracle, layer, K, nudge):
    """Every router row and bias duplicated in adjacent experts (same group):
    each choice occurs twice, so with K odd the K-th largest is tied with an
    expert left out and the set itself depends on route()'s scan order.
    With a nudge the odd expert's bias is larger by 2^-22: the choices of a
    pair differ in their last few bits only, so the K-th and (K+1)-th keys
    agree in their upper 24 bits (the set kernel's packed keys tie) while
    the reference's order is strict."""
    L, lay = layer
    Wg = lay.Wg.clone()
    Wg[1::2] = Wg[0::2]
    bias = lay.bias.clone()
    bias[1::2] = bias[0::2] + nudge
    L2 = L + 20
    fdm.attach_layer(L2, lay.experts, lay.expert_size, Wg, bias, lay.shared)
    try:
        h_in, got, gi, gw, ri, rw, moe, sd, want = run_layer(fdm, oracle, L2, lay, K, 9, Wg, bias)
    finally:
        fdm.release_layer(L2)
    assert np.array_equal(gi, ri)
    assert np.array_equal(gw.view(np.uint32), rw.view(np.uint32))
    assert rel_l2(got, want) <= TOL


def test_moe_forward_given_routing(fdm, oracle, layer):
    import torch
    L, lay = layer
    # metal_moe_forward semantics: any routing, repeated ids allowed, K = 16
    K = 16
    rng = np.random.default_rng(L)
    ids = rng.integers(0, 256, K).astype(np.int32)
    ids[3] = ids[2]
    ws = rng.uniform(0.05, 0.6, K).astype(np.float32)
    h = oracle.synth_normal(7168, 0.0, 1.0, 700)
    out = empty_f32(7168)
    say(f"moe_forward L={L} K={K}")
    fdm.moe_forward(L, to_dev(h), to_dev(ids), to_dev(ws), K, out)
    want = np.zeros(7168)
    cache = {}
    for k in range(K):
        e = int(ids[k])
        if e not in cache:
            cache[e] = oracle.expert_ffn(lay.expert_bytes(e), lay.down_q6, h)
        want += np.float64(ws[k]) * cache[e]
    assert rel_l2(to_host(out), want) <= TOL
    # host-pointer twin (synchronous, metal_moe_forward's convention)
    host_out = np.empty(7168, np.float32)
    fdm.moe_forward_host(L, h, ids, ws, K, host_out)
    assert np.array_equal(host_out, to_host(out))


def test_layer_wait_timeout_is_reported(fdm, oracle, layer):
    """A launch whose kernel waits give up (forced from the host with a limit
    of one poll; every workgroup still exits) is reported once by sync(),
    and the next launch computes correctly again."""
    L, lay = layer
    fdm.sync()
    h = oracle.synth_normal(7168, 0.0, 1.0, 42)
    out = empty_f32(7168)
    prev = fdm.set_layer_spin_limit(1)
    try:
        say(f"moe_layer L={L} with a one-poll wait limit")
        fdm.moe_layer(L, to_dev(h), None, 8, out)
        with pytest.raises(fdm.FdmError) as err:
            fdm.sync()
        assert err.value.code == -4  # FDM_E_STATE
        fdm.sync()  # reported once
    finally:
        fdm.set_layer_spin_limit(prev)
    say(f"moe_layer L={L} with the default wait limit")
    fdm.moe_layer(L, to_dev(h), None, 8, out)
    fdm.sync()
    ri, rw, moe, sd, want = oracle_layer(oracle, lay, h, np.zeros(7168, np.float32), 8)
    assert rel_l2(to_host(out), want) <= TOL


def test_errors(fdm, layer):
    L, _ = layer
    h = empty_f32(7168)
    with pytest.raises(fdm.FdmError):
        fdm.moe_layer(L, h, None, 17, empty_f32(7168))
    with pytest.raises(fdm.FdmError):
        fdm.moe_layer(60, h, None, 8, empty_f32(7168))  # not resident


@pytest.mark.parametrize("scale,tok", [(1.0, 20), (37.0, 21), (1e-3, 22)])
def test_moe_layer_norm_fused(fdm, oracle, layer, scale, tok):
    """fdm_moe_layer_norm (rms_norm inside the layer launch) against
    fdm_rms_norm followed by fdm_moe_layer on the same hidden state: the
    same h_post bits (and the oracle's rms_norm), the same routing and the
    same output bits; then once more in place (hidden = h)."""
    import torch
    L, lay = layer
    K = 8
    h = (oracle.synth_normal(7168, 0.0, 1.0, 700 + tok) * scale).astype(np.float32)
    nw = oracle.synth_normal(7168, 1.0, 0.1, 800 + tok)
    hd, nwd = to_dev(h), to_dev(nw)
    hid, hp = empty_f32(7168), empty_f32(7168)
    idx = torch.empty(K, dtype=torch.int32, device="cuda")
    w = empty_f32(K)
    say(f"moe_layer_norm L={L} tok={tok} scale={scale}")
    fdm.moe_layer_norm(L, hd, nwd, K, hid, hp, idx, w)
    hp_ref, hid_ref = empty_f32(7168), empty_f32(7168)
    idx_ref = torch.empty(K, dtype=torch.int32, device="cuda")
    w_ref = empty_f32(K)
    say(f"rms_norm + moe_layer L={L} tok={tok}")
    fdm.rms_norm(hd, nwd, hp_ref, 1)
    fdm.moe_layer(L, hp_ref, hd, K, hid_ref, idx_ref, w_ref)
    assert np.array_equal(to_host(hp).view(np.uint32), oracle.rms_norm(h, nw).view(np.uint32))
    assert np.array_equal(to_host(hp).view(np.uint32), to_host(hp_ref).view(np.uint32))
    assert np.array_equal(to_host(idx), to_host(idx_ref))
    assert np.array_equal(to_host(w).view(np.uint32), to_host(w_ref).view(np.uint32))
    assert np.array_equal(to_host(hid).view(np.uint32), to_host(hid_ref).view(np.uint32))
    ri, _ = oracle.route(oracle.router_logits(to_host(lay.Wg), oracle.rms_norm(h, nw)), to_host(lay.bias), K=K)
    assert np.array_equal(to_host(idx), ri)
    say(f"moe_layer_norm in place L={L} tok={tok}")
    hio = hd.clone()
    fdm.moe_layer_norm(L, hio, nwd, K, hio)
    assert np.array_equal(to_host(hio).view(np.uint32), to_host(hid_ref).view(np.uint32))


NORM_KINDS = [("normal", 6), ("scaled", 12), ("outliers", 6), ("dominant", 24), ("small_ints", 4),
              ("powers_of_two", 4), ("leading_zeros", 4), ("tiny_first", 4), ("tiny", 2)]


@pytest.mark.parametrize("kind,T", NORM_KINDS, ids=[k for k, _ in NORM_KINDS])
def test_moe_layer_norm_hidden_states(fdm, oracle, layer, kind, T):
    """The fused rms_norm on the hidden-state kinds of the rms_norm tests:
    h_post bit-exact with the oracle's rms_norm for every token, including
    sums with many ties or below 2^-100 (the two-pass and plain-chain paths)
    and a dominating element."""
    import zlib
    import torch
    from tests.test_gpu_rms import tokens
    L, _ = layer
    K = 8
    rng = np.random.default_rng(zlib.crc32(("layer-" + kind).encode()))
    x = tokens(kind, T, 7168, rng)
    nw = rng.normal(1.0, 0.1, 7168).astype(np.float32)
    nwd = to_dev(nw)
    hid, hp = empty_f32(7168), empty_f32(7168)
    idx = torch.empty(K, dtype=torch.int32, device="cuda")
    w = empty_f32(K)
    for t in range(T):
        say(f"moe_layer_norm L={L} kind={kind} token={t}")
        fdm.moe_layer_norm(L, to_dev(x[t]), nwd, K, hid, hp, idx, w)
        want = oracle.rms_norm(x[t], nw)
        assert np.array_equal(to_host(hp).view(np.uint32), want.view(np.uint32)), (kind, t)


def test_moe_layer_norm_rejects_h_post_overlapping_h(fdm, layer):
    """The norm item writes h_post while router rows and digit items still
    read h, so an h_post that overlaps h is rejected before any launch."""
    from flash_deepseek_amd._lib import FDM_E_INVAL
    L, _ = layer
    buf = empty_f32(2 * 7168)
    nw = empty_f32(7168).fill_(1.0)
    h = buf[:7168]
    hid = empty_f32(7168)
    for off in (0, 7167):  # the same buffer, and the last element of h under the first of h_post
        with pytest.raises(fdm.FdmError) as err:
            fdm.moe_layer_norm(L, h, nw, 8, hid, buf[off:off + 7168])
        assert err.value.code == FDM_E_INVAL
    fdm.sync()


def test_layer_read_ceiling_reads_the_layer_bytes(fdm, layer):
    """fdm_layer_read_ceiling (the streaming-ceiling launch of the bench)
    reads exactly the bytes one layer launch reads: the sum of its sink
    (mod 2^32) equals the sum of every byte of the router weights and bias,
    the K routed experts' packed blobs (the resident layout is a permutation
    of their bytes, so the sum is the same), the shared expert, h_post and
    h_in."""
    import torch
    L, lay = layer
    ids = np.array([3, 250, 17, 17, 99, 0, 128, 255], np.int32)  # a repeated id is read twice
    h = np.random.default_rng(71).standard_normal(7168).astype(np.float32)
    h_in = np.random.default_rng(72).standard_normal(7168).astype(np.float32)
    sink = torch.zeros(7168, dtype=torch.int32, device="cuda")
    say(f"layer_read_ceiling L={L} K={len(ids)}")
    fdm.layer_read_ceiling(L, to_dev(ids), len(ids), to_dev(h), to_dev(h_in), sink)
    got = int(to_host(sink).view(np.uint32).astype(np.uint64).sum()) % (1 << 32)

    def bytesum(a):
        return int(np.ascontiguousarray(a).view(np.uint8).astype(np.uint64).sum())

    want = bytesum(to_host(lay.Wg)) + bytesum(to_host(lay.bias)) + bytesum(lay.expert_bytes(-1))
    want += bytesum(h) + bytesum(h_in)
    for e in ids:
        want += bytesum(lay.expert_bytes(int(e)))
    assert got == want % (1 << 32), (hex(got), hex(want % (1 << 32)))
