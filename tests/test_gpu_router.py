"""Router logits and route() on the GPU against the oracle: bit-exact logits
(shared summation order), bit-exact indices in the reference's slot order
and bit-exact weights."""
import numpy as np
import pytest

from tests._helpers import empty_f32, say, to_dev, to_host

pytestmark = pytest.mark.gpu


def route_dev(fdm, logits, bias, K, T):
    import torch
    idx = torch.empty(T * K, dtype=torch.int32, device="cuda")
    w = empty_f32(T * K)
    fdm.route(to_dev(logits.reshape(-1)), None if bias is None else to_dev(bias), K, idx, w, T=T)
    return to_host(idx).reshape(T, K), to_host(w).reshape(T, K)


@pytest.mark.parametrize("T", [1, 5, 21, 64, 256, 512])
def test_router_logits_bit_exact(fdm, oracle, T):
    """T = 256 and 512 run the blocked kernel of batched decode and prefill
    (8 experts x 8 tokens per block); every logit of every token is checked."""
    say(f"router_logits T={T}")
    Wg = oracle.synth_normal(256 * 7168, 0.0, 0.01, 40).reshape(256, 7168)
    X = oracle.synth_normal(T * 7168, 0.0, 1.0, 41 + T).reshape(T, 7168)
    out = empty_f32(T * 256)
    fdm.router_logits(to_dev(Wg), to_dev(X), out, T=T)
    got = to_host(out).reshape(T, 256)
    for t in range(T):
        assert np.array_equal(got[t].view(np.uint32), oracle.router_logits(Wg, X[t]).view(np.uint32))


@pytest.mark.parametrize("K", [1, 4, 8, 16])
def test_route_bit_exact_random(fdm, oracle, K):
    T = 300
    say(f"route random T={T} K={K}")
    rng = np.random.default_rng(K)
    logits = rng.normal(0, 1.5, (T, 256)).astype(np.float32)
    bias = rng.normal(0, 0.1, 256).astype(np.float32)
    idx, w = route_dev(fdm, logits, bias, K, T)
    for t in range(T):
        ri, rw = oracle.route(logits[t], bias, K=K)
        assert np.array_equal(idx[t], ri), t
        assert np.array_equal(w[t].view(np.uint32), rw.view(np.uint32)), t


def test_route_ties_and_no_bias(fdm, oracle):
    # few distinct logits and biases: exact ties inside and across groups, at
    # the group boundary and at the top-K boundary
    T, K = 200, 8
    say("route ties")
    rng = np.random.default_rng(9)
    logits = rng.choice(np.float32([-1.0, 0.0, 0.5, 1.0, 2.0]), (T, 256)).astype(np.float32)
    bias = rng.choice(np.float32([0.0, 0.125]), 256).astype(np.float32)
    for b in (bias, None):
        idx, w = route_dev(fdm, logits, b, K, T)
        for t in range(T):
            ri, rw = oracle.route(logits[t], b, K=K)
            assert np.array_equal(idx[t], ri), t
            assert np.array_equal(w[t].view(np.uint32), rw.view(np.uint32)), t


def test_route_rejects_bad_k(fdm):
    logits = np.zeros(256, np.float32)
    for K in (0, 17):
        with pytest.raises(fdm.FdmError):
            route_dev(fdm, logits, None, K, 1)
