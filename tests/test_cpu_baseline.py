"""The two CPU baselines of the bench (oracle/cpu_baseline.c: the
reference-shaped path; oracle/cpu_tuned.c: fused row dequant-dot on every
core) compute the same MoE branch: both within fp32 rounding of the float64
oracle on the same experts and routing."""
import numpy as np

from oracle import oracle as O


import pytest


@pytest.mark.parametrize("q6", [False, True])
def test_cpu_baselines_agree_with_oracle(q6):
    K = 2
    rng = np.random.default_rng(3)
    blobs = [O.synth_expert(40 + i, down_is_q6=q6) for i in range(K + 1)]
    Wg = (rng.standard_normal((256, 7168)) * 0.01).astype(np.float32)
    bias = (rng.standard_normal(256) * 0.1).astype(np.float32)
    x = rng.standard_normal(7168).astype(np.float32)
    h_in = rng.standard_normal(7168).astype(np.float32)
    _, ref_out = O.cpu_layer_baseline(blobs, q6, Wg, bias, x, h_in, 1)
    _, tuned_out, threads = O.cpu_layer_tuned(blobs, q6, Wg, bias, x, h_in, 1, n_threads=4)
    assert threads == 4
    idx, w = O.route(O.router_logits(Wg, x), bias, K=K)
    # the baselines run blobs[0..K-1] in the routed slots whatever route() picks
    want = h_in.astype(np.float64)
    for k in range(K):
        want += np.float64(w[k]) * O.expert_ffn(blobs[k], q6, x)
    want += O.expert_ffn(blobs[K], q6, x)
    for got in (ref_out, tuned_out):
        err = np.linalg.norm(got - want) / np.linalg.norm(want)
        assert err <= 1e-5, err
