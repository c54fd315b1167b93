"""The C restatement of the router (oracle/moe_ref.c: orc_router_logits,
orc_sigmoidf, orc_route_ex), pinned by:
  - expf against the correctly rounded exp (math.exp, rounded once),
  - sigmoid against the reference's float formula 1/(1+expf(-x)),
  - routing invariants (distinct ids, group limits, weights sum to 2.5),
  - hand-worked examples of the slot order and tie rules of infer.m:920-991,
  - an independent list-based restatement on small inputs full of ties,
  - router logits against a float64 dot product.
"""
import math

import numpy as np
import pytest


def f32(x):
    return float(np.float32(x))


def ulp_diff(a, b):
    ai = np.array([a], np.float32).view(np.int32)[0]
    bi = np.array([b], np.float32).view(np.int32)[0]
    return abs(int(ai) - int(bi))


def test_expf_is_correctly_rounded(oracle):
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.uniform(-100, 88, 20000), rng.normal(0, 3, 20000),
                         [0.0, -0.0, 1.0, -1.0, 88.7, -103.9, -87.3, 1e-8, -1e-8]])
    exact = 0
    for x in xs.astype(np.float32):
        got = oracle.expf(float(x))
        ref = f32(math.exp(float(x)))
        assert ulp_diff(got, ref) <= 1, x
        exact += got == ref
    assert exact >= len(xs) - 2
    assert oracle.expf(100.0) == math.inf and oracle.expf(-200.0) == 0.0
    assert math.isnan(oracle.expf(float("nan")))


def test_sigmoid_is_the_float_formula(oracle):
    rng = np.random.default_rng(1)
    for x in rng.normal(0, 4, 5000).astype(np.float32):
        e = np.float32(math.exp(-float(x)))  # correctly rounded expf(-x)
        ref = np.float32(1.0) / (np.float32(1.0) + e)
        assert oracle.sigmoidf(float(x)) == float(ref)


# ---- an independent restatement of infer.m:920-991 on Python lists --------------
def route_lists(choice, score, n_group, topk_group, K, scale=2.5):
    n = len(choice)
    per = n // n_group
    gscore = []
    for g in range(n_group):
        vals = [v for v in choice[g * per:(g + 1) * per] if v > -1e30]
        vals = sorted(vals, reverse=True) + [-1e30, -1e30]
        gscore.append(f32(f32(vals[0]) + f32(vals[1])))
    chosen = []
    for _ in range(topk_group):
        cands = [g for g in range(n_group) if g not in chosen and gscore[g] > -1e30]
        if not cands:
            break
        best = max(gscore[g] for g in cands)
        chosen.append(min(g for g in cands if gscore[g] == best))
    masked = [choice[i] if i // per in chosen else -1e30 for i in range(n)]
    keys, ids = [-1e30] * K, [0] * K
    for i, v in enumerate(masked):
        low = min(keys)
        slot = keys.index(low)          # first slot holding the minimum
        if v > low:
            keys[slot], ids[slot] = v, i
    w = [score[i] for i in ids]
    s = np.float32(0)
    for x in w:
        s = np.float32(s + np.float32(x))
    if s > 0:
        f = np.float32(np.float32(scale) / s)
        w = [float(np.float32(np.float32(x) * f)) for x in w]
    return ids, w


def run_route(oracle, logits, bias, K, n_group, topk_group):
    logits = np.asarray(logits, np.float32)
    bias = np.asarray(bias, np.float32)
    idx, w = oracle.route(logits, bias, K=K, n_group=n_group, topk_group=topk_group)
    score = [oracle.sigmoidf(float(x)) for x in logits]
    choice = [f32(np.float32(s) + b) for s, b in zip(score, bias)]
    return list(idx), list(w), score, choice


def test_slot_order_hand_example(oracle):
    # K=2, one group: choices in index order 1, 5, 3, 7 (as sigmoid inputs).
    # i0 -> slot 0; i1 -> slot 1 (empty slot is the minimum); i2=3 beats the
    # minimum 1 in slot 0; i3=7 beats the minimum 3, again slot 0.
    logits = [-2.0, 1.0, 0.0, 2.0]
    idx, _, _, _ = run_route(oracle, logits, [0, 0, 0, 0], K=2, n_group=1, topk_group=1)
    assert idx == [3, 1]


def test_slot_tie_replaces_first_minimum(oracle):
    # equal keys 5, 5 in slots 0 and 1: a larger value replaces slot 0
    idx, _, _, _ = run_route(oracle, [1.0, 1.0, 2.0, -5.0], [0] * 4, K=2, n_group=1,
                             topk_group=1)
    assert idx == [2, 1]


def test_equal_value_does_not_displace(oracle):
    # strict >: a later expert equal to the minimum never enters
    idx, _, _, _ = run_route(oracle, [1.0, 2.0, 1.0, 1.0], [0] * 4, K=2, n_group=1,
                             topk_group=1)
    assert idx == [0, 1]


def test_group_tie_lowest_index_wins(oracle):
    # 4 groups of 2; groups 1 and 3 tie for the single slot left after group 0
    logits = [3.0, 3.0, 1.0, 1.0, -4.0, -4.0, 1.0, 1.0]
    idx, _, _, _ = run_route(oracle, logits, [0] * 8, K=2, n_group=4, topk_group=2)
    # groups 0 and 1 selected: experts 0..3; top 2 are experts 0 and 1
    assert sorted(idx) == [0, 1]
    idx, _, _, _ = run_route(oracle, logits, [0] * 8, K=4, n_group=4, topk_group=2)
    assert sorted(idx) == [0, 1, 2, 3]


def test_bias_steers_selection_but_not_weights(oracle):
    logits = np.zeros(256, np.float32)
    bias = np.zeros(256, np.float32)
    bias[200:208] = 1.0  # group 6 gets every pick
    idx, w = oracle.route(logits, bias, K=8)
    assert sorted(idx) == list(range(200, 208))
    # unbiased scores are all sigmoid(0) = 0.5: weights are 2.5 / 8
    assert np.allclose(w, 2.5 / 8, rtol=0, atol=1e-7)


@pytest.mark.parametrize("seed", range(40))
def test_matches_list_restatement_with_ties(oracle, seed):
    rng = np.random.default_rng(100 + seed)
    n_group, per = 4, 4
    n = n_group * per
    # few distinct values: ties everywhere, also across groups
    logits = rng.choice([-1.0, 0.0, 0.5, 1.0], n).astype(np.float32)
    bias = rng.choice([0.0, 0.25], n).astype(np.float32)
    K = int(rng.integers(1, 7))
    idx, w, score, choice = run_route(oracle, logits, bias, K, n_group, 2)
    ids2, w2 = route_lists(choice, score, n_group, 2, K)
    assert idx == ids2
    assert np.array_equal(np.float32(w), np.float32(w2))


@pytest.mark.parametrize("seed", range(20))
def test_r1_invariants(oracle, seed):
    rng = np.random.default_rng(seed)
    logits = rng.normal(0, 1, 256).astype(np.float32)
    bias = rng.normal(0, 0.1, 256).astype(np.float32)
    idx, w, score, choice = run_route(oracle, logits, bias, 8, 8, 4)
    assert len(set(idx)) == 8
    choice = np.array(choice, np.float32)
    g = choice.reshape(8, 32)
    gs = np.sort(g, axis=1)[:, -2:].sum(axis=1)
    top_groups = sorted(np.argsort(-gs, kind="stable")[:4])
    assert sorted({i // 32 for i in idx}) <= top_groups
    mask = np.full(256, -np.inf, np.float32)
    for gg in top_groups:
        mask[32 * gg:32 * gg + 32] = choice[32 * gg:32 * gg + 32]
    assert sorted(idx) == sorted(np.argsort(-mask, kind="stable")[:8].tolist())
    assert abs(sum(w) - 2.5) < 1e-5
    ws = np.array([score[i] for i in idx], np.float64)
    assert np.allclose(w, ws / ws.sum() * 2.5, rtol=1e-6)
    # agreement with the list restatement on the full R1 shape as well
    ids2, w2 = route_lists(list(choice), score, 8, 4, 8)
    assert idx == ids2 and np.array_equal(np.float32(w), np.float32(w2))


def test_router_logits_close_to_f64(oracle):
    rng = np.random.default_rng(5)
    Wg = rng.normal(0, 0.01, (256, 7168)).astype(np.float32)
    x = rng.normal(0, 1, 7168).astype(np.float32)
    got = oracle.router_logits(Wg, x)
    ref = Wg.astype(np.float64) @ x.astype(np.float64)
    assert np.max(np.abs(got - ref)) < 1e-5 * np.max(np.abs(ref)) + 1e-6


def test_router_logits_order_is_blocked(oracle):
    # The summation order is the blocked one (partial t holds the float4
    # chunks t, t+256, ...), not a plain column loop.  Columns 4 and 1028
    # (chunks 1 and 257) share partial 1, so their two 2^-24 terms meet
    # first and survive as 2^-23 when added to the 1.0 of partial 0; a
    # sequential loop would lose each 2^-24 against 1.0 (ties to even).
    Wg = np.zeros((1, 2048), np.float32)
    x = np.ones(2048, np.float32)
    Wg[0, 0] = 1.0
    Wg[0, 4] = 2.0 ** -24
    Wg[0, 1028] = 2.0 ** -24
    got = oracle.router_logits(Wg, x)[0]
    assert got == np.float32(1.0 + 2.0 ** -23)
    seq = np.float32(0)
    for v in Wg[0]:
        seq = np.float32(seq + v)
    assert seq == np.float32(1.0)
