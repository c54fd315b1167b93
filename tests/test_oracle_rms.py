"""The oracle's rms_norm (infer.m:369-374) pinned on the CPU, bit for bit,
against an exact evaluation: the sum of squares as the reference's loop
compiles (one fused multiply-add per element, index order; clang contracts
`ss += x[i]*x[i]` under its default -ffp-contract=on) computed in rational
arithmetic with round-to-nearest-even to binary32 after every step, then
1/sqrtf(ss/d + 1e-6) and x*inv*w in IEEE single precision (numpy float32
scalars).  The unfused order (product rounded first) is computed the same
way and must differ on these inputs, so the test tells the two apart."""
from fractions import Fraction

import numpy as np


def round_f32(q):
    """Fraction -> nearest binary32 value (ties to even), as a float."""
    if q == 0:
        return 0.0
    neg = q < 0
    a = -q if neg else q
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    quantum = Fraction(2) ** (max(e, -126) - 23)
    r = round(a / quantum)  # Fraction.__round__: half to even
    v = float(r * quantum)
    return -v if neg else v


def exact_rms(x, w, fused):
    ss = 0.0
    for v in x.astype(np.float64):
        sq = Fraction(v) * Fraction(v)
        if not fused:
            sq = Fraction(round_f32(sq))
        ss = round_f32(Fraction(ss) + sq)
    f = np.float32
    inv = f(1.0) / np.sqrt(f(ss) / f(x.size) + f(1e-6))
    o = x * inv
    return o * w if w is not None else o


def test_rms_norm_fused_sequential(oracle):
    rng = np.random.default_rng(369)
    differ = 0
    for d, scale in [(7168, 1.0), (7168, 37.0), (1000, 1e-3), (64, 5.0)]:
        x = (rng.normal(0, scale, d)).astype(np.float32)
        w = rng.normal(1, 0.1, d).astype(np.float32)
        got = oracle.rms_norm(x, w)
        want = exact_rms(x, w, fused=True)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), d
        assert np.array_equal(oracle.rms_norm(x).view(np.uint32), exact_rms(x, None, True).view(np.uint32))
        differ += int(not np.array_equal(exact_rms(x, w, fused=False).view(np.uint32), want.view(np.uint32)))
    assert differ >= 1  # the fused and the unfused loop are distinguishable here
