"""The oracle's dense-layer pieces, pinned on the CPU:

* orc_fp32_to_fp16, the (__fp16) cast of f32_to_f16_alloc
  (infer.m:521-528), against numpy's IEEE binary16 conversion (round to
  nearest even), bit for bit: random bit patterns, every half value, every
  midpoint between neighbouring halves (the ties) and its float neighbours,
  the overflow and subnormal boundaries, signed zeros, infinities and quiet
  NaNs.  Signalling NaNs are where numpy and the reference's host differ
  (numpy does not set the quiet bit); there the oracle follows the host's
  FCVT and nothing outside this repository pins it.
* orc_dense_ffn, the dense branch of layer_forward (infer.m:1852-1868),
  against an independent numpy float64 evaluation (BLAS matmuls) of
  h_in + W_down (silu(W_gate h) * (W_up h)).
"""
import numpy as np


def edge_floats():
    """float32 values at every place a binary16 conversion can go wrong."""
    halves = np.arange(0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)  # +0 .. max finite
    mids = (halves[:-1] + halves[1:]) / 2  # exact in float32 (12 significant bits)
    m32 = mids.astype(np.float32)
    up = np.nextafter(m32, np.float32(np.inf))
    dn = np.nextafter(m32, np.float32(0))
    special = np.array([65504.0, 65519.996, 65520.0, 65536.0, 1e38, 3.4028235e38,
                        2.0 ** -24, 2.0 ** -25, 2.0 ** -26, 2.0 ** -14, 6.1e-5, 1e-30, 1.4e-45,
                        0.0, np.inf], dtype=np.float32)
    special = np.concatenate([special, np.nextafter(special, np.float32(np.inf)),
                              np.nextafter(special, np.float32(0))])
    v = np.concatenate([halves.astype(np.float32), m32, up, dn, special])
    return np.concatenate([v, -v]).astype(np.float32)


def test_fp32_to_fp16_matches_ieee(oracle):
    x = edge_floats()
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.fp32_to_fp16(x), want)


def test_fp32_to_fp16_random_patterns(oracle):
    rng = np.random.default_rng(16)
    x = rng.integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = x[~np.isnan(x)]
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.fp32_to_fp16(x), want)


def test_fp32_to_fp16_quiet_nan(oracle):
    bits = np.array([0x7FC00000, 0xFFC00000, 0x7FC02000, 0x7FFFFFFF, 0xFFE00001], dtype=np.uint32)
    x = bits.view(np.float32)
    got = oracle.fp32_to_fp16(x)
    assert np.array_equal(got, x.astype(np.float16).view(np.uint16))
    assert np.all((got & 0x7E00) == 0x7E00)


def _weights(rng, inter):
    gate = (rng.normal(0, 7168 ** -0.5, (inter, 7168))).astype(np.float16)
    up = (rng.normal(0, 7168 ** -0.5, (inter, 7168))).astype(np.float16)
    down = (rng.normal(0, inter ** -0.5, (7168, inter))).astype(np.float16)
    return gate, up, down


def test_dense_ffn_matches_numpy(oracle):
    rng = np.random.default_rng(3)
    inter = 1024
    gate, up, down = _weights(rng, inter)
    h = rng.normal(0, 1, 7168).astype(np.float32)
    h_in = rng.normal(0, 1, 7168).astype(np.float32)
    got, act = oracle.dense_ffn(gate.view(np.uint16), up.view(np.uint16), down.view(np.uint16), h, h_in,
                                with_act=True)
    g = gate.astype(np.float64) @ h.astype(np.float64)
    u = up.astype(np.float64) @ h.astype(np.float64)
    a = g / (1.0 + np.exp(-g)) * u
    want = h_in.astype(np.float64) + down.astype(np.float64) @ a
    assert np.max(np.abs(act - a)) <= 1e-6 * np.max(np.abs(a))
    assert np.max(np.abs(got - want)) <= 1e-6 * np.max(np.abs(want))
    # no residual: the FFN alone
    alone = oracle.dense_ffn(gate.view(np.uint16), up.view(np.uint16), down.view(np.uint16), h)
    assert np.max(np.abs(alone - (want - h_in))) <= 1e-6 * np.max(np.abs(want - h_in))
    # gate and up play different roles: swapping them changes the result
    swapped = oracle.dense_ffn(up.view(np.uint16), gate.view(np.uint16), down.view(np.uint16), h, h_in)
    assert np.max(np.abs(swapped - want)) > 1e-2 * np.max(np.abs(want))
