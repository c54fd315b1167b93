"""Fused dequant matvecs (fdm_matvec_q4k / _q6k) against the oracle's
bit-exact dequantisation with a float64 dot product.  Tolerance: 1e-3
relative L2 (the bar for floating-point outputs)."""
import numpy as np
import pytest

from tests._helpers import empty_f32, rel_l2, say, to_dev, to_host

pytestmark = pytest.mark.gpu
TOL = 1e-3


def run(fdm, q6, raw, x, rows, cols):
    y = empty_f32(rows)
    fn = fdm.matvec_q6k if q6 else fdm.matvec_q4k
    fn(to_dev(raw), to_dev(x), y, rows, cols)
    return to_host(y)


@pytest.mark.parametrize("q6,rows,cols", [
    (False, 2048, 7168),   # gate/up shape: the single-matvec workload
    (False, 7168, 2048),   # down shape
    (True, 7168, 2048),    # Q6_K down
    (False, 37, 256),      # ragged rows, one block per row
    (False, 21, 1280),     # generic path (5 blocks per row)
    (True, 19, 7168),      # Q6_K generic path (56 halves per row)
    (True, 33, 512),
])
def test_matvec_matches_oracle(fdm, oracle, q6, rows, cols):
    say(f"matvec q6={q6} rows={rows} cols={cols}")
    nb = rows * cols // 256
    raw = oracle.synth_q6k(nb, rows + cols) if q6 else oracle.synth_q4k(nb, rows + cols)
    x = oracle.synth_normal(cols, 0.0, 1.0, 7)
    got = run(fdm, q6, raw, x, rows, cols)
    want = oracle.matvec(raw, x, rows, cols, "q6k" if q6 else "q4k")
    err = rel_l2(got, want)
    print(f"rel_l2={err:.3e}")
    assert err <= TOL


def test_matvec_heavy_tailed_input(fdm, oracle):
    # activations like silu(g)*u: a few huge entries per sub-block
    rows, cols = 512, 2048
    raw = oracle.synth_q4k(rows * cols // 256, 3)
    rng = np.random.default_rng(8)
    x = (rng.standard_normal(cols) * rng.standard_normal(cols) * 300).astype(np.float32)
    x[::97] *= 50
    err = rel_l2(run(fdm, False, raw, x, rows, cols), oracle.matvec(raw, x, rows, cols))
    assert err <= TOL


def test_matvec_zero_input_gives_zero(fdm, oracle):
    raw = oracle.synth_q4k(64 * 28, 2)
    got = run(fdm, False, raw, np.zeros(7168, np.float32), 64, 7168)
    assert np.array_equal(got, np.zeros(64, np.float32))


def test_matvec_special_scales(fdm, oracle):
    # d = 0 / dmin = 0 / subnormal halves in every block
    rows, cols = 16, 2048
    raw = oracle.synth_q4k(rows * 8, 9).reshape(-1, 144).copy()
    raw[0::3, 0:2] = 0                                   # d = 0
    raw[1::3, 2:4] = 0                                   # dmin = 0
    raw[2::3, 0:2] = np.array([0x0007], np.uint16).view(np.uint8)  # subnormal d
    raw = raw.reshape(-1)
    x = oracle.synth_normal(cols, 0.0, 1.0, 10)
    assert rel_l2(run(fdm, False, raw, x, rows, cols), oracle.matvec(raw, x, rows, cols)) <= TOL


def test_matvec_rejects_bad_shapes(fdm):
    W = to_dev(np.zeros(144 * 8, np.uint8))
    x = empty_f32(2048)
    y = empty_f32(8)
    with pytest.raises(fdm.FdmError):
        fdm.matvec_q4k(W, x, y, 8, 2000)
    with pytest.raises(fdm.FdmError):
        fdm.matvec_q4k(W, x, y, 0, 2048)
