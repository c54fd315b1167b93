"""Fused dequant matvecs (fdm_matvec_q4k / _q6k) against the oracle's
bit-exact dequantisation with a float64 dot product.  Tolerance: 1e-3
relative L2 (the bar for floating-point outputs), and fp32 grade: the error
against float64 at most 4x that of the reference's own arithmetic (fp32
products summed in fp32, shaders.metal:93-99), restated by the oracle."""
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
    (False, 37, 1024),     # one-launch column-part path, one part, ragged rows
    (False, 9, 3072),      # three parts
    (False, 100, 5120),
    (False, 45, 7168),     # seven parts, ragged rows
    (False, 3, 2048),
    (True, 5, 4096),       # one-launch Q6_K path, two halves per lane
    (True, 13, 6144),
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


def activations(kind, n, seed):
    """N(0,1); heavy-tailed (a product of normals, a few huge entries); or one
    outlier of +-1e3 in every 32-element sub-block among N(0,1) values."""
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
@pytest.mark.parametrize("q6,rows,cols", [(False, 2048, 7168), (False, 7168, 2048), (True, 7168, 2048)])
def test_matvec_fp32_grade(fdm, oracle, q6, rows, cols, kind):
    """The activation digits keep the dot products at fp32 grade: both the
    relative L2 error and the largest per-row error against float64 stay
    within 4x of the fp32 restatement's."""
    say(f"matvec fp32 grade q6={q6} rows={rows} cols={cols} input={kind}")
    nb = rows * cols // 256
    qt = "q6k" if q6 else "q4k"
    raw = oracle.synth_q6k(nb, 31 + rows) if q6 else oracle.synth_q4k(nb, 31 + rows)
    x = activations(kind, cols, rows + cols)
    got = run(fdm, q6, raw, x, rows, cols).astype(np.float64)
    want = oracle.matvec(raw, x, rows, cols, qt).astype(np.float64)
    f32 = oracle.matvec(raw, x, rows, cols, qt, f32=True).astype(np.float64)
    e_got, e_f32 = rel_l2(got, want), rel_l2(f32, want)
    m_got, m_f32 = np.abs(got - want).max(), np.abs(f32 - want).max()
    print(f"rel_l2 {e_got:.3e} (fp32 {e_f32:.3e}), max {m_got:.3e} (fp32 {m_f32:.3e})")
    assert e_got <= 4 * e_f32
    assert m_got <= 4 * m_f32


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
