"""Seeded synthetic tensors of the benchmark workload (oracle/synth.c):
determinism and the distributions the workload specifies."""
import numpy as np


def test_bytes_deterministic_and_uniform(oracle):
    a = oracle.synth_bytes(1 << 20, 5)
    assert np.array_equal(a, oracle.synth_bytes(1 << 20, 5))
    assert not np.array_equal(a, oracle.synth_bytes(1 << 20, 6))
    counts = np.bincount(a, minlength=256)
    assert counts.min() > 0.9 * a.size / 256 and counts.max() < 1.1 * a.size / 256
    # byte p is byte p % 8 of the 64-bit draw p // 8 (little endian)
    w = oracle.rand_u64(5, 3)
    assert bytes(a[24:32]) == int(w).to_bytes(8, "little")


def test_q4k_scales_are_half_abs_normal(oracle):
    nb = 20000
    raw = oracle.synth_q4k(nb, 9).reshape(nb, 144)
    d = raw[:, 0:2].copy().view(np.float16).astype(np.float64).ravel()
    dmin = raw[:, 2:4].copy().view(np.float16).astype(np.float64).ravel()
    for v in (d, dmin):
        assert (v >= 0).all()
        assert abs(v.mean() - 0.02 * np.sqrt(2 / np.pi)) < 0.03 * 0.016
        assert abs(v.std() - 0.02 * np.sqrt(1 - 2 / np.pi)) < 0.05 * 0.012
    # the qs/scale bytes are untouched uniform bytes
    assert abs(raw[:, 4:].mean() - 127.5) < 1.0


def test_q6k_layout(oracle):
    nb = 20000
    raw = oracle.synth_q6k(nb, 10).reshape(nb, 210)
    d = raw[:, 208:210].copy().view(np.float16).astype(np.float64).ravel()
    assert (d >= 0).all() and abs(d.mean() - 0.02 * np.sqrt(2 / np.pi)) < 0.03 * 0.016
    sc = raw[:, 192:208].view(np.int8)
    assert sc.min() == -128 and sc.max() == 127


def test_normal(oracle):
    x = oracle.synth_normal(200000, 1.0, 0.1, 3)
    assert abs(x.mean() - 1.0) < 1e-3 and abs(x.std() - 0.1) < 1e-3
