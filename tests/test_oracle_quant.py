"""The C restatement of quant.c (oracle/quant_ref.c), pinned against:
  - golden vectors written by the reference's own quant.c (compiled under
    oracle/_ref by oracle/Makefile; see tests/golden/make_golden.py),
  - the reference's own test format (quant_test.c:85-87, %.6f lines),
  - numpy's IEEE half conversion over all 65,536 bit patterns,
  - blocks assembled from the GGML K-quant layout by an independent packer
    with exactly representable values (hand-checkable answers), and
  - the 6-bit scale packing round trip.
"""
import os

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def bits_equal_nan_class(a, b):
    """Bitwise equality of float32 arrays, NaNs compared by class only."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan_a, nan_b = np.isnan(a), np.isnan(b)
    if not np.array_equal(nan_a, nan_b):
        return False
    return np.array_equal(a.view(np.uint32)[~nan_a], b.view(np.uint32)[~nan_b])


def test_fp16_all_patterns_match_golden(oracle, golden):
    ours = oracle.fp16_to_fp32_array(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    # the restatement keeps NaN payloads exactly as quant.c:18-19 does,
    # signalling NaNs included
    assert np.array_equal(ours.view(np.uint32), golden["fp16_out"])
    snan = golden["fp16_out"][0x7C01]
    assert snan == 0x7F802000  # half sNaN 0x7C01 -> float sNaN, payload shifted


def test_fp16_all_patterns_match_ieee(oracle):
    ours = oracle.fp16_to_fp32_array(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    ieee = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    assert bits_equal_nan_class(ours, ieee)
    # subnormals really are renormalised, not flushed
    assert oracle.fp16_to_fp32(0x0001) == 2.0 ** -24
    assert oracle.fp16_to_fp32(0x03FF) == 1023 * 2.0 ** -24
    assert oracle.fp16_to_fp32(0x8001) == -(2.0 ** -24)


def test_q4k_blocks_match_golden(oracle, golden):
    blocks, expect = golden["q4k_blocks"], golden["q4k_out"]
    for i in range(len(blocks)):
        out = oracle.dequant_q4k(blocks[i])
        assert bits_equal_nan_class(out, expect[i].view(np.float32)), f"block {i}"


def test_q6k_blocks_match_golden(oracle, golden):
    blocks, expect = golden["q6k_blocks"], golden["q6k_out"]
    for i in range(len(blocks)):
        out = oracle.dequant_q6k(blocks[i])
        assert bits_equal_nan_class(out, expect[i].view(np.float32)), f"block {i}"


def test_multiblock_rows_match_golden(oracle, golden):
    assert bits_equal_nan_class(oracle.dequant_q4k(golden["q4k_row"]),
                                golden["q4k_row_out"].view(np.float32))
    assert bits_equal_nan_class(oracle.dequant_q6k(golden["q6k_row"]),
                                golden["q6k_row_out"].view(np.float32))


def test_reference_text_format(oracle, golden):
    # quant_test.c prints "%.6f" per value; the reference test diffs that text.
    with open(os.path.join(ROOT, "tests", "golden", "q4k_row_first64.txt")) as f:
        expect = f.read()
    ours = "".join("%.6f\n" % v for v in oracle.dequant_q4k(golden["q4k_row"])[:64])
    assert ours == expect


@pytest.mark.skipif(not os.path.exists(os.path.join(ROOT, "oracle", "_ref", "libquant_ref.so")),
                    reason="reference quant.c not built here")
def test_random_blocks_match_compiled_reference(oracle):
    ref = oracle.load_ref()
    rng = np.random.default_rng(7)
    for trial in range(4):
        raw = rng.integers(0, 256, 144 * 64, dtype=np.uint8)
        out = np.empty(64 * 256, np.float32)
        ref.dequantize_row_q4_K(raw.ctypes.data, out, out.size)
        assert bits_equal_nan_class(oracle.dequant_q4k(raw), out)
        raw6 = rng.integers(0, 256, 210 * 64, dtype=np.uint8)
        ref.dequantize_row_q6_K(raw6.ctypes.data, out, out.size)
        assert bits_equal_nan_class(oracle.dequant_q6k(raw6), out)


# ---- independent packers written from the GGML K-quant layout ----------------------
def pack_scales_q4k(sc, m):
    """Eight 6-bit scales and mins -> the 12 packed bytes."""
    q = np.zeros(12, np.uint8)
    for j in range(4):
        q[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        q[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        q[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return q


def make_q4k(d, dmin, sc, m, q):
    """q: 256 nibbles in element order."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([d], np.float16).view(np.uint8)
    blk[2:4] = np.array([dmin], np.float16).view(np.uint8)
    blk[4:16] = pack_scales_q4k(sc, m)
    for c in range(4):
        for l in range(32):
            blk[16 + 32 * c + l] = q[64 * c + l] | (q[64 * c + 32 + l] << 4)
    return blk


def make_q6k(d, sc, q):
    """q: 256 six-bit values (0..63) in element order; sc: 16 int8."""
    blk = np.zeros(210, np.uint8)
    for e in range(256):
        h, r = divmod(e, 128)
        k, l = divmod(r, 32)
        qi = int(q[e])
        li = 64 * h + l + 32 * (k & 1)
        if k < 2:
            blk[li] |= qi & 15
        else:
            blk[li] |= (qi & 15) << 4
        blk[128 + 32 * h + l] |= (qi >> 4) << (2 * k)
    blk[192:208] = np.asarray(sc, np.int8).view(np.uint8)
    blk[208:210] = np.array([d], np.float16).view(np.uint8)
    return blk


def test_q4k_known_answer(oracle):
    rng = np.random.default_rng(1)
    sc = rng.integers(0, 64, 8)
    m = rng.integers(0, 64, 8)
    q = rng.integers(0, 16, 256)
    out = oracle.dequant_q4k(make_q4k(1.0, 0.5, sc, m, q))
    # d = 1, dmin = 1/2: every value is a small exact number
    expect = np.array([sc[e // 32] * q[e] - 0.5 * m[e // 32] for e in range(256)], np.float32)
    assert np.array_equal(out, expect)


def test_q6k_known_answer(oracle):
    rng = np.random.default_rng(2)
    sc = rng.integers(-128, 128, 16)
    q = rng.integers(0, 64, 256)
    out = oracle.dequant_q6k(make_q6k(1.0, sc, q))
    expect = np.array([sc[e // 16] * (q[e] - 32) for e in range(256)], np.float32)
    assert np.array_equal(out, expect)


def test_q4k_scale_packing_round_trip(oracle):
    # Every one of the 96 bits is used exactly once: packing then decoding
    # recovers any 16 six-bit values (quant.c:26-34).
    rng = np.random.default_rng(3)
    for _ in range(200):
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        blk = make_q4k(1.0, 1.0, sc, m, np.ones(256, np.int64))
        out = oracle.dequant_q4k(blk)
        # element e (sub-block j = e // 32) = sc_j * 1 - m_j
        got = out[::32].astype(np.int64)
        assert np.array_equal(got, sc - m)
        blk0 = make_q4k(1.0, 1.0, sc, m, np.zeros(256, np.int64))
        assert np.array_equal(oracle.dequant_q4k(blk0)[::32].astype(np.int64), -m)


def test_q4k_fused_and_unfused_agree():
    # d is a half (11 significant bits), sc <= 63 (6 bits) and q <= 15 (4
    # bits), so d*sc and d*sc*q are exact in float32: y = d1*q - m1 rounds
    # once whether or not the compiler fuses it into an fma.  Checked over
    # every half d and every (sc, q).
    d = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    for sc in (1, 17, 37, 63):
        d1 = (d * sc).astype(np.float32)
        assert np.array_equal(d1.astype(np.float64), d * sc)
        for q in (3, 7, 11, 13, 15):
            prod = d1.astype(np.float64) * q
            assert np.array_equal(prod.astype(np.float32).astype(np.float64), prod)
