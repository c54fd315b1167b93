"""Device twins of quant.h against the oracle and the reference's golden
vectors: bit-exact (NaNs by class)."""
import numpy as np
import pytest

from tests._helpers import bits_equal_nan_class, empty_f32, say, to_dev, to_host

pytestmark = pytest.mark.gpu


def test_fp16_all_patterns(fdm, golden):
    say("fp16_to_fp32: all 65536 patterns")
    src = to_dev(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    dst = empty_f32(65536)
    fdm.fp16_to_fp32(src, dst)
    assert np.array_equal(to_host(dst).view(np.uint32), golden["fp16_out"])


def test_q4k_golden_blocks(fdm, golden):
    say("dequant_q4k: golden blocks")
    blocks = golden["q4k_blocks"]
    src = to_dev(blocks.reshape(-1))
    dst = empty_f32(blocks.shape[0] * 256)
    fdm.dequantize_row_q4_K(src, dst, blocks.shape[0] * 256)
    out = to_host(dst).reshape(-1, 256)
    for i in range(blocks.shape[0]):
        assert bits_equal_nan_class(out[i], golden["q4k_out"][i].view(np.float32)), i


def test_q6k_golden_blocks(fdm, golden):
    say("dequant_q6k: golden blocks")
    blocks = golden["q6k_blocks"]
    src = to_dev(blocks.reshape(-1))
    dst = empty_f32(blocks.shape[0] * 256)
    fdm.dequantize_row_q6_K(src, dst, blocks.shape[0] * 256)
    out = to_host(dst).reshape(-1, 256)
    for i in range(blocks.shape[0]):
        assert bits_equal_nan_class(out[i], golden["q6k_out"][i].view(np.float32)), i


@pytest.mark.parametrize("kind", ["synthetic", "any_bits"])
def test_large_rows_match_oracle(fdm, oracle, kind):
    nb = 57344 + 3  # one full 2048x7168 matrix plus a ragged tail
    rng = np.random.default_rng(4)
    for q6 in (False, True):
        say(f"dequant large: kind={kind} q6={q6} blocks={nb}")
        bs = 210 if q6 else 144
        if kind == "synthetic":
            raw = oracle.synth_q6k(nb, 77) if q6 else oracle.synth_q4k(nb, 77)
        else:
            raw = rng.integers(0, 256, nb * bs, dtype=np.uint8)
        dst = empty_f32(nb * 256)
        fn = fdm.dequantize_row_q6_K if q6 else fdm.dequantize_row_q4_K
        fn(to_dev(raw), dst, nb * 256)
        want = oracle.dequant_q6k(raw) if q6 else oracle.dequant_q4k(raw)
        assert bits_equal_nan_class(to_host(dst), want)


def test_q6k_source_at_odd_block_offset(fdm, oracle):
    # a Q6_K row slice starting at an odd block: 2-byte aligned source
    raw = oracle.synth_q6k(9, 5)
    src = to_dev(raw)
    dst = empty_f32(8 * 256)
    fdm.dequantize_row_q6_K(src.data_ptr() + 210, dst, 8 * 256)
    assert bits_equal_nan_class(to_host(dst), oracle.dequant_q6k(raw[210:]))


def test_bad_sizes_are_rejected(fdm):
    src = to_dev(np.zeros(144 * 2, np.uint8))
    dst = empty_f32(512)
    with pytest.raises(fdm.FdmError):
        fdm.dequantize_row_q4_K(src, dst, 300)
