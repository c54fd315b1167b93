"""Write the quant golden vectors from the reference's own quant.c.

Run in a container that has the reference tree:  make -C oracle ref  then
python tests/golden/make_golden.py.  It loads oracle/_ref/libquant_ref.so (the
reference's quant.c compiled where it lies, by oracle/Makefile, with
-ffp-contract=off) and records, for crafted and seeded random blocks, the
input bytes and the dequantised outputs, plus fp16_to_fp32 over all 65,536
half-precision bit patterns.  Output: tests/golden/quant_golden.npz (plain
arrays, no pickle).
"""
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import oracle as O  # noqa: E402


def h16(v):
    return int(np.array(v, dtype=np.float16).view(np.uint16))


def q4k_block(d, dmin, scales, qs):
    b = np.zeros(144, dtype=np.uint8)
    b[0:2] = np.array([d], dtype=np.uint16).view(np.uint8)
    b[2:4] = np.array([dmin], dtype=np.uint16).view(np.uint8)
    b[4:16] = scales
    b[16:144] = qs
    return b


def q6k_block(ql, qh, sc, d):
    b = np.zeros(210, dtype=np.uint8)
    b[0:128] = ql
    b[128:192] = qh
    b[192:208] = np.asarray(sc, dtype=np.int8).view(np.uint8)
    b[208:210] = np.array([d], dtype=np.uint16).view(np.uint8)
    return b


def crafted_q4k(rng):
    rs = lambda n: rng.integers(0, 256, n, dtype=np.uint8)  # noqa: E731
    blocks = []
    one, half = h16(1.0), h16(0.5)
    blocks.append(q4k_block(0, 0, rs(12), rs(128)))                      # d = dmin = 0
    blocks.append(q4k_block(h16(0.02), h16(0.01), rs(12), np.zeros(128, np.uint8)))  # qs 0
    blocks.append(q4k_block(h16(0.02), h16(0.01), rs(12), np.full(128, 0xFF, np.uint8)))
    blocks.append(q4k_block(one, half, np.zeros(12, np.uint8), rs(128)))  # sc = m = 0
    blocks.append(q4k_block(one, half, np.full(12, 0xFF, np.uint8), rs(128)))  # sc = m = 63
    blocks.append(q4k_block(0x0001, 0x03FF, rs(12), rs(128)))            # subnormal d, dmin
    blocks.append(q4k_block(0x8001, 0x0200, rs(12), rs(128)))            # negative subnormal
    blocks.append(q4k_block(0x7C00, half, rs(12), rs(128)))              # d = +inf
    blocks.append(q4k_block(one, 0xFC00, rs(12), rs(128)))               # dmin = -inf
    blocks.append(q4k_block(0x7E00, half, rs(12), rs(128)))              # d = NaN
    blocks.append(q4k_block(0x7BFF, 0x7BFF, np.full(12, 0xFF, np.uint8), rs(128)))  # max half
    blocks.append(q4k_block(0x8000, 0x8000, rs(12), rs(128)))            # -0
    blocks.append(q4k_block(h16(-1.0), h16(0.25), rs(12), rs(128)))      # negative d
    # one scale/min byte at a time, to pin the 6-bit packing (quant.c:26-34)
    for j in range(12):
        sc = np.zeros(12, np.uint8)
        sc[j] = 0xFF
        blocks.append(q4k_block(one, half, sc, np.arange(128, dtype=np.uint8)))
    return blocks


def crafted_q6k(rng):
    rs = lambda n: rng.integers(0, 256, n, dtype=np.uint8)  # noqa: E731
    ri8 = lambda n: rng.integers(-128, 128, n)  # noqa: E731
    one = h16(1.0)
    blocks = []
    blocks.append(q6k_block(np.zeros(128, np.uint8), np.zeros(64, np.uint8), ri8(16), one))  # q=-32
    blocks.append(q6k_block(np.full(128, 0xFF, np.uint8), np.full(64, 0xFF, np.uint8), ri8(16),
                            one))                                                  # q=+31
    blocks.append(q6k_block(rs(128), rs(64), np.full(16, -128), one))              # sc=-128
    blocks.append(q6k_block(rs(128), rs(64), np.full(16, 127), one))               # sc=+127
    blocks.append(q6k_block(rs(128), rs(64), ri8(16), 0))                          # d = 0
    blocks.append(q6k_block(rs(128), rs(64), ri8(16), 0x0001))                     # subnormal
    blocks.append(q6k_block(rs(128), rs(64), ri8(16), 0x7C00))                     # +inf
    blocks.append(q6k_block(rs(128), rs(64), ri8(16), 0x7E00))                     # NaN
    blocks.append(q6k_block(rs(128), rs(64), ri8(16), 0x7BFF))                     # max half
    blocks.append(q6k_block(rs(128), rs(64), np.zeros(16), one))                   # sc = 0
    # one qh bit pair at a time (pins which 2 bits feed which quarter)
    for sh in range(4):
        blocks.append(q6k_block(np.arange(128, dtype=np.uint8),
                                np.full(64, 3 << (2 * sh), np.uint8),
                                np.arange(16) - 8, one))
    return blocks


def main():
    ref = O.load_ref()
    if ref is None:
        sys.exit("oracle/_ref/libquant_ref.so missing: run `make -C oracle ref` first")
    rng = np.random.default_rng(20261201)

    q4 = crafted_q4k(rng)
    n_q4_crafted = len(q4)
    q4 += [np.frombuffer(O.synth_q4k(1, 1000 + i).tobytes(), np.uint8) for i in range(24)]
    q4 += [rng.integers(0, 256, 144, dtype=np.uint8) for _ in range(24)]   # any bit pattern
    q4 = np.stack(q4)
    q6 = crafted_q6k(rng)
    n_q6_crafted = len(q6)
    q6 += [np.frombuffer(O.synth_q6k(1, 2000 + i).tobytes(), np.uint8) for i in range(24)]
    q6 += [rng.integers(0, 256, 210, dtype=np.uint8) for _ in range(24)]
    q6 = np.stack(q6)

    q4_out = np.empty((len(q4), 256), np.float32)
    for i, b in enumerate(q4):
        ref.dequantize_row_q4_K(np.ascontiguousarray(b).ctypes.data, q4_out[i], 256)
    q6_out = np.empty((len(q6), 256), np.float32)
    for i, b in enumerate(q6):
        ref.dequantize_row_q6_K(np.ascontiguousarray(b).ctypes.data, q6_out[i], 256)
    # a multi-block row, to pin block stepping
    row4 = np.ascontiguousarray(q4[:28].reshape(-1))
    row4_out = np.empty(28 * 256, np.float32)
    ref.dequantize_row_q4_K(row4.ctypes.data, row4_out, row4_out.size)
    row6 = np.ascontiguousarray(q6[:8].reshape(-1))
    row6_out = np.empty(8 * 256, np.float32)
    ref.dequantize_row_q6_K(row6.ctypes.data, row6_out, row6_out.size)

    # fp16 table from a C harness linked to the reference quant.c: the bits
    # must not pass through a Python float (that would quiet signalling NaNs)
    raw = subprocess.run([O.REF_DUMP], check=True, capture_output=True).stdout
    fp16 = np.frombuffer(raw, dtype=np.float32)
    assert fp16.size == 65536

    np.savez_compressed(
        os.path.join(HERE, "quant_golden.npz"),
        q4k_blocks=q4, q4k_out=q4_out.view(np.uint32), n_q4k_crafted=n_q4_crafted,
        q6k_blocks=q6, q6k_out=q6_out.view(np.uint32), n_q6k_crafted=n_q6_crafted,
        q4k_row=row4, q4k_row_out=row4_out.view(np.uint32),
        q6k_row=row6, q6k_row_out=row6_out.view(np.uint32),
        fp16_out=fp16.view(np.uint32),
    )
    # The reference's own test format (quant_test.c:85-87): first values, %.6f.
    with open(os.path.join(HERE, "q4k_row_first64.txt"), "w") as f:
        for v in row4_out[:64]:
            f.write("%.6f\n" % v)
    print("wrote", len(q4), "Q4_K and", len(q6), "Q6_K blocks")


if __name__ == "__main__":
    main()
