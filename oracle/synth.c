/*
 * synth.c -- seeded synthetic tensors for the checker and the CPU baseline.
 * TEST INFRASTRUCTURE ONLY.
 *
 * The same counter-based generator is implemented on the device by the
 * shipped library (fdm_synth_*), so data generated on the GPU can be
 * regenerated here.  Integer streams (uniform bytes) match bit for bit;
 * normal draws use Box-Muller in double and are then rounded to fp16/fp32,
 * so they match except where libm and the device's log/cos differ by an ulp
 * right at a rounding boundary.
 *
 * Distributions (the benchmark workload):
 *   Q4_K block: d, dmin = fp16(|N(0, 0.02)|); 12 scale bytes and 128 qs
 *               bytes uniform (which makes the sixteen 6-bit scales/mins
 *               uniform on 0..63 and the nibbles uniform on 0..15).
 *   Q6_K block: ql, qh uniform bytes; 16 int8 scales uniform on -128..127;
 *               d = fp16(|N(0, 0.02)|).
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

/* splitmix64 finaliser over a Weyl sequence. */
uint64_t orc_rand_u64(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Derived stream seed for a field (e.g. "d" of a Q4_K block). */
static uint64_t sub_seed(uint64_t seed, uint64_t field) { return orc_rand_u64(seed, ~field); }

void orc_synth_bytes(uint8_t *dst, size_t n, uint64_t seed) {
    for (size_t p = 0; p < n; ++p) dst[p] = (uint8_t)(orc_rand_u64(seed, p >> 3) >> (8 * (p & 7)));
}

/* Standard normal number i of stream `seed` (Box-Muller, cosine branch). */
static double std_normal(uint64_t seed, uint64_t i) {
    const double u1 = ((double)(orc_rand_u64(seed, 2 * i) >> 11) + 1.0) * 0x1.0p-53;
    const double u2 = (double)(orc_rand_u64(seed, 2 * i + 1) >> 11) * 0x1.0p-53;
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

void orc_synth_normal(float *dst, size_t n, float mean, float std, uint64_t seed) {
    for (size_t i = 0; i < n; ++i) dst[i] = (float)((double)mean + (double)std * std_normal(seed, i));
}

/* double -> IEEE half, round to nearest even (finite inputs of modest size). */
static uint16_t to_half(double v) {
    uint16_t sign = 0;
    if (v < 0) {
        sign = 0x8000;
        v = -v;
    }
    if (v >= 65520.0) return sign | 0x7C00;
    if (v < 0x1.0p-25) return sign; /* rounds to zero (ties to even at 2^-25) */
    int e;
    double m = frexp(v, &e); /* v = m * 2^e, m in [0.5, 1) */
    int exp_h = e - 1 + 15;  /* biased exponent of v = (2m) * 2^(e-1) */
    if (exp_h <= 0) {
        /* subnormal: units of 2^-24 */
        double q = ldexp(v, 24);
        double r = nearbyint(q); /* default rounding mode is to-nearest-even */
        return sign | (uint16_t)r;
    }
    double frac = ldexp(m, 11); /* in [1024, 2048) */
    double r = nearbyint(frac);
    uint32_t mant = (uint32_t)r;
    if (mant == 2048) {
        mant = 1024;
        ++exp_h;
    }
    if (exp_h >= 31) return sign | 0x7C00;
    return sign | (uint16_t)(exp_h << 10) | (uint16_t)(mant - 1024);
}

void orc_synth_q4k(uint8_t *dst, size_t n_blocks, uint64_t seed) {
    orc_synth_bytes(dst, n_blocks * ORC_Q4K_BLOCK, seed);
    const uint64_t sd = sub_seed(seed, 1);
    for (size_t b = 0; b < n_blocks; ++b) {
        uint16_t d = to_half(fabs(0.02 * std_normal(sd, 2 * b)));
        uint16_t dm = to_half(fabs(0.02 * std_normal(sd, 2 * b + 1)));
        uint8_t *blk = dst + b * ORC_Q4K_BLOCK;
        blk[0] = (uint8_t)d;
        blk[1] = (uint8_t)(d >> 8);
        blk[2] = (uint8_t)dm;
        blk[3] = (uint8_t)(dm >> 8);
    }
}

void orc_synth_q6k(uint8_t *dst, size_t n_blocks, uint64_t seed) {
    orc_synth_bytes(dst, n_blocks * ORC_Q6K_BLOCK, seed);
    const uint64_t sd = sub_seed(seed, 1);
    for (size_t b = 0; b < n_blocks; ++b) {
        uint16_t d = to_half(fabs(0.02 * std_normal(sd, b)));
        uint8_t *blk = dst + b * ORC_Q6K_BLOCK;
        blk[208] = (uint8_t)d;
        blk[209] = (uint8_t)(d >> 8);
    }
}
