/*
 * quant_ref.c -- CPU restatement of the GGML K-quant block decoders used by
 * the reference (quant.c).  TEST INFRASTRUCTURE ONLY: this is the checker
 * the HIP kernels are compared with; the shipped library never calls it.
 *
 * Contraction.  quant.c:55-56 writes y = d1 * q - m1.  Because d is a half
 * (11 significant bits), sc <= 63 and q <= 15, the products d * sc and
 * d1 * q are exact in single precision, so the result rounds once whether
 * or not a compiler fuses the multiply and subtract: the reference's clang
 * build, gguf-py's numpy decoder (gen_reference.py:35-37) and this file
 * agree bit for bit.  The directory is still built with -ffp-contract=off
 * so that every other expression rounds as written.
 *
 * Pinned by: the golden vectors that tests/golden/make_golden.py writes from
 * the reference's own quant.c compiled under oracle/_ref, the exhaustive
 * 65,536-input fp16 check against numpy's float16 conversion, and the
 * packing round trip of the 6-bit scales (tests/test_oracle_quant.py).
 */
#include "oracle.h"

#include <string.h>

/* quant.c:4-24.  Exact IEEE half -> single, including subnormals (which are
 * renormalised) and inf/NaN (payload kept, shifted into the top mantissa). */
float orc_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t f = h & 0x3FFu;
    uint32_t bits;
    if (e == 0x1Fu) {
        bits = sign | 0x7F800000u | (f << 13);
    } else if (e != 0) {
        bits = sign | ((e + 112u) << 23) | (f << 13); /* rebias 15 -> 127 */
    } else if (f == 0) {
        bits = sign;
    } else {
        /* value = f * 2^-24; shift the leading one up to bit 10 */
        uint32_t shift = 0;
        while ((f & 0x400u) == 0) {
            f <<= 1;
            ++shift;
        }
        bits = sign | ((113u - shift) << 23) | ((f & 0x3FFu) << 13);
    }
    float out;
    memcpy(&out, &bits, sizeof out);
    return out;
}

/* Array form of the above (keeps signalling NaN payloads intact, which a
 * per-value call through a double-returning binding would not). */
void orc_fp16_to_fp32_array(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = orc_fp16_to_fp32(src[i]);
}

/* quant.c:26-34.  Twelve bytes hold eight 6-bit scales and eight 6-bit
 * mins.  Sub-blocks 0-3 keep theirs in the low six bits of bytes 0-3
 * (scale) and 4-7 (min); sub-blocks 4-7 take their low four bits from the
 * nibbles of bytes 8-11 and their top two bits from the spare top bits of
 * bytes 0-3 (scale) and 4-7 (min). */
void orc_get_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = (uint8_t)(q[j] & 0x3F);
        *m = (uint8_t)(q[4 + j] & 0x3F);
    } else {
        uint8_t packed = q[4 + j]; /* bytes 8..11 */
        *sc = (uint8_t)((packed & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((packed >> 4) | ((q[j] >> 6) << 4));
    }
}

static uint16_t load_le16(const uint8_t *p) { return (uint16_t)(p[0] | ((uint16_t)p[1] << 8)); }

/* quant.c:36-61.  Block = [d f16][dmin f16][12 scale bytes][128 qs bytes].
 * For each 64-element chunk c, byte qs[32c + l] holds element 64c + l in
 * its low nibble (sub-block 2c) and element 64c + 32 + l in its high nibble
 * (sub-block 2c + 1); value = (d * sc) * q - dmin * m. */
void orc_dequantize_row_q4_K(const void *src, float *dst, size_t n) {
    const uint8_t *blk = (const uint8_t *)src;
    for (size_t b = 0; b < n / ORC_QK_K; ++b, blk += ORC_Q4K_BLOCK) {
        const float d = orc_fp16_to_fp32(load_le16(blk));
        const float dmin = orc_fp16_to_fp32(load_le16(blk + 2));
        const uint8_t *scales = blk + 4;
        float *y = dst + b * ORC_QK_K;
        for (int c = 0; c < 4; ++c) {
            uint8_t sc_lo, m_lo, sc_hi, m_hi;
            orc_get_scale_min_k4(2 * c, scales, &sc_lo, &m_lo);
            orc_get_scale_min_k4(2 * c + 1, scales, &sc_hi, &m_hi);
            const float mul_lo = d * (float)sc_lo, sub_lo = dmin * (float)m_lo;
            const float mul_hi = d * (float)sc_hi, sub_hi = dmin * (float)m_hi;
            const uint8_t *qs = blk + 16 + 32 * c;
            for (int l = 0; l < 32; ++l) {
                y[64 * c + l] = mul_lo * (float)(qs[l] & 0x0F) - sub_lo;
                y[64 * c + 32 + l] = mul_hi * (float)(qs[l] >> 4) - sub_hi;
            }
        }
    }
}

/* quant.c:63-92.  Block = [ql 128][qh 64][16 int8 scales][d f16].  Each
 * 128-element half h uses ql[64h .. 64h+63], qh[32h .. 32h+31] and scales
 * [8h .. 8h+7].  For l < 32 the four values l, l+32, l+64, l+96 of the half
 * take the low nibble of ql[l], the low nibble of ql[l+32], the high nibble
 * of ql[l] and the high nibble of ql[l+32], each with two bits of qh[l]
 * (bits 0-1, 2-3, 4-5, 6-7) on top, minus 32.  Scale index = l/16 + 2*k for
 * the k-th of the four values.  value = (d * sc) * q. */
void orc_dequantize_row_q6_K(const void *src, float *dst, size_t n) {
    const uint8_t *blk = (const uint8_t *)src;
    for (size_t b = 0; b < n / ORC_QK_K; ++b, blk += ORC_Q6K_BLOCK) {
        const float d = orc_fp16_to_fp32(load_le16(blk + 208));
        float *y = dst + b * ORC_QK_K;
        for (int h = 0; h < 2; ++h) {
            const uint8_t *ql = blk + 64 * h;
            const uint8_t *qh = blk + 128 + 32 * h;
            const int8_t *sc = (const int8_t *)(blk + 192 + 8 * h);
            float *yh = y + 128 * h;
            for (int l = 0; l < 32; ++l) {
                const int s = l / 16;
                const int q0 = ((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q1 = ((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q2 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q3 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                yh[l] = d * (float)sc[s] * (float)q0;
                yh[l + 32] = d * (float)sc[s + 2] * (float)q1;
                yh[l + 64] = d * (float)sc[s + 4] * (float)q2;
                yh[l + 96] = d * (float)sc[s + 6] * (float)q3;
            }
        }
    }
}
