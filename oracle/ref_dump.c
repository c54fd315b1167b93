/*
 * ref_dump.c -- writes fp16_to_fp32 of all 65,536 half bit patterns, as raw
 * little-endian float32 bits, to stdout.  Linked by oracle/Makefile against
 * the reference's own quant.c (into _ref/ref_dump) so that the golden table
 * is produced without any value passing through another language's float
 * type (a float -> double conversion would quiet signalling NaNs).
 */
#include <stdint.h>
#include <stdio.h>

float fp16_to_fp32(uint16_t h);

int main(void) {
    static float out[65536];
    for (uint32_t h = 0; h < 65536; ++h) out[h] = fp16_to_fp32((uint16_t)h);
    return fwrite(out, sizeof(float), 65536, stdout) == 65536 ? 0 : 1;
}
