// planes_device.h -- the grouped GEMMs' activation planes, per row: s = the
// power of two that puts the row's largest |x| in [2^13, 2^14), x' = x * 2^s
// split into P fp16 planes (round to nearest, each the rounding of what the
// previous planes left), xs[sb] = the fp32 sum over the 32-element
// sub-block of the planes' values, xe = 2^-s.  Planes: [P][n_rows][kd], each
// run of 8 elements stored in the order 0 2 1 3 4 6 5 7 (the order of the
// GEMM's weight operand).  One thread converts one sub-block held in
// registers.
#pragma once
#include "fdm_device.h"

namespace fdm {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// s of a row whose largest |x| is amax (0 for an all-zero or non-finite row).
__device__ __forceinline__ int planes_shift(float amax) {
  int s = 0;
  if (amax > 0.0f && amax <= 3.4028234e38f) {
    int E;
    (void)frexpf(amax, &E);  // amax in [2^(E-1), 2^E)
    s = 14 - E;
  }
  return s;
}

__device__ __forceinline__ float subblock_absmax(const f32x4 (&v)[8]) {
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    m = fmaxf(m, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
  return m;
}

// Sub-block v (32 consecutive elements of a row) into the planes: dst points
// at the sub-block's first element in plane 0, plane p lies p * plane
// elements further; returns the sub-block's sum of the planes' values.
template <int P>
__device__ __forceinline__ float planes_subblock(const f32x4 (&v)[8], int s, _Float16* dst, size_t plane) {
  float sum = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    _Float16 h[P][8];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const f32x4 a = v[2 * q + u];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float r = ldexpf(a[e], s);
        float tot = 0.0f;
#pragma unroll
        for (int p = 0; p < P; ++p) {
          const _Float16 hp = (_Float16)r;
          h[p][4 * u + e] = hp;
          r -= (float)hp;
          tot += (float)hp;
        }
        sum += tot;
      }
    }
#pragma unroll
    for (int p = 0; p < P; ++p)
      *reinterpret_cast<f16x8*>(dst + (size_t)p * plane + 8 * q) =
          (f16x8){h[p][0], h[p][2], h[p][1], h[p][3], h[p][4], h[p][6], h[p][5], h[p][7]};
  }
  return sum;
}

}  // namespace fdm
