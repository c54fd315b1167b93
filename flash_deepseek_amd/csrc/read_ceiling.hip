// read_ceiling.hip -- the streaming ceiling of a batch-1 layer's bytes.
//
// One dependency-free launch that reads exactly what one launch of the
// batch-1 layer kernel reads -- the router weights and bias, the K routed
// experts, the shared expert, h_post and h_in -- with that kernel's load
// policy (16-byte nontemporal loads, ~64 KB per workgroup, four workgroups
// per CU), and writes 7168 words.  Its time is what the device's memory
// system gives for the layer's bytes with no hand-off, no route and no math;
// the layer kernel's time against it separates the device ceiling from the
// kernel's own losses.  Each workgroup sums its bytes (mod 2^32, one dot4
// against ones per word) into one word (sink[tile]); the other sink words
// are written as 0, so the sum of the sink is the sum of every byte read (a
// check of what was read that no byte permutation, such as the resident
// expert layout, changes).
#include "fdm_internal.h"

namespace fdm {
namespace {

constexpr int kTileBytes = 65536;          // bytes per workgroup
constexpr int kVecPerThread = kTileBytes / 16 / 256;

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void k_read_ceiling(
    ReadCeilArgs a) {
  __shared__ uint32_t red[4];
  const int t = blockIdx.x;
  int s = 0;
  while (s + 1 < a.n_seg && a.tile0[s + 1] <= t) ++s;
  const uint8_t* base = a.seg[s];
  if (s >= a.first_routed && s < a.first_routed + a.K) {
    const int e = a.idx[s - a.first_routed];
    base = a.experts + (size_t)(e >= 0 && e < a.n_experts ? e : 0) * a.expert_size;
  }
  const size_t off = (size_t)(t - a.tile0[s]) * kTileBytes;
  const size_t n = a.bytes[s] - off < (size_t)kTileBytes ? a.bytes[s] - off : (size_t)kTileBytes;
  const u32x4* p = reinterpret_cast<const u32x4*>(base + off);
  u32x4 v[kVecPerThread];
#pragma unroll
  for (int j = 0; j < kVecPerThread; ++j) {
    const size_t k = (size_t)j * 256 + threadIdx.x;
    v[j] = k * 16 < n ? __builtin_nontemporal_load(p + k) : u32x4{0u, 0u, 0u, 0u};
  }
  uint32_t x = 0;
#pragma unroll
  for (int j = 0; j < kVecPerThread; ++j) {
    x = __builtin_amdgcn_udot4(v[j].x, 0x01010101u, x, false);
    x = __builtin_amdgcn_udot4(v[j].y, 0x01010101u, x, false);
    x = __builtin_amdgcn_udot4(v[j].z, 0x01010101u, x, false);
    x = __builtin_amdgcn_udot4(v[j].w, 0x01010101u, x, false);
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += (uint32_t)__shfl_xor((int)x, m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    a.sink[t] = (red[0] + red[1]) + (red[2] + red[3]);
    if (t + a.n_tiles < kHidden) a.sink[t + a.n_tiles] = 0u;
  }
}

}  // namespace

int read_ceiling_tiles(size_t bytes) { return (int)((bytes + kTileBytes - 1) / kTileBytes); }

hipError_t launch_read_ceiling(const ReadCeilArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(k_read_ceiling, dim3(a.n_tiles), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace fdm
