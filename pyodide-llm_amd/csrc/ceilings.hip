// ceilings.hip — what the hardware gives the kernels at most, measured (the counterparts of the reference's CPU
// ceiling loops, kernels/ceilings.ts:12-25 (a read-only loop) and kernels/ceilings_relaxed.ts:34-52 (the dot
// product's rate)):
//   hq_ceiling_read: every byte of a buffer read once (4 KB a wave, non-temporal 16-byte loads), the achievable
//                    HBM read bandwidth for a matrix past the caches;
//   hq_ceiling_mfma: v_mfma_i32_32x32x32_i8 on registers only, the achievable dense int8 rate.
#include "common.hpp"
#include "launch.hpp"

namespace hq {

namespace {

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v16i __attribute__((ext_vector_type(16)));

// bytes: a multiple of 16.  Wave w reads the 4 KB at 4096 w: four 16-byte loads a lane, the 64 lanes of a load
// contiguous, all four in flight at once, non-temporal (nothing is read twice).  Every lane folds what it read into
// one word, stored only if it is a value a random buffer almost never gives, so that no load can be left out.
// Measured against the other patterns tried (a grid-stride walk, 1..256 KB a wave, normal loads): the fastest past
// the 256 MB Infinity Cache.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void read_kernel(const uint4 *p, int64_t n16, uint32_t *sink) {
  const int64_t base = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 256 + (threadIdx.x & 63);
  uint32_t acc = 0;
#pragma unroll
  for (int u = 0; u < 4; u++) {
    const int64_t i = base + 64 * u;
    if (i < n16) {
      const u32x4 v = __builtin_nontemporal_load((const u32x4 *)(p + i));
      acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
  }
  if (acc == 0x9e3779b9u) sink[threadIdx.x] = acc;
}

// iterations of 8 independent MFMAs a wave: 8 x 32 x 32 x 32 MACs an iteration
__global__ __launch_bounds__(256) void mfma_kernel(int32_t iterations, int32_t *sink) {
  v4i a, b;
  for (int q = 0; q < 4; q++) {
    a[q] = (int32_t)(threadIdx.x * 2654435761u + q);
    b[q] = (int32_t)(threadIdx.x * 40503u + 7 * q);
  }
  v16i c[8];
  for (int k = 0; k < 8; k++)
    for (int r = 0; r < 16; r++) c[k][r] = 0;
  for (int it = 0; it < iterations; it++) {
#pragma unroll
    for (int k = 0; k < 8; k++) c[k] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c[k], 0, 0, 0);
  }
  int32_t s = 0;
  for (int k = 0; k < 8; k++)
    for (int r = 0; r < 16; r++) s ^= c[k][r];
  if (s == 0x12345678) sink[threadIdx.x] = s;  // keeps the chain; almost never stores
}

}  // namespace

hipError_t launch_ceiling_read(const char *p, int64_t bytes, uint32_t *sink, hipStream_t s) {
  const int64_t blocks = (bytes / 16 + 1023) / 1024;  // 16 KB a block
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(read_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, (const uint4 *)p, bytes / 16, sink);
  return hipGetLastError();
}

hipError_t launch_ceiling_mfma(int32_t blocks, int32_t iterations, int32_t *sink, hipStream_t s) {
  hipLaunchKernelGGL(mfma_kernel, dim3(blocks), dim3(256), 0, s, iterations, sink);
  return hipGetLastError();
}

}  // namespace hq
