// ceilings.hip — what the hardware gives the kernels at most, measured (the counterparts of the reference's CPU
// ceiling loops, kernels/ceilings.ts:12-25 (a read-only loop) and kernels/ceilings_relaxed.ts:34-52 (the dot
// product's rate)):
//   hq_ceiling_read: every byte of a buffer read once (16 bytes a lane a load, a grid-stride walk), the achievable
//                    HBM read bandwidth for a matrix past the caches;
//   hq_ceiling_mfma: v_mfma_i32_32x32x32_i8 on registers only, the achievable dense int8 rate.
#include "common.hpp"
#include "launch.hpp"

namespace hq {

namespace {

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v16i __attribute__((ext_vector_type(16)));

// bytes: a multiple of 16; every lane folds what it read into one word, stored only if it is a value a random
// buffer almost never gives, so that no load can be left out
__global__ __launch_bounds__(256) void read_kernel(const uint4 *p, int64_t n16, uint32_t *sink) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  uint32_t acc = 0;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const uint4 a = p[i], b = p[i + stride], c = p[i + 2 * stride], d = p[i + 3 * stride];
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n16; i += stride) {
    const uint4 a = p[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
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
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  hipLaunchKernelGGL(read_kernel, dim3(cus * 8), dim3(256), 0, s, (const uint4 *)p, bytes / 16, sink);
  return hipGetLastError();
}

hipError_t launch_ceiling_mfma(int32_t blocks, int32_t iterations, int32_t *sink, hipStream_t s) {
  hipLaunchKernelGGL(mfma_kernel, dim3(blocks), dim3(256), 0, s, iterations, sink);
  return hipGetLastError();
}

}  // namespace hq
