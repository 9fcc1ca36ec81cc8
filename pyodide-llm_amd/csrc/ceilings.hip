// ceilings.hip — what the hardware gives the kernels at most, measured (the counterparts of the reference's CPU
// ceiling loops, kernels/ceilings.ts:12-25 (a read-only loop) and kernels/ceilings_relaxed.ts:34-52 (the dot
// product's rate)):
//   hq_ceiling_read: every byte of a buffer read once (4 KB a wave, non-temporal 16-byte loads), the achievable
//                    HBM read bandwidth for a matrix past the caches;
//   hq_ceiling_mfma: v_mfma_i32_32x32x32_i8 on registers only, the achievable dense int8 rate;
//   hq_ceiling_epilogue: the prompt tiles' work per 32 x 32 sub-tile and group on registers only (no loads, no LDS),
//                    two waves a SIMD as the tiles run: the most a tile of that epilogue can give.
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

// The prompt tiles' register work on a wave's four 32 x 32 sub-tiles (two row slices x two token halves, or one slice
// x four halves) and one group, as the tiles issue it:
//   form 0, the bit-exact tile (gemm.hip's q_stage): per slice a correction MFMA (-64 against the weights) and the
//     scales' outer product (v_mfma_f32_32x32x1_2b_f32), per sub-tile a v_mfma_i32_32x32x32_i8 issued one sub-tile
//     ahead of its fold, f(f(C) f(ws xs)) added an output: convert, multiply, add;
//   form 1, the tolerance tile (gemm_tol.hip's group): the slice's weights widened to float16 once, per sub-tile two
//     v_mfma_f32_32x32x16_f16, two outer products, the previous group's fold (its products issued a group ahead), one
//     fused multiply-add an output.
// An iteration is one group: 4 x 65 536 operations (4 sub-tiles of 32 x 32 x 32 multiply-adds); the operands change
// every group so that nothing is hoisted.
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

HQ_DEV void fold_exact(float a[16], const v16i &c, const v32f &sc, int h) {
#pragma unroll
  for (int r = 0; r < 16; r++) a[r] = fadd(a[r], fmul((float)c[r], sc[16 * h + r]));
}
HQ_DEV void fold_tol(float a[16], const v16f &c, const v32f &sc, int h) {
#pragma unroll
  for (int r = 0; r < 16; r++) a[r] = __builtin_fmaf(c[r], sc[16 * h + r], a[r]);
}
HQ_DEV h8 widen(uint32_t d0, uint32_t d1) {
  const h2 minus = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  d0 ^= 0x80808080u;
  d1 ^= 0x80808080u;
  const h2 p0 = __builtin_bit_cast(h2, perm(0x64646464u, d0, 0x05010400u)) + minus;
  const h2 p1 = __builtin_bit_cast(h2, perm(0x64646464u, d0, 0x07030602u)) + minus;
  const h2 p2 = __builtin_bit_cast(h2, perm(0x64646464u, d1, 0x05010400u)) + minus;
  const h2 p3 = __builtin_bit_cast(h2, perm(0x64646464u, d1, 0x07030602u)) + minus;
  return (h8){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

template <int FORM>
__global__ __launch_bounds__(256, 2) void epilogue_kernel(int32_t iterations, int32_t *sink) {
  const int lane = threadIdx.x & 63;
  v4i x0, x1, w0, w1;
  for (int q = 0; q < 4; q++) {
    x0[q] = (int32_t)(threadIdx.x * 2654435761u + q);
    x1[q] = x0[q] ^ 0x5a5a5a5a;
    w0[q] = (int32_t)(threadIdx.x * 40503u + 7 * q);
    w1[q] = w0[q] ^ 0x3c3c3c3c;
  }
  float xs = 1e-3f * (1 + lane), ws0 = 2e-3f * (2 + lane), ws1 = 3e-3f * (1 + lane);
  float acc[4][16];
  for (int i = 0; i < 4; i++)
    for (int r = 0; r < 16; r++) acc[i][r] = 0.0f;
  const v32f z32 = {};
  if (FORM == 0) {
    const v4i m64 = {(int32_t)0xc0c0c0c0, (int32_t)0xc0c0c0c0, (int32_t)0xc0c0c0c0, (int32_t)0xc0c0c0c0};
    const v16i z = {};
    for (int it = 0; it < iterations; it++) {
      x0[0] += 1;
      x1[0] += 3;
      w0 += (v4i){5, 7, 9, 11};
      w1[1] += 13;
      xs += 1.0f;
      const v16i cin0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(m64, w0, z, 0, 0, 0);
      const v32f S0 = __builtin_amdgcn_mfma_f32_32x32x1f32(xs, ws0, z32, 0, 0, 0);
      const v16i C0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(x0, w0, cin0, 0, 0, 0);
      const v16i C1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(x1, w0, cin0, 0, 0, 0);
      const v16i cin1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(m64, w1, z, 0, 0, 0);
      fold_exact(acc[0], C0, S0, 0);
      const v32f S1 = __builtin_amdgcn_mfma_f32_32x32x1f32(xs, ws1, z32, 0, 0, 0);
      const v16i C2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(x0, w1, cin1, 0, 0, 0);
      fold_exact(acc[1], C1, S0, 1);
      const v16i C3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(x1, w1, cin1, 0, 0, 0);
      fold_exact(acc[2], C2, S1, 0);
      fold_exact(acc[3], C3, S1, 1);
    }
  } else {
    v16f P[4] = {};
    v32f S[2] = {};
    for (int it = 0; it < iterations; it++) {
      x0[0] += 1;
      x1[0] += 3;
      w0 += (v4i){5, 7, 9, 11};
      w1[2] += 17;
      xs += 1.0f;
      const h8 k0 = widen((uint32_t)w0[0], (uint32_t)w0[1]), k1 = widen((uint32_t)w0[2], (uint32_t)w0[3]);
      const h8 a[4] = {__builtin_bit_cast(h8, x0), __builtin_bit_cast(h8, x1), __builtin_bit_cast(h8, x0 ^ w1),
                       __builtin_bit_cast(h8, x1 ^ w1)};
      const v16f z = {};
#pragma unroll
      for (int h = 0; h < 4; h++) {  // the four token halves: this group's products, the previous group's fold
        v16f p = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[h], k0, z, 0, 0, 0);
        p = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[(h + 1) & 3], k1, p, 0, 0, 0);
        fold_tol(acc[h], P[h], S[h >> 1], h & 1);
        P[h] = p;
      }
      S[0] = __builtin_amdgcn_mfma_f32_32x32x1f32(xs, ws0, z32, 0, 0, 0);
      S[1] = __builtin_amdgcn_mfma_f32_32x32x1f32(xs + 0.5f, ws0, z32, 0, 0, 0);
    }
  }
  int32_t s = 0;
  for (int i = 0; i < 4; i++)
    for (int r = 0; r < 16; r++) s ^= __float_as_int(acc[i][r]);
  if (s == 0x12345679) sink[threadIdx.x] = s;  // keeps the work; almost never stores
}

}  // namespace

hipError_t launch_ceiling_epilogue(int32_t form, int32_t blocks, int32_t iterations, int32_t *sink, hipStream_t s) {
  if (form == 0) hipLaunchKernelGGL(epilogue_kernel<0>, dim3(blocks), dim3(256), 0, s, iterations, sink);
  else hipLaunchKernelGGL(epilogue_kernel<1>, dim3(blocks), dim3(256), 0, s, iterations, sink);
  return hipGetLastError();
}

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
