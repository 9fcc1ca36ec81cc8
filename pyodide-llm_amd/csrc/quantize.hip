// quantize.hip — the activations' preparation and the weights' corrections:
//   quantize_x (kernels/kernel/quantize.ts:124-151), interleave (kernels/kernel/matmul.ts:107-146),
//   int8_sums (matmul.ts:50-58), six_sums (matmul.ts:38-46), and the converters' packers quantize6_x, ternary_x,
//   binary_x (quantize.ts:153-247: used at load).
// Byte-for-byte the reference's outputs; small, latency-bound kernels (a token's activations are a few KB).
#include "common.hpp"
#include "launch.hpp"

namespace hq {

// quantize_x: one group of 32 values a half-wave, lane j its value j.  Lane j belongs to WebAssembly lane j % 4 of
// groupMax (quantize.ts:10-19): the maxima of each residue are reduced first (NaN kept), then lanes 1..3 compared
// with lane 0's in order (a NaN there is passed over).
__global__ __launch_bounds__(256) void quantize_kernel(char *xq, char *xs, const char *x, int32_t n, int32_t bias,
                                                       int64_t total_groups, int64_t frame, int64_t x_stride) {
  const int32_t ng = n >> 5;
  const uint32_t gi = blockIdx.x * 8u + (threadIdx.x >> 5);
  const int j = threadIdx.x & 31;
  const bool live = gi < (uint64_t)total_groups;
  const uint32_t gg = live ? gi : 0;
  const uint32_t t = total_groups <= ng ? 0u : gg / (uint32_t)ng;
  const int32_t g = (int32_t)(gg - t * (uint32_t)ng);
  const float v = ((const float *)(x + t * x_stride))[g * GS + j];

  float m = fabsf(v);
  m = wasm_max_abs(m, from_lane_plus<4>(m));  // values 4i + r of this row of 16
  m = wasm_max_abs(m, from_lane_plus<8>(m));
  m = wasm_max_abs(m, __shfl_xor(m, 16, 64));  // and of the other row of the group
  const float m0 = quad_lane<0>(m), m1 = quad_lane<1>(m), m2 = quad_lane<2>(m), m3 = quad_lane<3>(m);
  float amax = m0;
  if (m1 > amax) amax = m1;
  if (m2 > amax) amax = m2;
  if (m3 > amax) amax = m3;

  const float qmax = bias == 0 ? 127.0f : 63.0f;
  const float scale = fdiv(amax, qmax);
  const float inv = scale > 0.0f ? fdiv(1.0f, scale) : 0.0f;
  const int32_t tq = trunc_sat(rintf(fmul(v, inv)));
  int32_t q = (int32_t)((uint32_t)tq + (uint32_t)bias);  // i32x4.add wraps
  q = q > 127 ? 127 : (q < -128 ? -128 : q);             // the two saturating narrowings
  if (live) {
    xq[t * frame + g * GS + j] = (char)(int8_t)q;
    if (j == 0) ((float *)(xs + t * frame))[g] = scale;
  }
}

hipError_t launch_quantize_x(char *xq, char *xs, const char *x, int32_t n, int32_t bias, int32_t count,
                             int64_t frame, int64_t x_stride, hipStream_t s) {
  const int64_t groups = (int64_t)count * (n >> 5);
  if (groups >= (int64_t)1 << 32) return hipErrorInvalidValue;  // the kernel's group index is 32-bit
  const int64_t blocks = (groups + 7) / 8;
  hipLaunchKernelGGL(quantize_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, xq, xs, x, n, bias, groups, frame,
                     x_stride);
  return hipGetLastError();
}

// interleave: one block of 64 activations a thread, in place.  Byte 16 p + c of the block becomes activation
// 4 c + p (byte p of the block's dword c), and after the n / 32 scales come the blocks' two group sums, negated.
__global__ __launch_bounds__(256) void interleave_kernel(char *xq, char *xs, int32_t n, int64_t total_blocks,
                                                         int64_t frame) {
  const int64_t bi = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (bi >= total_blocks) return;
  const int32_t nb = n >> 6;
  const int64_t t = bi / nb;
  const int32_t b = (int32_t)(bi - t * nb);
  uint4 *p = (uint4 *)(xq + t * frame + (int64_t)b * 64);
  const uint4 q0 = p[0], q1 = p[1], q2 = p[2], q3 = p[3];
  const uint32_t d[16] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w,
                          q2.x, q2.y, q2.z, q2.w, q3.x, q3.y, q3.z, q3.w};
  int32_t s0 = 0, s1 = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    s0 = sdot4((int32_t)d[i], 0x01010101, s0);
    s1 = sdot4((int32_t)d[8 + i], 0x01010101, s1);
  }
  uint32_t o[16];
#pragma unroll
  for (int pl = 0; pl < 4; pl++) {
#pragma unroll
    for (int m = 0; m < 4; m++) {
      // bytes c = 4m..4m+3 of plane pl: byte pl of dwords 4m..4m+3
      const uint32_t lo = perm(d[4 * m + 1], d[4 * m], (uint32_t)pl | ((uint32_t)(4 + pl) << 8));
      const uint32_t hi = perm(d[4 * m + 3], d[4 * m + 2], (uint32_t)pl | ((uint32_t)(4 + pl) << 8));
      o[4 * pl + m] = perm(hi, lo, 0x05040100u);
    }
  }
  p[0] = make_uint4(o[0], o[1], o[2], o[3]);
  p[1] = make_uint4(o[4], o[5], o[6], o[7]);
  p[2] = make_uint4(o[8], o[9], o[10], o[11]);
  p[3] = make_uint4(o[12], o[13], o[14], o[15]);
  int32_t *sums = (int32_t *)(xs + t * frame) + (n >> 5);
  sums[2 * b] = -s0;
  sums[2 * b + 1] = -s1;
}

hipError_t launch_interleave(char *xq, char *xs, int32_t n, int32_t count, int64_t frame, hipStream_t s) {
  const int64_t blocks = (int64_t)count * (n >> 6);
  hipLaunchKernelGGL(interleave_kernel, dim3((uint32_t)((blocks + 255) / 256)), dim3(256), 0, s, xq, xs, n, blocks,
                     frame);
  return hipGetLastError();
}

// int8_sums / six_sums: a group a thread, -64 times the sum of its int8 values (exact in int32)
__global__ __launch_bounds__(256) void int8_sums_kernel(int32_t *out, const char *w, int32_t groups) {
  const int32_t g = blockIdx.x * 256 + threadIdx.x;
  if (g >= groups) return;
  const uint4 *p = (const uint4 *)(w + (int64_t)g * 32);
  const uint4 a = p[0], b = p[1];
  int32_t s = 0;
  s = sdot4((int32_t)a.x, 0x01010101, s);
  s = sdot4((int32_t)a.y, 0x01010101, s);
  s = sdot4((int32_t)a.z, 0x01010101, s);
  s = sdot4((int32_t)a.w, 0x01010101, s);
  s = sdot4((int32_t)b.x, 0x01010101, s);
  s = sdot4((int32_t)b.y, 0x01010101, s);
  s = sdot4((int32_t)b.z, 0x01010101, s);
  s = sdot4((int32_t)b.w, 0x01010101, s);
  out[g] = -64 * s;
}

__global__ __launch_bounds__(256) void six_sums_kernel(int32_t *out, const char *w, int32_t groups) {
  const int32_t g = blockIdx.x * 256 + threadIdx.x;
  if (g >= groups) return;
  const uint2 *p = (const uint2 *)(w + (int64_t)g * 24);
  const uint2 a = p[0], b = p[1], c = p[2];
  const uint32_t d[6] = {a.x, a.y, b.x, b.y, c.x, c.y};
  uint32_t v[8];
  six_widen(d, v);
  int32_t s = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) s = sdot4((int32_t)v[i], 0x01010101, s);
  out[g] = -64 * s;
}

// binary_x: a group of 128 values a 16-lane row, lane c its byte c: values 4c..4c+3 (bits 0..3) and 64+4c.. (bits
// 4..7), a bit set where the value is not below 0 (v128.not of f32x4.lt: -0 and NaN too).  The scale is groupLargest's
// (quantize.ts:186-191): the largest |value|, NaN where there is one (a non-negative float's bits order as the float
// does and every NaN's are above +inf's, so the largest bits are the result; which NaN is the engine's choice in
// WebAssembly too).  A value that is not plus or minus it (a NaN never is) makes *bad 1.
__global__ __launch_bounds__(256) void binary_x_kernel(uint8_t *out, float *xs, const float *x, int32_t groups,
                                                       int32_t *bad) {
  const int64_t g = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int c = threadIdx.x & 15;
  const bool live = g < groups;
  const int64_t gg = live ? g : 0;
  const float4 lo = ((const float4 *)(x + gg * 128))[c], hi = ((const float4 *)(x + gg * 128 + 64))[c];
  const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) m = max(m, __float_as_uint(v[i]) & 0x7fffffffu);
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o, 16));
  const float scale = __uint_as_float(m);
  uint32_t byte = 0;
  bool refused = false;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    byte |= (uint32_t)(!(v[i] < 0.0f)) << i;
    refused |= !(fabsf(v[i]) == scale);
  }
  if (live) {
    out[gg * 16 + c] = (uint8_t)byte;
    if (c == 0) xs[gg] = scale;
    if (refused && bad) *bad = 1;
  }
}

hipError_t launch_binary_x(uint8_t *out, float *xs, const float *x, int32_t groups, int32_t *bad, hipStream_t s) {
  if (groups <= 0) return hipSuccess;
  hipLaunchKernelGGL(binary_x_kernel, dim3((groups + 15) / 16), dim3(256), 0, s, out, xs, x, groups, bad);
  return hipGetLastError();
}

// quantize6_x (quantize.ts:161-182): one group of 32 values a half-wave, lane j its value j; groupMax as
// quantize_x's; v = clamp(trunc_sat(nearest(value / scale)), -32, 31) (six(), 158-160), its six bits packed as
// six.ts reads them: byte j < 16 the low nibbles of values j and j + 16, byte 16 + k the top two bits of values k,
// k + 8, k + 16, k + 24 at bits 0, 2, 4, 6; the scale stored / 4
__global__ __launch_bounds__(256) void quantize6_kernel(uint8_t *out, float *xs, const float *x, int32_t groups) {
  const int64_t gi = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
  const int j = threadIdx.x & 31;
  const bool live = gi < groups;
  const int64_t g = live ? gi : 0;
  const float v = x[g * GS + j];
  float m = fabsf(v);
  m = wasm_max_abs(m, from_lane_plus<4>(m));
  m = wasm_max_abs(m, from_lane_plus<8>(m));
  m = wasm_max_abs(m, __shfl_xor(m, 16, 64));
  const float m0 = quad_lane<0>(m), m1 = quad_lane<1>(m), m2 = quad_lane<2>(m), m3 = quad_lane<3>(m);
  float amax = m0;
  if (m1 > amax) amax = m1;
  if (m2 > amax) amax = m2;
  if (m3 > amax) amax = m3;
  const float scale = fdiv(amax, 31.0f);
  const float inv = scale > 0.0f ? fdiv(1.0f, scale) : 0.0f;
  int32_t q = trunc_sat(rintf(fmul(v, inv)));
  q = q > 31 ? 31 : (q < -32 ? -32 : q);
  const uint32_t six = (uint32_t)q & 63u;
  // every lane reads what its byte needs from the lanes of its group (lanes j + 8, j + 16, j + 24 of the half-wave)
  const int base = threadIdx.x & ~31;
  const uint32_t s8 = (uint32_t)__shfl((int)six, base + ((j + 8) & 31), 64);
  const uint32_t s16 = (uint32_t)__shfl((int)six, base + ((j + 16) & 31), 64);
  const uint32_t s24 = (uint32_t)__shfl((int)six, base + ((j + 24) & 31), 64);
  if (live) {
    uint8_t *at = out + g * 24;
    if (j < 16) at[j] = (uint8_t)((six & 15u) | ((s16 & 15u) << 4));
    if (j < 8) at[16 + j] = (uint8_t)((six >> 4) | ((s8 >> 4) << 2) | ((s16 >> 4) << 4) | ((s24 >> 4) << 6));
    if (j == 0) xs[g] = fmul(scale, 0.25f);
  }
}

hipError_t launch_quantize6_x(uint8_t *out, float *xs, const float *x, int32_t groups, hipStream_t s) {
  if (groups <= 0) return hipSuccess;
  hipLaunchKernelGGL(quantize6_kernel, dim3((groups + 7) / 8), dim3(256), 0, s, out, xs, x, groups);
  return hipGetLastError();
}

// ternary_x (quantize.ts:197-225): a group of 128 values a half-wave, lane c its byte c (values 4c..4c+3).  The
// scale is groupLargest's (the largest |value|, NaN where there is one: the largest bits, as binary_x takes it); a
// value's code 1 + (v > 0) - (v < 0) at bits 2 (its place in the four); *bad = 1 where a value is neither 0 nor of
// the scale's size (a NaN never is).
__global__ __launch_bounds__(256) void ternary_x_kernel(uint8_t *out, float *xs, const float *x, int32_t groups,
                                                        int32_t *bad) {
  const int64_t gi = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
  const int c = threadIdx.x & 31;
  const bool live = gi < groups;
  const int64_t g = live ? gi : 0;
  const float4 f = ((const float4 *)(x + g * 128))[c];
  const float v[4] = {f.x, f.y, f.z, f.w};
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) m = max(m, __float_as_uint(v[i]) & 0x7fffffffu);
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o, 32));
  const float scale = __uint_as_float(m);
  uint32_t byte = 0;
  bool refused = false;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    byte |= (1u + (v[i] > 0.0f ? 1u : 0u) - (v[i] < 0.0f ? 1u : 0u)) << (2 * i);
    refused |= !(fabsf(v[i]) == scale || v[i] == 0.0f);
  }
  if (live) {
    out[g * 32 + c] = (uint8_t)byte;
    if (c == 0) xs[g] = scale;
    if (refused && bad) *bad = 1;
  }
}

hipError_t launch_ternary_x(uint8_t *out, float *xs, const float *x, int32_t groups, int32_t *bad, hipStream_t s) {
  if (groups <= 0) return hipSuccess;
  hipLaunchKernelGGL(ternary_x_kernel, dim3((groups + 7) / 8), dim3(256), 0, s, out, xs, x, groups, bad);
  return hipGetLastError();
}

hipError_t launch_int8_sums(int32_t *out, const char *w, int32_t groups, hipStream_t s) {
  hipLaunchKernelGGL(int8_sums_kernel, dim3((groups + 255) / 256), dim3(256), 0, s, out, w, groups);
  return hipGetLastError();
}

hipError_t launch_six_sums(int32_t *out, const char *w, int32_t groups, hipStream_t s) {
  hipLaunchKernelGGL(six_sums_kernel, dim3((groups + 255) / 256), dim3(256), 0, s, out, w, groups);
  return hipGetLastError();
}

}  // namespace hq
