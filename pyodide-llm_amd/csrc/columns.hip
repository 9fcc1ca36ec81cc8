// columns.hip — the classifier's outlier channels (src/runtime/forward/engine.ts:459-466, tensors.ts:170-187,
// kernels/kernel/matmul.ts:246-266): the channels of the classifier's input taken apart before quantize_x, their
// columns of the packed classifier widened to float32 once at load, and add_columns, which adds their products to the
// logits in float32.
#include "common.hpp"
#include "launch.hpp"

namespace hq {

namespace {

// matmul.ts:248-266: y[j] = (..((y[j] + f(a[0] rows[0][j])) + f(a[1] rows[1][j])) ..) — the reference's four-wide
// and scalar loops add in this one order.  A thread a column j; a wave reads 256 contiguous bytes of each row.  The
// rows' values are loaded 8 at a time before they are added (the loads in flight together, the sums in order).
__global__ __launch_bounds__(256) void add_columns_kernel(float *y, const float *rows, const float *a, int32_t count,
                                                          int32_t n) {
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= n) return;
  float acc = y[j];
  for (int32_t c0 = 0; c0 < count; c0 += 8) {
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = c0 + k < count ? rows[(int64_t)(c0 + k) * n + j] : 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++)
      if (c0 + k < count) acc = fadd(acc, fmul(a[c0 + k], v[k]));
  }
  y[j] = acc;
}

// a packed weight as the integer it holds (jobs.ts:398-433, each packing's value()): weight i of the tensor at v
HQ_DEV int32_t packed_value(int32_t packing, const uint8_t *v, int64_t i) {
  switch (packing) {
  case kPackInt6: {  // 32 weights in 24 bytes: low nibbles, then the top two bits of four (six.ts:1-11)
    const uint8_t *g = v + (i >> 5) * 24;
    const int j = (int)(i & 31);
    const uint32_t low = j < 16 ? g[j] & 15u : g[j - 16] >> 4;
    const uint32_t top = (g[16 + (j & 7)] >> (2 * (j >> 3))) & 3u;
    return (int32_t)(int8_t)(uint8_t)((low | (top << 4)) << 2);
  }
  case kPackTernary: return (int32_t)((v[i >> 2] >> (2 * (i & 3))) & 3u) - 1;
  case kPackBinary:
    return (int32_t)(((v[((i >> 7) << 4) + ((i >> 2) & 15)] >> ((((i >> 6) & 1) << 2) | (i & 3))) & 1u) << 1) - 1;
  default: return (int32_t)(int8_t)v[i];
  }
}

// tensors.ts:175-186: columns[i][w] = f(value(w dim + c_i) scale(w groups + c_i / group)) for every word w of the
// vocabulary; a thread a (channel, word)
__global__ __launch_bounds__(256) void outlier_columns_kernel(float *columns, const uint8_t *values,
                                                              const uint8_t *scales, int32_t packing, Channels ch,
                                                              int32_t vocab, int32_t dim, int32_t group) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= (int64_t)ch.count * vocab) return;
  const int32_t i = (int32_t)(e / vocab), w = (int32_t)(e - (int64_t)i * vocab), c = ch.c[i];
  const int64_t g = (int64_t)w * (dim / group) + c / group;
  const float scale = packing == kPackTernary || packing == kPackBinary
                          ? half_to_float(((const uint16_t *)scales)[g])
                          : ((const float *)scales)[g];
  columns[e] = fmul((float)packed_value(packing, values, (int64_t)w * dim + c), scale);
}

// engine.ts:461-464: picked[i] = x[c_i], then x[c_i] = 0, channel by channel in order
__global__ void take_channels_kernel(float *picked, float *x, Channels ch) {
  if (threadIdx.x != 0) return;
  for (int32_t i = 0; i < ch.count; i++) {
    picked[i] = x[ch.c[i]];
    x[ch.c[i]] = 0.0f;
  }
}

}  // namespace

hipError_t launch_add_columns(float *y, const float *rows, const float *a, int32_t count, int32_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(add_columns_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s, y, rows, a, count, n);
  return hipGetLastError();
}

hipError_t launch_outlier_columns(float *columns, const uint8_t *values, const uint8_t *scales, int32_t packing,
                                  const Channels &ch, int32_t vocab, int32_t dim, int32_t group, hipStream_t s) {
  const int64_t total = (int64_t)ch.count * vocab;
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL(outlier_columns_kernel, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, s, columns, values,
                     scales, packing, ch, vocab, dim, group);
  return hipGetLastError();
}

hipError_t launch_take_channels(float *picked, float *x, const Channels &ch, hipStream_t s) {
  if (ch.count <= 0) return hipSuccess;
  hipLaunchKernelGGL(take_channels_kernel, dim3(1), dim3(64), 0, s, picked, x, ch);
  return hipGetLastError();
}

}  // namespace hq
