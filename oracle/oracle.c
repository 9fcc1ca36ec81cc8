/* oracle.c — TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * A scalar restatement of the reference's kernels in their float32 order.  Built with -ffp-contract=off and no
 * fast-math, so every float operation below is one IEEE binary32 operation rounded to nearest-even, as WebAssembly's
 * f32 / f32x4 operations are.  Integer sums are computed as the WASM SIMD instructions compute them (including the
 * int16 pair sums of kernels/kernel/matmul.ts:68-72 and the wrap of i32x4.add in quantize_x).
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <string.h>
#include <time.h>

#define GS 32 /* kernels/kernel/math.ts:4 */

/* ---- helpers ------------------------------------------------------------------------------------------------ */

/* f32x4.max lane semantics: NaN if either operand is NaN, and -0 below +0 (kernels/kernel/quantize.ts:10-19) */
static float wasm_max(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  if (a == b) return signbit(a) ? b : a;
  return a > b ? a : b;
}

/* i32x4.trunc_sat_f32x4_s: NaN -> 0, saturating at the int32 ends */
static int32_t trunc_sat(float v) {
  if (v != v) return 0;
  if (v >= 2147483648.0f) return INT32_MAX;
  if (v <= -2147483648.0f) return INT32_MIN;
  return (int32_t)v;
}

static int32_t wrap16(int32_t v) { return (int32_t)(int16_t)(uint16_t)(uint32_t)v; }

/* kernels/kernel/halves.ts:6-23: ((h sign-extended) << 13 & 0x8fffffff) as float, times 2^112 */
float o_half(uint16_t h) {
  int32_t bits = ((int32_t)(int16_t)h * 8192) & (int32_t)0x8fffffff;
  float f;
  memcpy(&f, &bits, 4);
  return f * 5.192296858534828e33f;
}

/* ---- quantize_x: kernels/kernel/quantize.ts:124-151 --------------------------------------------------------- */
void o_quantize_x(void *xq_, float *xs, const float *x, int32_t n, int32_t bias) {
  uint8_t *xq = (uint8_t *)xq_;
  const float qmax = bias == 0 ? 127.0f : 63.0f;
  for (int32_t g = 0; g < n; g += GS) {
    /* groupMax (quantize.ts:10-19): lane j holds the max over values 4i + j, then lanes 1..3 compared in order */
    float m[4];
    for (int j = 0; j < 4; j++) {
      float v = fabsf(x[g + j]);
      for (int i = 1; i < 8; i++) v = wasm_max(v, fabsf(x[g + 4 * i + j]));
      m[j] = v;
    }
    float amax = m[0];
    if (m[1] > amax) amax = m[1];
    if (m[2] > amax) amax = m[2];
    if (m[3] > amax) amax = m[3];
    const float scale = amax / qmax;
    xs[g / GS] = scale;
    const float inv = scale > 0 ? 1.0f / scale : 0.0f;
    for (int j = 0; j < GS; j++) {
      const float p = x[g + j] * inv;
      const int32_t t = trunc_sat(rintf(p));
      int32_t q = (int32_t)((uint32_t)t + (uint32_t)bias); /* i32x4.add wraps */
      if (q > 127) q = 127;                                /* narrow i32->i16->i8 with saturation */
      if (q < -128) q = -128;
      xq[g + j] = (uint8_t)(int8_t)q;
    }
  }
}

/* ---- corrections: kernels/kernel/matmul.ts:38-58 ------------------------------------------------------------ */
void o_int8_sums(int32_t *out, const int8_t *w, int32_t groups) {
  for (int32_t g = 0; g < groups; g++) {
    int32_t s = 0;
    for (int j = 0; j < GS; j++) s += w[(int64_t)g * GS + j];
    out[g] = -64 * s;
  }
}

/* kernels/six.ts:1-31, layout of src/python/engine/packing.py:56-70: value j's low nibble in byte j (j < 16) or the
 * high nibble of byte j - 16; its top two bits at bits 2 (j / 8) of byte 16 + j % 8; the int8 is the six bits << 2 */
void o_six_unpack(int8_t *out, const uint8_t *p) {
  for (int j = 0; j < 32; j++) {
    const int low = j < 16 ? (p[j] & 15) : (p[j - 16] >> 4);
    const int top = (p[16 + (j & 7)] >> (2 * (j >> 3))) & 3;
    out[j] = (int8_t)(uint8_t)((low | (top << 4)) << 2);
  }
}

void o_six_sums(int32_t *out, const uint8_t *w, int32_t groups) {
  int8_t v[32];
  for (int32_t g = 0; g < groups; g++) {
    o_six_unpack(v, w + (int64_t)g * 24);
    int32_t s = 0;
    for (int j = 0; j < 32; j++) s += v[j];
    out[g] = -64 * s;
  }
}

/* ---- interleave: kernels/kernel/matmul.ts:107-146 ----------------------------------------------------------- */
void o_interleave(int8_t *xq, float *xs, int32_t n) {
  int32_t *sums = (int32_t *)(xs + (n >> 5));
  int8_t a[64];
  for (int32_t b = 0; b < n; b += 64) {
    memcpy(a, xq + b, 64);
    int32_t s0 = 0, s1 = 0;
    for (int j = 0; j < 32; j++) s0 += a[j];
    for (int j = 32; j < 64; j++) s1 += a[j];
    sums[(b >> 5)] = -s0;
    sums[(b >> 5) + 1] = -s1;
    for (int p = 0; p < 4; p++)
      for (int c = 0; c < 16; c++) xq[b + 16 * p + c] = a[4 * c + p];
  }
}

/* ---- int8 products ------------------------------------------------------------------------------------------ */

/* the group's exact integer sum with the correction in it: relaxed/int8.ts:29-37 (relaxed_dot with activations
 * 0..127, int8.ts:6-11) */
static int32_t dot_relaxed(const int8_t *w, const uint8_t *q) {
  int32_t s = 0;
  for (int j = 0; j < GS; j++) s += (int32_t)w[j] * (int32_t)q[j];
  return s;
}

/* relaxed/int8.ts:17-50 over one row's int8 values (w, ng groups), scales srow, corrections crow */
static float q8r_row(const int8_t *w, const uint8_t *xq, const float *xs, const float *srow, const int32_t *crow,
                     int32_t ng) {
  const int32_t ng4 = ng & ~3;
  float lane[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  int32_t g = 0;
  for (; g < ng4; g++) { /* lane g & 3 adds the groups 4j + (g & 3) in order (int8.ts:26-39) */
    const float s = srow[g] * xs[g];
    const int32_t d = dot_relaxed(w + g * GS, xq + g * GS) + crow[g];
    const float p = (float)d * s;
    lane[g & 3] = lane[g & 3] + p;
  }
  float sum = ((lane[0] + lane[1]) + lane[2]) + lane[3]; /* hsum, math.ts:7-9 */
  for (; g < ng; g++) {                                /* the groups past the fours (int8.ts:41-47) */
    const int32_t d = dot_relaxed(w + g * GS, xq + g * GS) + crow[g];
    const float s = srow[g] * xs[g];
    const float p = (float)d * s;
    sum = sum + p;
  }
  return sum;
}

void o_matmul_q8r(float *xout, const uint8_t *xq, const float *xs, const int8_t *wq, const float *ws,
                  const int32_t *wc, int32_t n, int32_t r0, int32_t r1) {
  const int32_t ng = n / GS;
  for (int32_t i = r0; i < r1; i++)
    xout[i] = q8r_row(wq + (int64_t)i * n, xq, xs, ws + (int64_t)i * ng, wc + (int64_t)i * ng, ng);
}

/* dot32 (kernel/matmul.ts:68-72): lane k holds products 2k, 2k+1, 2k+8, 2k+9 of each 16-byte half, two products
 * added in int16 first (i16x8.add of the low and high extmuls, which wraps) */
static void dot32_lanes(int32_t lane[4], const int8_t *w, const int8_t *x) {
  for (int k = 0; k < 4; k++) {
    int32_t s = 0;
    for (int half = 0; half < 32; half += 16) {
      const int32_t a = wrap16((int32_t)w[half + 2 * k] * x[half + 2 * k] + (int32_t)w[half + 2 * k + 8] * x[half + 2 * k + 8]);
      const int32_t b = wrap16((int32_t)w[half + 2 * k + 1] * x[half + 2 * k + 1] +
                               (int32_t)w[half + 2 * k + 9] * x[half + 2 * k + 9]);
      s += a + b;
    }
    lane[k] = s;
  }
}

/* kernel/matmul.ts:77-97 over one row's int8 values: each lane times the scales' product into its own float32
 * lane, group by group; the four lanes added in order at the end */
static float q8_row(const int8_t *w, const int8_t *xq, const float *xs, const float *srow, int32_t ng) {
  float lane[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  int32_t d[4];
  for (int32_t g = 0; g < ng; g++) {
    const float s = srow[g] * xs[g];
    dot32_lanes(d, w + g * GS, xq + g * GS);
    for (int k = 0; k < 4; k++) {
      const float p = (float)d[k] * s;
      lane[k] = lane[k] + p;
    }
  }
  return ((lane[0] + lane[1]) + lane[2]) + lane[3];
}

void o_matmul_q8(float *xout, const int8_t *xq, const float *xs, const int8_t *wq, const float *ws, int32_t n,
                 int32_t r0, int32_t r1) {
  const int32_t ng = n / GS;
  for (int32_t i = r0; i < r1; i++) xout[i] = q8_row(wq + (int64_t)i * n, xq, xs, ws + (int64_t)i * ng, ng);
}

/* relaxed/int8.ts:147-166: every (row, token) is matmul_q8r's number to the bit (int8.ts:60-65), token t's
 * activations and scales at xq + t frame, xs + t frame, its outputs at xout + t os */
void o_matmul_q8r_tile(void *xout, const void *xq, const void *xs, const int8_t *wq, const float *ws,
                       const int32_t *wc, int32_t n, int32_t r0, int32_t r1, int32_t count, int32_t os,
                       int32_t frame) {
  for (int32_t t = 0; t < count; t++)
    o_matmul_q8r((float *)((char *)xout + (int64_t)t * os), (const uint8_t *)((const char *)xq + (int64_t)t * frame),
                 (const float *)((const char *)xs + (int64_t)t * frame), wq, ws, wc, n, r0, r1);
}

/* ---- int6 products: relaxed/six.ts:10-39, kernel/matmul.ts:227-244 ---------------------------------------- */
void o_matmul_q6r(float *xout, const uint8_t *xq, const float *xs, const uint8_t *wq, const float *ws,
                  const int32_t *wc, int32_t n, int32_t r0, int32_t r1) {
  const int32_t ng = n / GS;
  int8_t row[32 * 2048]; /* rows up to 65536 values: matmul_q8r's order on the widened row */
  if (ng > 2048) return;
  for (int32_t i = r0; i < r1; i++) {
    const uint8_t *packed = wq + (int64_t)i * ng * 24;
    for (int32_t g = 0; g < ng; g++) o_six_unpack(row + g * GS, packed + g * 24);
    xout[i] = q8r_row(row, xq, xs, ws + (int64_t)i * ng, wc + (int64_t)i * ng, ng);
  }
}

void o_matmul_q6(float *xout, const int8_t *xq, const float *xs, const uint8_t *wq, const float *ws, int32_t n,
                 int32_t r0, int32_t r1) {
  const int32_t ng = n / GS;
  int8_t v[32];
  int32_t d[4];
  for (int32_t i = r0; i < r1; i++) {
    const uint8_t *packed = wq + (int64_t)i * ng * 24;
    float lane[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int32_t g = 0; g < ng; g++) {
      o_six_unpack(v, packed + g * 24);
      dot32_lanes(d, v, xq + g * GS);
      const float s = ws[(int64_t)i * ng + g] * xs[g];
      for (int k = 0; k < 4; k++) lane[k] = lane[k] + (float)d[k] * s;
    }
    xout[i] = ((lane[0] + lane[1]) + lane[2]) + lane[3];
  }
}

/* ---- ternary and binary products: kernels/ternary.ts:23-34, binary.ts:19-22, relaxed/signs.ts:17-55 -------------- */

/* codes(v, p, three) (ternary.ts:25-27): i16x8.shr_u by 2p, then the mask; byte c of a 16-byte vector */
static int32_t code_of(const uint8_t *v16, int c, int p, int32_t three) {
  if (p == 0) return v16[c] & three;
  const int lo = c & ~1;
  const uint32_t lane = (uint32_t)v16[lo] | ((uint32_t)v16[lo + 1] << 8);
  const uint32_t shifted = (lane >> (2 * p)) & 0xffff;
  const uint32_t byte = (c & 1) ? (shifted >> 8) : (shifted & 0xff);
  return (int32_t)(int8_t)(uint8_t)(byte & (uint32_t)three);
}

/* bitCodes(v, k, two) (binary.ts:19-22): byte c of (k == 0 ? v + v (i8x16.add) : k == 1 ? v : v >> (k - 1) in 16-bit
 * lanes), masked with two: twice the bit k of byte c */
static int32_t bit_code_of(const uint8_t *v16, int c, int k, int32_t two) {
  uint32_t byte;
  if (k == 0) {
    byte = (uint8_t)(v16[c] + v16[c]);
  } else if (k == 1) {
    byte = v16[c];
  } else {
    const int lo = c & ~1;
    const uint32_t lane = (uint32_t)v16[lo] | ((uint32_t)v16[lo + 1] << 8);
    const uint32_t shifted = (lane >> (k - 1)) & 0xffff;
    byte = (c & 1) ? (shifted >> 8) : (shifted & 0xff);
  }
  return (int32_t)(int8_t)(uint8_t)(byte & (uint32_t)two);
}

/* one row of signsRows<P> (relaxed/signs.ts:28-55; kernel/matmul.ts:196-224 gives the same numbers): lane k adds
 * sub-group k (activations 32k..32k+31) of every group of 128, in order, f(f(whole * xs) * d)
 * (tests/ternary-check.ts:129-139).  Ternary (binary == 0): block h of a group is its bytes 16h..16h+15, plane p
 * codes(v, p) (ternary.ts:25-27); binary: both blocks are the group's 16 bytes, plane p of block h
 * bitCodes(v, 4h + p) (signs.ts:33-37) */
static float signs_row(const uint8_t *row, const uint16_t *srow, const int8_t *xq, const float *xs,
                       const int32_t *sums, int32_t groups, int32_t code, int binary) {
  float lane[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int32_t bytes = binary ? 16 : 32;
  for (int32_t g = 0; g < groups; g++) {
    const float d = o_half(srow[g]);
    for (int k = 0; k < 4; k++) {
      const int h = k >> 1, s = k & 1;
      const uint8_t *v = row + (int64_t)g * bytes + (binary ? 0 : 16 * h);
      const int8_t *x = xq + (int64_t)g * 128 + 64 * h;
      int32_t dot = 0;
      for (int p = 0; p < 4; p++)
        for (int c = 8 * s; c < 8 * s + 8; c++) {
          const int32_t cd = binary ? bit_code_of(v, c, 4 * h + p, code) : code_of(v, c, p, code);
          dot += cd * (int32_t)x[16 * p + c];
        }
      const int32_t whole = dot + sums[4 * g + k];
      const float a = (float)whole * xs[4 * g + k];
      const float b = a * d;
      lane[k] = lane[k] + b;
    }
  }
  return ((lane[0] + lane[1]) + lane[2]) + lane[3];
}

static void signs_rows(float *xout, const int8_t *xq, const float *xs, const uint8_t *wq, const uint16_t *ws,
                       int32_t n, int32_t r0, int32_t r1, int32_t code, int binary) {
  const int32_t groups = n >> 7;
  const int32_t *sums = (const int32_t *)(xs + (n >> 5));
  const int64_t row_bytes = binary ? (n >> 3) : (n >> 2);
  for (int32_t i = r0; i < r1; i++)
    xout[i] = signs_row(wq + (int64_t)i * row_bytes, ws + (int64_t)i * groups, xq, xs, sums, groups, code, binary);
}

void o_matmul_t2r(float *xout, const int8_t *xq, const float *xs, const uint8_t *wq, const uint16_t *ws,
                  int32_t n, int32_t r0, int32_t r1, int32_t three) {
  signs_rows(xout, xq, xs, wq, ws, n, r0, r1, three, 0);
}

void o_matmul_b1r(float *xout, const int8_t *xq, const float *xs, const uint8_t *wq, const uint16_t *ws,
                  int32_t n, int32_t r0, int32_t r1, int32_t two) {
  signs_rows(xout, xq, xs, wq, ws, n, r0, r1, two, 1);
}

/* signsTile<P> (relaxed/signs.ts:77-114): every (row, token) is the token kernel's number */
static void signs_tile(void *xout, const void *xq, const void *xs, const uint8_t *wq, const uint16_t *ws,
                       int32_t n, int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame, int32_t code,
                       int binary) {
  for (int32_t t = 0; t < count; t++)
    signs_rows((float *)((char *)xout + (int64_t)t * os), (const int8_t *)((const char *)xq + (int64_t)t * frame),
               (const float *)((const char *)xs + (int64_t)t * frame), wq, ws, n, r0, r1, code, binary);
}

void o_matmul_t2r_tile(void *xout, const void *xq, const void *xs, const uint8_t *wq, const uint16_t *ws,
                       int32_t n, int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame,
                       int32_t three) {
  signs_tile(xout, xq, xs, wq, ws, n, r0, r1, count, os, frame, three, 0);
}

void o_matmul_b1r_tile(void *xout, const void *xq, const void *xs, const uint8_t *wq, const uint16_t *ws,
                       int32_t n, int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame,
                       int32_t two) {
  signs_tile(xout, xq, xs, wq, ws, n, r0, r1, count, os, frame, two, 1);
}

/* ---- binary_x: kernels/kernel/quantize.ts:184-247 ------------------------------------------------------------ */
int32_t o_binary_x(uint8_t *out, float *xs, const float *x, int32_t n) {
  int32_t bad = 0;
  for (int32_t g = 0; g < n; g += 128) {
    const float *p = x + g;
    /* groupLargest (quantize.ts:186-191): lane j's f32x4.max of |values 4i + j|, then max(max(l0, l1), max(l2, l3)) */
    float lane[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < 32; i++)
      for (int j = 0; j < 4; j++) lane[j] = wasm_max(lane[j], fabsf(p[4 * i + j]));
    const float scale = wasm_max(wasm_max(lane[0], lane[1]), wasm_max(lane[2], lane[3]));
    xs[g >> 7] = scale;
    uint8_t *to = out + (g >> 3);
    for (int c = 0; c < 16; c++) {
      uint32_t byte = 0;
      for (int j = 0; j < 4; j++) {
        const float v0 = p[4 * c + j], v1 = p[64 + 4 * c + j];
        byte |= (uint32_t)(!(v0 < 0.0f)) << j;
        byte |= (uint32_t)(!(v1 < 0.0f)) << (4 + j);
        if (!(fabsf(v0) == scale && fabsf(v1) == scale)) bad = 1;
      }
      to[c] = (uint8_t)byte;
    }
  }
  return bad;
}

/* ---- the converters' packers: kernels/kernel/quantize.ts:153-225 ---------------------------------------------- */

/* quantize6_x (quantize.ts:161-182): per group of 32, scale = groupMax / 31 (groupMax as quantize_x's), xs =
 * scale / 4 (a multiply by 0.25), v = clamp(trunc_sat(nearest(value * (1 / scale))), -32, 31) (six(), 158-160), and
 * the six bits of v packed into 24 bytes: byte j (j < 16) the low nibbles of values j and j + 16, byte 16 + k
 * (k < 8) the top two bits of values k, k + 8, k + 16, k + 24 at bits 0, 2, 4, 6 (the shuffle at 177-179). */
void o_quantize6_x(uint8_t *out, float *xs, const float *x, int32_t n) {
  for (int32_t g = 0; g < n; g += GS) {
    float m[4];
    for (int j = 0; j < 4; j++) {
      float v = fabsf(x[g + j]);
      for (int i = 1; i < 8; i++) v = wasm_max(v, fabsf(x[g + 4 * i + j]));
      m[j] = v;
    }
    float amax = m[0];
    if (m[1] > amax) amax = m[1];
    if (m[2] > amax) amax = m[2];
    if (m[3] > amax) amax = m[3];
    const float scale = amax / 31.0f;
    xs[g / GS] = scale * 0.25f;
    const float inv = scale > 0 ? 1.0f / scale : 0.0f;
    uint8_t six[GS];
    for (int j = 0; j < GS; j++) {
      int32_t v = trunc_sat(rintf(x[g + j] * inv));
      if (v > 31) v = 31;
      if (v < -32) v = -32;
      six[j] = (uint8_t)((uint32_t)v & 63u);
    }
    uint8_t *at = out + (g / GS) * 24;
    for (int j = 0; j < 16; j++) at[j] = (uint8_t)((six[j] & 15) | ((six[j + 16] & 15) << 4));
    for (int k = 0; k < 8; k++)
      at[16 + k] = (uint8_t)((six[k] >> 4) | ((six[k + 8] >> 4) << 2) | ((six[k + 16] >> 4) << 4) | ((six[k + 24] >> 4) << 6));
  }
}

/* ternary_x (quantize.ts:197-225): per group of 128, the scale is groupLargest's (186-191: lane j's f32x4.max of
 * |values 4i + j|, then max(max(l0, l1), max(l2, l3)), NaN kept), the code of a value 1 + (v > 0) - (v < 0) (a NaN
 * gets 1) at bits 2 (j & 3) of byte j >> 2; the result is 1 where a value is neither 0 nor of the scale's size */
int32_t o_ternary_x(uint8_t *out, float *xs, const float *x, int32_t n) {
  int32_t bad = 0;
  for (int32_t g = 0; g < n; g += 128) {
    const float *p = x + g;
    float lane[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < 32; i++)
      for (int j = 0; j < 4; j++) lane[j] = wasm_max(lane[j], fabsf(p[4 * i + j]));
    const float scale = wasm_max(wasm_max(lane[0], lane[1]), wasm_max(lane[2], lane[3]));
    xs[g >> 7] = scale;
    uint8_t *to = out + (g >> 2);
    for (int b = 0; b < 32; b++) {
      uint32_t byte = 0;
      for (int q = 0; q < 4; q++) {
        const float v = p[4 * b + q];
        const uint32_t code = 1u + (v > 0.0f ? 1u : 0u) - (v < 0.0f ? 1u : 0u);
        byte |= code << (2 * q);
        if (!(fabsf(v) == scale || v == 0.0f)) bad = 1;
      }
      to[b] = (uint8_t)byte;
    }
  }
  return bad;
}

/* ---- CPU baseline: phase()-style row chunks over host threads ------------------------------------------------ */
typedef struct {
  int32_t kind;
  float *xout;
  const void *xq, *xs, *wq, *ws, *wc;
  int32_t n, rows, chunk, chunks;
  atomic_int next;
} gemv_job;

static void run_rows(gemv_job *j, int32_t r0, int32_t r1) {
  switch (j->kind) {
  case 0: o_matmul_q8r(j->xout, j->xq, j->xs, j->wq, j->ws, j->wc, j->n, r0, r1); break;
  case 1: o_matmul_q8(j->xout, j->xq, j->xs, j->wq, j->ws, j->n, r0, r1); break;
  case 2: o_matmul_q6r(j->xout, j->xq, j->xs, j->wq, j->ws, j->wc, j->n, r0, r1); break;
  case 3: o_matmul_q6(j->xout, j->xq, j->xs, j->wq, j->ws, j->n, r0, r1); break;
  default: o_matmul_t2r(j->xout, j->xq, j->xs, j->wq, j->ws, j->n, r0, r1, 3); break;
  }
}

static void *worker(void *arg) {
  gemv_job *j = (gemv_job *)arg;
  for (;;) {
    const int32_t c = atomic_fetch_add(&j->next, 1);
    if (c >= j->chunks) break;
    const int32_t r0 = c * j->chunk;
    const int32_t r1 = r0 + j->chunk < j->rows ? r0 + j->chunk : j->rows;
    run_rows(j, r0, r1);
  }
  return NULL;
}

static double now_s(void) {
  struct timespec t;
  clock_gettime(CLOCK_MONOTONIC, &t);
  return (double)t.tv_sec + 1e-9 * (double)t.tv_nsec;
}

double o_time_gemv(int32_t kind, float *xout, const void *xq, const void *xs, const void *wq, const void *ws,
                   const void *wc, int32_t n, int32_t rows, int32_t threads, int32_t reps) {
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  pthread_t tid[256];
  double best = 1e30;
  for (int32_t r = 0; r < reps; r++) {
    gemv_job j = {kind, xout, xq, xs, wq, ws, wc, n, rows, 0, 0, 0};
    int32_t want = threads * 4; /* CHUNKS_PER_THREAD, threads.ts:45 */
    j.chunk = (rows + want - 1) / want;
    if (j.chunk < 1) j.chunk = 1;
    j.chunks = (rows + j.chunk - 1) / j.chunk;
    atomic_init(&j.next, 0);
    const double t0 = now_s();
    for (int32_t t = 1; t < threads; t++) pthread_create(&tid[t], NULL, worker, &j);
    worker(&j);
    for (int32_t t = 1; t < threads; t++) pthread_join(tid[t], NULL);
    const double dt = now_s() - t0;
    if (dt < best) best = dt;
  }
  return best;
}

/* ---- llama.cpp's blocks of 256 weights: kernels/blocks/types.ts, token.ts, row.ts ----------------------------------
 * A weight is F S W - Fm M (types.ts:32-47): W a small integer of its own (decoded here as the kernels hold it,
 * magnitudes / minuses / weights, types.ts:194-270), S the integer of its unit of 16 or 32 (scaleOf, 273-292), for
 * the K types M the minimum of its unit (minimumOf, 294-300), F and Fm the block's (blockScale, blockMinimum,
 * 302-319).  The tables are sb_tables's (types.ts:323-348). */
enum { SB_Q2_K = 10, SB_Q4_K = 12, SB_IQ2_XXS = 16, SB_IQ2_XS = 17, SB_IQ3_XXS = 18, SB_IQ1_S = 19, SB_IQ3_S = 21,
       SB_IQ2_S = 22, SB_IQ4_XS = 23, SB_IQ1_M = 29 };
enum { T_IQ2XS = 2048, T_IQ2S = 6144, T_IQ3XXS = 14336, T_IQ3S = 15360, T_IQ1S = 17408, T_SIGNS = 33792,
       T_IQ4 = 34816, T_VECTORS = 34864, SB_GRIDS = 33792, SB_TABLES = 34992 };

int32_t o_sb_bytes(int32_t type) {
  switch (type) {
  case SB_IQ2_XXS: return 66;
  case SB_IQ3_S: return 110;
  case SB_IQ2_XS: return 74;
  case SB_IQ2_S: return 82;
  case SB_IQ3_XXS: return 98;
  case SB_IQ1_M: return 56;
  case SB_IQ1_S: return 50;
  case SB_Q2_K: return 84;
  case SB_IQ4_XS: return 136;
  case SB_Q4_K: return 144;
  }
  return 0;
}

static uint32_t u16_at(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }
static uint32_t u32_at(const uint8_t *p) { return u16_at(p) | (u16_at(p + 2) << 16); }

/* sb_tables (types.ts:323-348): the grids as the codebooks row has them (IQ1_S's plus one: codes 0, 1, 2), the
 * signs of 8 weights by a 7-bit index (the eighth makes the number of minus signs even), IQ4_XS's values, their
 * magnitudes and their signs, then the constant vectors */
int32_t o_sb_tables(uint8_t *area, const uint8_t *codebooks) {
  for (int i = 0; i < SB_GRIDS; i++) area[i] = (uint8_t)(codebooks[i] + (i >= T_IQ1S ? 1 : 0));
  for (int i = 0; i < 128; i++) {
    int ones = 0;
    for (int j = 0; j < 7; j++) ones += (i >> j) & 1;
    const int held = i | ((ones & 1) << 7);
    for (int j = 0; j < 8; j++) area[T_SIGNS + 8 * i + j] = ((held >> j) & 1) ? 255 : 0;
  }
  for (int i = 0; i < 16; i++) {
    const int8_t v = (int8_t)codebooks[SB_GRIDS + i];
    area[T_IQ4 + i] = (uint8_t)v;
    area[T_IQ4 + 16 + i] = (uint8_t)(int8_t)(v < 0 ? -v : v);
    area[T_IQ4 + 32 + i] = v < 0 ? 255 : 0;
  }
  uint8_t *v = area + T_VECTORS;
  for (int j = 0; j < 16; j++) {
    v[0 + j] = (uint8_t)(1u << (j & 7));
    v[16 + j] = (uint8_t)(j >> 3);
    v[32 + j] = 3;
    v[48 + j] = 15;
    v[80 + j] = 7;
    v[96 + j] = 1;
  }
  for (int j = 0; j < 4; j++) {
    const int32_t p3 = 512 >> (3 * j), p4 = 4096 >> (4 * j);
    memcpy(v + 64 + 4 * j, &p3, 4);
    memcpy(v + 112 + 4 * j, &p4, 4);
  }
  return SB_TABLES;
}

/* sums_x (token.ts:149-165): after the n/32 scales at xs, n/16 int16 sums of each 16 activations, then n/8 of each 8 */
void o_sums_x(void *xs, const int8_t *xq, int32_t n) {
  int16_t *s16 = (int16_t *)((char *)xs + 4 * (n >> 5)), *s8 = s16 + (n >> 4);
  for (int32_t i = 0; i < n / 8; i++) {
    int32_t s = 0;
    for (int j = 0; j < 8; j++) s += xq[8 * i + j];
    s8[i] = (int16_t)s;
  }
  for (int32_t i = 0; i < n / 16; i++) s16[i] = (int16_t)(s8[2 * i] + s8[2 * i + 1]);
}

/* halfOf (halves.ts:26-28): a half's 16 bits in the low bits of an int */
static float half_of(uint32_t bits) { return o_half((uint16_t)bits); }

/* one block at p: W[256], S[16] and M[16] (a unit's integer for each 16 weights), F, Fm; and, for sb_row, the block's
 * d (the float16 before the type's power of two), and IQ1's grid codes and shifts */
typedef struct {
  int32_t W[256], S[16], M[16];
  int32_t code[256], down[256];
  float F, Fm, d;
} sb_block;

/* The grids' bytes are signed: the reference's plain dot product multiplies them with extmul_*_i8x16_s
 * (types.ts:171-173). The converter's grids hold magnitudes of 0 to 127 (IQ1: codes 0, 1, 2), where the relaxed dot
 * (types.ts:170) agrees; other bytes give the plain kernel's numbers. */
static void sb_decode(const uint8_t *p, const uint8_t *tab, int32_t type, sb_block *B) {
  int32_t *S = B->S, *M = B->M;
  for (int h = 0; h < 16; h++) {
    const int g = h >> 1;
    int32_t *w = B->W + 16 * h;
    int mag[16], neg[16] = {0}, down[16] = {0};
    switch (type) {
    case SB_IQ2_XXS: {  /* types.ts:197-200, 227-230, 277 */
      const uint8_t *q = p + 2 + 8 * (h >> 1) + 2 * (h & 1);
      const uint32_t aux = u32_at(p + 6 + 8 * (h >> 1)) >> (14 * (h & 1));
      for (int j = 0; j < 16; j++) {
        mag[j] = (int8_t)tab[8 * q[j >> 3] + (j & 7)];
        neg[j] = tab[T_SIGNS + 8 * ((aux >> (7 * (j >> 3))) & 127) + (j & 7)] != 0;
      }
      S[h] = (int32_t)((u32_at(p + 6 + 8 * g) >> 27) | 1);
      break;
    }
    case SB_IQ2_XS: {  /* types.ts:201-204, 232-235, 279 */
      const uint8_t *q = p + 2 + 4 * h;
      for (int j = 0; j < 16; j++) {
        const uint32_t word = u16_at(q + 2 * (j >> 3));
        mag[j] = (int8_t)tab[T_IQ2XS + 8 * (word & 511) + (j & 7)];
        neg[j] = tab[T_SIGNS + 8 * (word >> 9) + (j & 7)] != 0;
      }
      S[h] = (int32_t)((((p[66 + g] >> (4 * (h & 1))) & 15) << 1) | 1);
      break;
    }
    case SB_IQ2_S: {  /* types.ts:205-208, 237, 280 */
      const uint8_t *q = p + 2 + 2 * h;
      const uint32_t high = p[66 + (h >> 1)] >> (4 * (h & 1)), bits = u16_at(p + 34 + 2 * h);
      const uint32_t idx[2] = {q[0] | ((high & 3) << 8), q[1] | ((high & 12) << 6)};
      for (int j = 0; j < 16; j++) {
        mag[j] = (int8_t)tab[T_IQ2S + 8 * idx[j >> 3] + (j & 7)];
        neg[j] = (bits >> j) & 1;
      }
      S[h] = (int32_t)((((p[74 + g] >> (4 * (h & 1))) & 15) << 1) | 1);
      break;
    }
    case SB_IQ3_XXS: {  /* types.ts:209-212, 227-230, 278 */
      const uint8_t *q = p + 2 + 4 * h;
      const uint32_t aux = u32_at(p + 66 + 4 * (h >> 1)) >> (14 * (h & 1));
      for (int j = 0; j < 16; j++) {
        mag[j] = (int8_t)tab[T_IQ3XXS + 4 * q[j >> 2] + (j & 3)];
        neg[j] = tab[T_SIGNS + 8 * ((aux >> (7 * (j >> 3))) & 127) + (j & 7)] != 0;
      }
      S[h] = (int32_t)((u32_at(p + 66 + 4 * g) >> 27) | 1);
      break;
    }
    case SB_IQ3_S: {  /* types.ts:213-217, 238, 281 */
      const uint8_t *q = p + 2 + 4 * h;
      const uint32_t high = p[66 + (h >> 1)] >> (4 * (h & 1)), bits = u16_at(p + 74 + 2 * h);
      for (int j = 0; j < 16; j++) {
        const int t = j >> 2;
        mag[j] = (int8_t)tab[T_IQ3S + 4 * (q[t] | (((high >> t) & 1) << 8)) + (j & 3)];
        neg[j] = (bits >> j) & 1;
      }
      S[h] = (int32_t)((((p[106 + (g >> 1)] >> (4 * ((h >> 1) & 1))) & 15) << 1) | 1);
      break;
    }
    case SB_IQ1_S: {  /* types.ts:218-221, 247-249, 260-261, 282 */
      const uint8_t *q = p + 2 + 2 * h;
      const uint32_t word = u16_at(p + 34 + 2 * (h >> 1)), high = word >> (6 * (h & 1));
      const uint32_t idx[2] = {q[0] | ((high & 7) << 8), q[1] | ((high & 56) << 5)};
      for (int j = 0; j < 16; j++) {
        mag[j] = (int8_t)tab[T_IQ1S + 8 * idx[j >> 3] + (j & 7)];
        down[j] = (int)(word >> 15);
      }
      S[h] = (int32_t)((((word >> 12) & 7) << 1) | 1);
      break;
    }
    case SB_IQ1_M: {  /* types.ts:222-225, 247-249, 262-264, 283 */
      const uint8_t *q = p + 2 * h;
      const uint32_t high = p[32 + h];
      const uint32_t idx[2] = {q[0] | ((high & 7) << 8), q[1] | ((high & 0x70) << 4)};
      for (int j = 0; j < 16; j++) {
        mag[j] = (int8_t)tab[T_IQ1S + 8 * idx[j >> 3] + (j & 7)];
        down[j] = (int)(j < 8 ? (high >> 3) & 1 : high >> 7);
      }
      S[h] = (int32_t)((((u16_at(p + 48 + 2 * (h >> 2)) >> (3 * (h & 3))) & 7) << 1) | 1);
      break;
    }
    case SB_Q2_K: {  /* types.ts:226-229 (bits 2 s, 2 s + 1 of byte b of a half's 32 are weight 32 s + b), 284, 297 */
      const uint8_t *v = p + 16 + 32 * (h >> 3) + 16 * (h & 1);
      const int s = (h & 7) >> 1;
      for (int j = 0; j < 16; j++) mag[j] = (v[j] >> (2 * s)) & 3;
      S[h] = p[h] & 15;
      M[h] = p[h] >> 4;
      break;
    }
    case SB_Q4_K: {  /* types.ts:230-232, 285-287, 298-300 */
      const uint8_t *v = p + 16 + 32 * (h >> 2) + 16 * (h & 1);
      const int hi = (h >> 1) & 1;
      for (int j = 0; j < 16; j++) mag[j] = (v[j] >> (4 * hi)) & 15;
      S[h] = h < 8 ? (p[4 + g] & 63) : ((p[8 + g] & 15) | ((p[g] >> 6) << 4));
      M[h] = h < 8 ? (p[8 + g] & 63) : ((p[8 + g] >> 4) | ((p[4 + g] >> 6) << 4));
      break;
    }
    case SB_IQ4_XS: {  /* types.ts:233-234, 288-290 */
      const uint8_t *v = p + 8 + 16 * (h >> 1);
      for (int j = 0; j < 16; j++) mag[j] = (int8_t)tab[T_IQ4 + ((v[j] >> (4 * (h & 1))) & 15)];
      S[h] = (int32_t)((((p[4 + (g >> 1)] >> (4 * ((h >> 1) & 1))) & 15) | (((u16_at(p + 2) >> (2 * (h >> 1))) & 3) << 4)) - 32);
      break;
    }
    }
    for (int j = 0; j < 16; j++) {
      if (type == SB_IQ1_S || type == SB_IQ1_M) w[j] = 8 * mag[j] - 7 - 2 * down[j];  /* 8 code - 7, 2 less when down */
      else w[j] = neg[j] ? -mag[j] : mag[j];
      B->code[16 * h + j] = mag[j];
      B->down[16 * h + j] = down[j];
    }
    if (type != SB_Q2_K && type != SB_Q4_K) M[h] = 0;
  }
  if (type == SB_IQ1_M) {  /* wholeScale (types.ts:312-316): the top four bits of the four words, the first's lowest */
    const uint32_t w0 = u16_at(p + 48), w1 = u16_at(p + 50), w2 = u16_at(p + 52), w3 = u16_at(p + 54);
    B->d = half_of((w0 >> 12) | ((w1 >> 8) & 0xf0) | ((w2 >> 4) & 0xf00) | (w3 & 0xf000));
  } else {
    B->d = o_half((uint16_t)u16_at(p + (type == SB_Q2_K ? 80 : 0)));
  }
  switch (type) {  /* blockScale (types.ts:302-310) */
  case SB_IQ2_XXS: case SB_IQ2_XS: case SB_IQ2_S: case SB_IQ1_S: case SB_IQ1_M: B->F = B->d * 0.125f; break;
  case SB_IQ3_XXS: B->F = B->d * 0.25f; break;
  default: B->F = B->d; break;
  }
  /* blockMinimum (types.ts:318-320) */
  B->Fm = type == SB_Q2_K ? o_half((uint16_t)u16_at(p + 82)) : type == SB_Q4_K ? o_half((uint16_t)u16_at(p + 2)) : 0.0f;
}

/* one row of matmul_sbr / matmul_sb (token.ts:111-134, types.ts:48-57): per block, G[k] = sum over group k of
 * S W a (exact), M[k] = sum over group k of M a (K types); lane k += f(f(f(G[k] xs[k]) + f(G[k+4] xs[k+4])) F), less
 * f(f(f(M[k] xs[k]) + f(M[k+4] xs[k+4])) Fm) for the K types; ((l0 + l1) + l2) + l3 at the end */
static float sb_row_dot(const uint8_t *row, const uint8_t *tab, const int8_t *xq, const float *xs, int32_t n,
                        int32_t type) {
  const int32_t size = o_sb_bytes(type);
  const int minimums = type == SB_Q2_K || type == SB_Q4_K;
  float lane[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  sb_block B;
  const int32_t *W = B.W, *S = B.S, *M = B.M;
  for (int32_t b = 0; b < (n >> 8); b++) {
    sb_decode(row + (int64_t)b * size, tab, type, &B);
    const float F = B.F, Fm = B.Fm;
    const int8_t *a = xq + 256 * b;
    const float *s = xs + 8 * b;
    int32_t G[8] = {0}, Mi[8] = {0};
    for (int i = 0; i < 256; i++) {
      G[i >> 5] += S[i >> 4] * W[i] * (int32_t)a[i];
      Mi[i >> 5] += M[i >> 4] * (int32_t)a[i];
    }
    for (int k = 0; k < 4; k++) {
      const float lo = (float)G[k] * s[k], hi = (float)G[k + 4] * s[k + 4];
      const float sum = lo + hi;
      float part = sum * F;
      if (minimums) {
        const float mlo = (float)Mi[k] * s[k], mhi = (float)Mi[k + 4] * s[k + 4];
        const float msum = mlo + mhi;
        part = part - msum * Fm;
      }
      lane[k] = lane[k] + part;
    }
  }
  return ((lane[0] + lane[1]) + lane[2]) + lane[3];
}

void o_matmul_sbr(float *xout, const int8_t *xq, const void *xs, const uint8_t *w, const uint8_t *tab, int32_t n,
                  int32_t r0, int32_t r1, int32_t type) {
  const int32_t size = o_sb_bytes(type);
  if (!size) return;  /* an unknown type writes nothing (token.ts:136-149) */
  for (int32_t i = r0; i < r1; i++)
    xout[i] = sb_row_dot(w + (int64_t)i * (n >> 8) * size, tab, xq, (const float *)xs, n, type);
}

void o_matmul_sbr_tile(void *xout, const void *xq, const void *xs, const uint8_t *w, const uint8_t *tab, int32_t n,
                       int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame, int32_t type) {
  for (int32_t t = 0; t < count; t++)
    o_matmul_sbr((float *)((char *)xout + (int64_t)t * os), (const int8_t *)((const char *)xq + (int64_t)t * frame),
                 (const char *)xs + (int64_t)t * frame, w, tab, n, r0, r1, type);
}

/* sb_row (row.ts:7-58): the row's n weights as float32, each f(f(scale) W) (less f(Fm M) for the K types), scale the
 * reader's product of the block's and the unit's floats; IQ1: f(scale (g + or - 1/8)), g the grid's -1, 0, 1 */
void o_sb_row(float *out, const uint8_t *w, const uint8_t *tab, int32_t n, int32_t type) {
  const int32_t size = o_sb_bytes(type);
  if (!size) return;
  sb_block B;
  for (int32_t b = 0; b < (n >> 8); b++) {
    const uint8_t *p = w + (int64_t)b * size;
    sb_decode(p, tab, type, &B);
    for (int h = 0; h < 16; h++) {
      float scale;
      const float s = (float)(B.S[h] >> 1);
      switch (type) {  /* row.ts:9-17 (floatScale) */
      case SB_IQ2_XXS: case SB_IQ2_XS: case SB_IQ2_S: scale = B.d * (0.5f + s) * 0.25f; break;
      case SB_IQ3_XXS: scale = B.d * (0.5f + s) * 0.5f; break;
      default: scale = B.d * (float)B.S[h]; break;
      }
      for (int j = 0; j < 16; j++) {
        const int i = 16 * h + j;
        float v;
        /* W as an int8 (row.ts:32-37: the signs put on the magnitudes with i8x16.sub, IQ1's code less 1 with
         * i8x16.sub (row.ts:24), both wrapping: only a grid byte of -128 shows it) */
        if (type == SB_IQ1_S || type == SB_IQ1_M)  /* the grid's -1, 0, 1 and an eighth more or less (row.ts:22-31) */
          v = (float)(int8_t)(B.code[i] - 1) + (B.down[i] ? -0.125f : 0.125f);
        else
          v = (float)(int8_t)B.W[i];
        float x = scale * v;
        if (type == SB_Q2_K || type == SB_Q4_K) {
          const float least = B.Fm * (float)B.M[h];
          x = x - least;
        }
        out[256 * b + i] = x;
      }
    }
  }
}

/* matmul.ts:248-266: for each j the reference starts from y[j] and adds f(a[c] rows[c][j]) for c in order; its
 * four-wide loop (v128 lanes j .. j+3) and its scalar tail (j from n & ~3) do the same for every j */
void o_add_columns(float *y, const float *rows, const float *a, int32_t count, int32_t n) {
  for (int32_t j = 0; j < n; j++) {
    float acc = y[j];
    for (int32_t c = 0; c < count; c++) {
      const float product = a[c] * rows[(int64_t)c * n + j];
      acc = acc + product;
    }
    y[j] = acc;
  }
}
