// common.hpp — device helpers shared by the kernels of libhq.so (gfx950, wave64).
//
// Everything here is compiled with -ffp-contract=off and denormals kept: a float operation written below is one
// IEEE binary32 operation rounded to nearest-even, as the reference's WebAssembly f32 / f32x4 operations are.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define HQ_DEV __device__ __forceinline__

namespace hq {

constexpr int GS = 32;  // int8 quantization group (kernels/kernel/math.ts:4)

HQ_DEV float fmul(float a, float b) { return __fmul_rn(a, b); }
HQ_DEV float fadd(float a, float b) { return __fadd_rn(a, b); }
HQ_DEV float fdiv(float a, float b) { return __fdiv_rn(a, b); }
HQ_DEV float fsub(float a, float b) { return __fsub_rn(a, b); }

// v_dot4_i32_i8: c + the four products of signed bytes (exact in int32 for every byte)
HQ_DEV int32_t sdot4(int32_t a, int32_t b, int32_t c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// a raw buffer over [base, base + bytes) (bytes clamped to 32 bits): a load past its end reads nothing and returns
// zeros
HQ_DEV __amdgpu_buffer_rsrc_t resource(const char *base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0,
                                           (int)max((int64_t)0, min(bytes, (int64_t)0xFFFFFFFF)), 0x00020000);
}

// DPP moves within a row of 16 lanes (row_ror:n gives lane l the value of lane (l - n) mod 16 of its row)
template <int CTRL>
HQ_DEV int32_t dpp(int32_t v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
// lane l of a row of 16 gets the value of lane (l + S) mod 16
template <int S>
HQ_DEV int32_t from_lane_plus(int32_t v) {
  static_assert(S > 0 && S < 16, "shift within a row");
  return dpp<0x120 + (16 - S)>(v);
}
template <int S>
HQ_DEV float from_lane_plus(float v) {
  return __int_as_float(from_lane_plus<S>(__float_as_int(v)));
}
// lanes 0..15 (32..47) get lanes 16..31's (48..63's) values: v_permlane16_swap's second result, of v with itself
HQ_DEV float upper_row(float v) {
  return __uint_as_float(__builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false)[1]);
}
// lane l gets lane (l ^ 1)'s value (quad_perm [1, 0, 3, 2])
HQ_DEV int32_t swap_pair(int32_t v) { return dpp<0xB1>(v); }
// every lane of a quad gets that quad's lane Q (quad_perm [Q, Q, Q, Q])
template <int Q>
HQ_DEV float quad_lane(float v) {
  return __int_as_float(dpp<Q * 0x55>(__float_as_int(v)));
}

// f32x4.max lane semantics: NaN if either is NaN (kernels/kernel/quantize.ts:10-19); the inputs are |x| >= +0
HQ_DEV float wasm_max_abs(float a, float b) { return (a != a || b != b) ? __int_as_float(0x7fc00000) : fmaxf(a, b); }

// kernels/kernel/halves.ts:6-23: a half's bits sign-extended, << 13, & 0x8fffffff, as float, times 2^112:
// exact for every finite half, an infinity reads as 65536
HQ_DEV float half_to_float(uint32_t h16) {
  const int32_t bits = ((int32_t)(int16_t)(uint16_t)h16 * 8192) & (int32_t)0x8fffffff;
  return fmul(__int_as_float(bits), 5.192296858534828e33f);
}

// i32x4.trunc_sat_f32x4_s: NaN -> 0, saturating at the int32 ends
HQ_DEV int32_t trunc_sat(float v) {
  if (v != v) return 0;
  if (v >= 2147483648.0f) return INT32_MAX;
  if (v <= -2147483648.0f) return INT32_MIN;
  return (int32_t)v;
}

// kernels/kernel/quantize.ts:124-151 for one group of 32 float32 values v: its 32 bytes (eight dwords, values
// 4i..4i+3 in dword i) and its scale.  groupMax (quantize.ts:10-19): lane j's maximum of |values 4i + j| with a NaN
// kept (a non-negative float's bits order as the float does, and every NaN's bits are above +inf's), then lanes 1..3
// compared with lane 0's in order, where a NaN is passed over.
HQ_DEV void quantize_values(const float v[32], int32_t bias, uint32_t q[8], float &scale) {
  uint32_t m[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 8; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) m[j] = max(m[j], __float_as_uint(v[4 * i + j]) & 0x7fffffffu);
  float amax = __uint_as_float(m[0]);
#pragma unroll
  for (int j = 1; j < 4; j++) {
    const float mj = __uint_as_float(m[j]);
    if (mj > amax) amax = mj;
  }
  scale = fdiv(amax, bias == 0 ? 127.0f : 63.0f);
  const float inv = scale > 0.0f ? fdiv(1.0f, scale) : 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    uint32_t d = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int32_t t = trunc_sat(rintf(fmul(v[4 * i + j], inv)));
      int32_t r = (int32_t)((uint32_t)t + (uint32_t)bias);  // i32x4.add wraps
      r = min(max(r, -128), 127);                           // the two saturating narrowings
      d |= ((uint32_t)r & 0xffu) << (8 * j);
    }
    q[i] = d;
  }
}

// the same for the group at p (16-byte aligned)
HQ_DEV void quantize_group(const float *p, int32_t bias, uint32_t q[8], float &scale) {
  float v[32];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float4 f = ((const float4 *)p)[i];
    v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
  }
  quantize_values(v, bias, q, scale);
}

// v_perm_b32: byte i of the result is byte sel.i of {hi:lo} (0..3 from lo, 4..7 from hi)
HQ_DEV uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) { return __builtin_amdgcn_perm(hi, lo, sel); }

// the ternary codes of plane p of four bytes: (v >> 2p) & 3 a byte (kernels/ternary.ts:23-27).  The reference
// shifts 16-bit lanes; with the mask 3 a 32-bit shift leaves the same bits (what a byte takes from its neighbour
// lands at bit 8 - 2p >= 2 and is masked away).
template <int P>
HQ_DEV uint32_t codes(uint32_t v) {
  return (P == 0 ? v : (v >> (2 * P))) & 0x03030303u;
}

// kernels/six.ts:16-31, src/python/engine/packing.py:56-70: one group of 24 bytes (six dwords: d[0..3] the low
// nibbles, d[4..5] the top bits) -> its 32 int8 values (eight dwords, values 4i..4i+3 in dword i)
HQ_DEV void six_widen(const uint32_t d[6], uint32_t v[8]) {
  // value j (0..15): low nibble of byte j, top bits 2 (j / 8) of byte 16 + j % 8 -> (nibble << 2) | (top << 6)
  // value 16 + j: high nibble of byte j, top bits 4 + 2 (j / 8) of byte 16 + j % 8
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t lo = d[i];
    const uint32_t t = d[4 + (i & 1)];  // the top bytes of values 4i..4i+3 (mod 8)
    const uint32_t tlo = (i < 2) ? (t << 6) : (t << 4);       // bits 0-1 (j < 8) or 2-3 (j >= 8) to 6-7
    const uint32_t thi = (i < 2) ? (t << 2) : t;              // bits 4-5 or 6-7 to 6-7
    v[i] = ((lo << 2) & 0x3c3c3c3cu) | (tlo & 0xc0c0c0c0u);
    v[4 + i] = ((lo >> 2) & 0x3c3c3c3cu) | (thi & 0xc0c0c0c0u);
  }
}

}  // namespace hq
