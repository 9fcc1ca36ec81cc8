// gemm.hip — the prompt kernels on the matrix cores (more than four tokens):
//   matmul_q8r_tile (kernels/relaxed/int8.ts:52-166), matmul_q6r for many tokens (jobs.ts:243-248 runs it a token at
//   a time: every (row, token) is matmul_q6r's number), matmul_t2r_tile (kernels/relaxed/signs.ts:232-297).
//
// A block is 4 waves and a 64 x 64 tile of (rows, tokens); a wave owns one 32 x 32 tile and runs one
// v_mfma_i32_32x32x32_i8 a group of 32: K = 32 is one scale group, so the MFMA's int32 results are the groups' exact
// integer sums (for ternary, one part of 32 of a group of 128).  The corrections ride in the MFMA's accumulator
// input: int8_sums' wc (one a row and group) for int8 / int6, interleave()'s sums (one a token and part) for
// ternary, so the integer is the reference's, correction included, with no VALU work.
//
// Float32 order: every (row, token) is the token kernel's number to the bit.  The reference's lane k adds groups
// 4 j + k (int8, int6) or part k of every group (ternary) in order; here a stage is 4 groups (int8, int6) or one group
// of 128 (ternary), stage after stage in order, and accumulator set k of the stage takes group / part k: four
// running sums a register, added ((a0 + a1) + a2) + a3 at the end (math.ts:7-9), then (int8, int6) the groups past
// the last four one at a time (relaxed/int8.ts:40-47).  Each term is f(f(C) * f(ws * xs)) (int8) or
// f(f(C * xs) * d) (ternary), rounded as the reference rounds it (-ffp-contract=off).
//
// The scales' product of int8 / int6, f(ws * xs) for every (row, token), is an outer product: a
// v_mfma_f32_32x32x2_f32 with K = 2 and its second column zero gives it, each product rounded once as v_mul_f32
// rounds it (subnormals included), on the matrix core.  Roofline: per output element and group the epilogue is then
// 3 VALU operations (convert, multiply, add; ternary 4: f(f(C * xs) * d) has no such product) against 32 MACs on the
// matrix core; CDNA4's VALU does 64 lanes a clock a CU against 4096 int8 MACs, so the epilogue, not the MFMA, bounds
// this kernel (at best 32 / (3 x 4096 / 64) = 16.7 % of dense int8 peak, 12.5 % for ternary).
#include "common.hpp"
#include "launch.hpp"

namespace hq {

namespace {

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int BR = 64, BT = 64;     // block tile: rows x tokens
constexpr int XPAD = 128 + 16;      // LDS row of a stage's 128 bytes, padded against bank conflicts
constexpr int TPAD = 32 + 16;       // ternary: a row's 32 raw bytes, padded

HQ_DEV uint4 ld16(const char *p) { return *(const uint4 *)p; }
HQ_DEV uint2 ld8(const char *p) { return *(const uint2 *)p; }

// ---------------------------------------------------------------------------------------------------------------
// int8 / int6 weights, relaxed activations (matmul_q8r_tile, matmul_q6r)
// MFMA A = weights (m = row), B = activations (n = token): lane l holds token l % 32 and rows
// 8 (r / 4) + 4 (l / 32) + r % 4 of its wave's 32 (r = 0..15).
// ---------------------------------------------------------------------------------------------------------------
struct StageQ {
  char w[BR][XPAD];   // 4 groups of each row, widened to int8
  char x[BT][XPAD];   // 4 groups of each token
  float ws[4][BR];    // the rows' scales, group-major
  int32_t wc[4][BR];  // the rows' corrections (the caller's, or -64 sum(w) made at staging), group-major
  float xs[BT][4];    // the tokens' scales
};

template <int PACK, bool WC>
struct LoaderQ {
  uint32_t w[8], x[8];
  int32_t wsum;  // without the caller's corrections: -64 times the group's sum, made here (int8_sums' value)
  float sc[4];   // ws (threads 0..63), wc (64..127) or xs (128..191) of the stage's four groups
  HQ_DEV void load(const Job &J, int row0, int tok0, int M, int j, int ng) {
    const int i = threadIdx.x;
    const int r = i >> 2, k = i & 3;
    const int g = min(4 * j + k, ng - 1);
    const int row = min(row0 + r, J.r1 - 1);
    constexpr int GB = PACK == 8 ? 32 : 24;
    const char *wp = J.wq + ((int64_t)row * ng + g) * GB;
    if (PACK == 8) {
      const uint4 a = ld16(wp), b = ld16(wp + 16);
      w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
    } else {
      const uint2 a = ld8(wp), b = ld8(wp + 8), c = ld8(wp + 16);
      const uint32_t d[6] = {a.x, a.y, b.x, b.y, c.x, c.y};
      six_widen(d, w);
    }
    if (!WC) {
      int32_t s = 0;
#pragma unroll
      for (int q = 0; q < 8; q++) s = sdot4((int32_t)w[q], 0x01010101, s);
      wsum = -64 * s;
    }
    const int tok = min(tok0 + r, M - 1);
    const char *xp = J.xq + tok * J.frame + (int64_t)g * 32;
    const uint4 a = ld16(xp), b = ld16(xp + 16);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    const float *src = nullptr;
    if (i < 64) src = (const float *)J.ws + (int64_t)min(row0 + i, J.r1 - 1) * ng;
    else if (i < 128) { if (WC) src = (const float *)((const int32_t *)J.wc + (int64_t)min(row0 + i - 64, J.r1 - 1) * ng); }
    else if (i < 192) src = (const float *)(J.xs + min(tok0 + i - 128, M - 1) * J.sframe);
    if (src) {
#pragma unroll
      for (int q = 0; q < 4; q++) sc[q] = src[min(4 * j + q, ng - 1)];
    }
  }
  HQ_DEV void store(StageQ &S) const {
    const int i = threadIdx.x;
    const int r = i >> 2, k = i & 3;
    uint4 *wd = (uint4 *)(S.w[r] + 32 * k);
    wd[0] = make_uint4(w[0], w[1], w[2], w[3]);
    wd[1] = make_uint4(w[4], w[5], w[6], w[7]);
    uint4 *xd = (uint4 *)(S.x[r] + 32 * k);
    xd[0] = make_uint4(x[0], x[1], x[2], x[3]);
    xd[1] = make_uint4(x[4], x[5], x[6], x[7]);
    if (!WC) S.wc[k][r] = wsum;
    if (i < 64) {
#pragma unroll
      for (int q = 0; q < 4; q++) S.ws[q][i] = sc[q];
    } else if (i < 128) {
      if (WC) {
#pragma unroll
        for (int q = 0; q < 4; q++) S.wc[q][i - 64] = __float_as_int(sc[q]);
      }
    } else if (i < 192) {
#pragma unroll
      for (int q = 0; q < 4; q++) S.xs[i - 128][q] = sc[q];
    }
  }
};

// f(ws * xs) for the wave's 32 rows x 32 tokens of group k: the outer product on the matrix core (A lane l < 32: the
// scale of row l, B lane l < 32: the scale of token l, the K = 1 half zero), laid out as the int8 MFMA's result
HQ_DEV v16f q_scales(const StageQ &S, int k, int wrow, int wtok, int lane) {
  const float a = lane < 32 ? S.ws[k][wrow + lane] : 0.0f;
  const float b = lane < 32 ? S.xs[wtok + lane][k] : 0.0f;
  v16f z;
#pragma unroll
  for (int r = 0; r < 16; r++) z[r] = 0.0f;
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, z, 0, 0, 0);
}

HQ_DEV v16i q_mfma(const StageQ &S, int k, int wrow, int wtok, int lane) {
  const v4i A = *(const v4i *)(S.w[wrow + (lane & 31)] + 32 * k + 16 * (lane >> 5));
  const v4i B = *(const v4i *)(S.x[wtok + (lane & 31)] + 32 * k + 16 * (lane >> 5));
  // the accumulator starts at the rows' corrections: dot(w, q) + wc = dot(w, q - 64)
  const int rbase = wrow + 4 * (lane >> 5);
  v16i C;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int4 c4 = *(const int4 *)&S.wc[k][rbase + 8 * q];
    C[4 * q] = c4.x; C[4 * q + 1] = c4.y; C[4 * q + 2] = c4.z; C[4 * q + 3] = c4.w;
  }
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, C, 0, 0, 0);
}

template <int PACK, bool WC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void gemm_relaxed(Job J) {
  __shared__ StageQ stage[2];
  const int M = J.count;
  const int ng = J.n >> 5, ng4 = ng & ~3;
  const int row0 = J.r0 + blockIdx.x * BR, tok0 = blockIdx.y * BT;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wrow = 32 * (wave >> 1), wtok = 32 * (wave & 1);
  const int rbase = wrow + 4 * (lane >> 5);   // this lane's first row in the tile (then + 8 q + e)

  float acc[4][16];
#pragma unroll
  for (int k = 0; k < 4; k++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[k][r] = 0.0f;

  LoaderQ<PACK, WC> L;
  const int stages = ng4 >> 2;
  if (stages > 0) {
    L.load(J, row0, tok0, M, 0, ng);
    L.store(stage[0]);
  }
  __syncthreads();
  for (int j = 0; j < stages; ++j) {
    const StageQ &S = stage[j & 1];
    if (j + 1 < stages) L.load(J, row0, tok0, M, j + 1, ng);
#pragma unroll
    for (int k = 0; k < 4; k++) {  // group 4 j + k: the reference's lane k (relaxed/int8.ts:26-39)
      const v16i C = q_mfma(S, k, wrow, wtok, lane);
      const v16f sc = q_scales(S, k, wrow, wtok, lane);
#pragma unroll
      for (int r = 0; r < 16; r++) acc[k][r] = fadd(acc[k][r], fmul((float)C[r], sc[r]));
    }
    if (j + 1 < stages) L.store(stage[(j + 1) & 1]);
    __syncthreads();
  }
  float sum[16];
#pragma unroll
  for (int r = 0; r < 16; r++) sum[r] = fadd(fadd(fadd(acc[0][r], acc[1][r]), acc[2][r]), acc[3][r]);
  if (ng4 < ng) {  // the groups past the fours: one more stage of groups ng4.., each added in order
    L.load(J, row0, tok0, M, stages, ng);
    L.store(stage[stages & 1]);
    __syncthreads();
    const StageQ &S = stage[stages & 1];
    for (int k = 0; k < ng - ng4; k++) {
      const v16i C = q_mfma(S, k, wrow, wtok, lane);
      const v16f sc = q_scales(S, k, wrow, wtok, lane);
#pragma unroll
      for (int r = 0; r < 16; r++) sum[r] = fadd(sum[r], fmul((float)C[r], sc[r]));
    }
  }
  const int t = tok0 + wtok + (lane & 31);  // this lane's token
  if (t < M) {
    float *out = (float *)(J.out + t * J.os);
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int row = row0 + rbase + 8 * q + e;
        if (row < J.r1) out[row] = sum[4 * q + e];
      }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// ternary (matmul_t2r_tile)
// MFMA A = activations (m = token), B = codes (n = row): lane l holds row l % 32 and tokens 8 (r / 4) + 4 (l / 32)
// + r % 4.  Part k of the group of 128 (block h = k / 2, bytes c = 8 (k % 2) .. + 7 of it) as 32 K values in the
// order plane-major: K-half kh of a lane is planes 2 kh, 2 kh + 1, eight c's each, for the codes and for
// interleave()'s activation bytes 64 h + 16 p + 8 (k % 2) .. + 7 alike.
// ---------------------------------------------------------------------------------------------------------------
struct StageT {
  char w[BR][TPAD];      // the group's 32 bytes of each row
  char x[BT][XPAD];      // the group's 128 interleaved activations of each token
  float xs[4][BT];       // the tokens' scales of the group's four parts, part-major
  int32_t sums[4][BT];   // and their sums
  float d[BR];           // the rows' group scale, widened
};

struct LoaderT {
  uint4 w, x[2];
  uint4 s;
  uint32_t h;
  HQ_DEV void load(const Job &J, int row0, int tok0, int M, int g) {
    const int i = threadIdx.x;
    const int groups = J.n >> 7;
    // weights: 64 rows x 32 bytes, 16 bytes a thread of the first 128 threads
    if (i < 128) {
      const int row = min(row0 + (i >> 1), J.r1 - 1);
      w = ld16(J.wq + ((int64_t)row * groups + g) * 32 + 16 * (i & 1));
    }
    // activations: 64 tokens x 128 bytes, 32 bytes a thread
    const int tk = min(tok0 + (i >> 2), M - 1);
    const char *xp = J.xq + tk * J.frame + (int64_t)g * 128 + 32 * (i & 3);
    x[0] = ld16(xp);
    x[1] = ld16(xp + 16);
    if (i >= 128 && i < 192) {  // the scales and sums of the group's four parts
      const int tt = min(tok0 + i - 128, M - 1);
      s = *(const uint4 *)((const float *)(J.xs + tt * J.sframe) + 4 * g);
    } else if (i >= 192) {
      const int tt = min(tok0 + i - 192, M - 1);
      s = *(const uint4 *)((const int32_t *)((const float *)(J.xs + tt * J.sframe) + (J.n >> 5)) + 4 * g);
    }
    if (i < 64) {
      const int row = min(row0 + i, J.r1 - 1);
      h = ((const uint16_t *)J.ws)[(int64_t)row * groups + g];
    }
  }
  HQ_DEV void store(StageT &S) const {
    const int i = threadIdx.x;
    if (i < 128) *(uint4 *)(S.w[i >> 1] + 16 * (i & 1)) = w;
    uint4 *xd = (uint4 *)(S.x[i >> 2] + 32 * (i & 3));
    xd[0] = x[0];
    xd[1] = x[1];
    const uint32_t v[4] = {s.x, s.y, s.z, s.w};
    if (i >= 128 && i < 192) {
#pragma unroll
      for (int q = 0; q < 4; q++) S.xs[q][i - 128] = __uint_as_float(v[q]);
    } else if (i >= 192) {
#pragma unroll
      for (int q = 0; q < 4; q++) S.sums[q][i - 192] = (int32_t)v[q];
    }
    if (i < 64) S.d[i] = half_to_float(h);
  }
};

template <int P0>
HQ_DEV v4i plane_pair(uint32_t w0, uint32_t w1) {
  v4i b;
  b[0] = (int32_t)codes<P0>(w0);
  b[1] = (int32_t)codes<P0>(w1);
  b[2] = (int32_t)codes<P0 + 1>(w0);
  b[3] = (int32_t)codes<P0 + 1>(w1);
  return b;
}

HQ_DEV v16i t_mfma(const StageT &S, int k, int wrow, int wtok, int lane) {
  const int h = k >> 1, s = k & 1, kh = lane >> 5;
  // A: token lane % 32's bytes of planes 2 kh, 2 kh + 1 (eight each) of part k
  const char *xp = S.x[wtok + (lane & 31)] + 64 * h + 8 * s + 32 * kh;
  const uint2 a0 = *(const uint2 *)xp, a1 = *(const uint2 *)(xp + 16);
  v4i A;
  A[0] = (int32_t)a0.x; A[1] = (int32_t)a0.y; A[2] = (int32_t)a1.x; A[3] = (int32_t)a1.y;
  // B: row lane % 32's codes of the same planes and c's
  const uint2 wv = *(const uint2 *)(S.w[wrow + (lane & 31)] + 16 * h + 8 * s);
  const v4i B = kh == 0 ? plane_pair<0>(wv.x, wv.y) : plane_pair<2>(wv.x, wv.y);
  // the accumulator starts at interleave()'s sums of the lane's 16 tokens
  const int tbase = wtok + 4 * kh;
  v16i C;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int4 c4 = *(const int4 *)&S.sums[k][tbase + 8 * q];
    C[4 * q] = c4.x; C[4 * q + 1] = c4.y; C[4 * q + 2] = c4.z; C[4 * q + 3] = c4.w;
  }
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, C, 0, 0, 0);
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void gemm_ternary(Job J) {
  __shared__ StageT stage[2];
  const int M = J.count;
  const int groups = J.n >> 7;
  const int row0 = J.r0 + blockIdx.x * BR, tok0 = blockIdx.y * BT;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wrow = 32 * (wave >> 1), wtok = 32 * (wave & 1);
  const int row = wrow + (lane & 31);          // this lane's row in the tile
  const int tbase = wtok + 4 * (lane >> 5);    // its first token (then + 8 q + e)

  float acc[4][16];
#pragma unroll
  for (int k = 0; k < 4; k++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[k][r] = 0.0f;

  LoaderT L;
  L.load(J, row0, tok0, M, 0);
  L.store(stage[0]);
  __syncthreads();
  for (int g = 0; g < groups; ++g) {
    const StageT &S = stage[g & 1];
    if (g + 1 < groups) L.load(J, row0, tok0, M, g + 1);
    const float d = S.d[row];
#pragma unroll
    for (int k = 0; k < 4; k++) {  // part k of the group: the reference's lane k (relaxed/signs.ts:198-207)
      const v16i C = t_mfma(S, k, wrow, wtok, lane);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float4 x4 = *(const float4 *)&S.xs[k][tbase + 8 * q];
        const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
        for (int e = 0; e < 4; e++)
          acc[k][4 * q + e] = fadd(acc[k][4 * q + e], fmul(fmul((float)C[4 * q + e], xv[e]), d));
      }
    }
    if (g + 1 < groups) L.store(stage[(g + 1) & 1]);
    __syncthreads();
  }
  const int rw = row0 + row;
  if (rw < J.r1) {
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int t = tok0 + tbase + 8 * q + e;
        if (t < M) {
          const int r = 4 * q + e;
          ((float *)(J.out + t * J.os))[rw] = fadd(fadd(fadd(acc[0][r], acc[1][r]), acc[2][r]), acc[3][r]);
        }
      }
  }
}

}  // namespace

bool gemm_supported(Kind kind) { return kind == Q8R || kind == Q6R || kind == T2R || kind == T2; }

hipError_t launch_gemm(Kind kind, const Job &job, hipStream_t s) {
  const int rows = job.r1 - job.r0;
  if (rows <= 0 || job.count <= 0) return hipSuccess;
  dim3 grid((rows + BR - 1) / BR, (job.count + BT - 1) / BT), block(256);
  const bool wc = job.wc != nullptr;
  switch (kind) {
  case Q8R:
    if (wc) hipLaunchKernelGGL((gemm_relaxed<8, true>), grid, block, 0, s, job);
    else hipLaunchKernelGGL((gemm_relaxed<8, false>), grid, block, 0, s, job);
    break;
  case Q6R:
    if (wc) hipLaunchKernelGGL((gemm_relaxed<6, true>), grid, block, 0, s, job);
    else hipLaunchKernelGGL((gemm_relaxed<6, false>), grid, block, 0, s, job);
    break;
  case T2R:
  case T2: hipLaunchKernelGGL(gemm_ternary, grid, block, 0, s, job); break;
  default: return hipErrorNotSupported;
  }
  return hipGetLastError();
}

}  // namespace hq
