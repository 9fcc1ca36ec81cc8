// gemm.hip — the prompt kernels on the matrix cores (a prompt's many tokens):
//   matmul_q8r_tile (kernels/relaxed/int8.ts:52-166), matmul_q6r for many tokens (jobs.ts:243-248 runs it a token at
//   a time: every (row, token) is matmul_q6r's number), matmul_t2r_tile (kernels/relaxed/signs.ts:232-297).
//
// The matrix core gives each group's exact integer: v_mfma_i32_32x32x32_i8 with K = 32 is one scale group of 32 (for
// ternary, one part of 32 of a group of 128).
//
// Corrections (int8, int6).  The relaxed activations are 7-bit, 0..127 (the second factor of the reference's
// relaxed_dot_i8x16_i7x16, kernels/relaxed/int8.ts:5-10, kernels/ceilings_relaxed.ts:6-8), biased by 64, and the
// reference adds wc = int8_sums(w) = -64 sum(w) to each group's integer.  Staging subtracts the bias from the
// activations (q - 64 lies in -64..63, an int8), so that dot(w, q - 64) is the corrected integer with the MFMA's
// accumulator input 0.  A caller's wc may be anything, though: staging also keeps delta = wc + 64 sum(w) of every
// (row, group), and a stage where any delta of the block is not 0 takes delta as the MFMA's accumulator input
// (dot(w, q - 64) + delta = dot(w, q) + wc, wrapping in int32 as the reference's i32x4.add does).
// Ternary: the accumulator input is interleave()'s sums of the part (one a token), as the reference adds them.
//
// Float32 order: every (row, token) is the token kernel's number to the bit.  The reference's lane k adds groups
// 4 j + k (int8, int6) or part k of every group (ternary), in order, and the four lanes are added
// ((l0 + l1) + l2) + l3 at the end (math.ts:7-9), then (int8, int6) the groups past the last four one at a time
// (relaxed/int8.ts:40-47).  Here a wave IS a lane k of the reference: the 4 waves of one 32 x 32 tile of (rows,
// tokens) take chain k = 0..3 each, adding their groups / parts in order into 16 registers, and at the end add their
// sums in LDS in that order.  Each term is f(f(C) * f(ws * xs)) (int8, int6) or f(f(f(C) * xs) * d) (ternary),
// rounded as the reference rounds it (-ffp-contract=off).
//
// The scales' product of int8 / int6, f(ws * xs) for every (row, token), is an outer product: a
// v_mfma_f32_32x32x2_f32 with K = 2 and its second column zero gives it, each product rounded once as v_mul_f32
// rounds it (subnormals included), on the matrix core.  Roofline: per output element and group the epilogue is then
// 3 VALU operations (convert, multiply, add; ternary 4: f(f(C * xs) * d) has no such product) against 32 MACs on the
// matrix core; CDNA4's VALU does 64 lanes a clock a CU against 4096 int8 MACs, so the epilogue, not the MFMA, bounds
// this kernel (at best 32 / (3 x 4096 / 64) = 16.7 % of dense int8 peak, 12.5 % for ternary).
//
// A block is 8 waves and a 64 x 32 tile of (rows, tokens): two 32 x 32 tiles x four chains.  A stage brings 8 groups
// (int8, int6: two a chain) or 2 groups of 128 (ternary: part k of both for wave k) into LDS, double-buffered: the
// next stage's global loads are in flight while the current one is computed, and a wave issues its second group's
// MFMAs before its first group's epilogue.  Two blocks share a CU (64 KB of LDS each, at most 128 VGPRs a lane).
#include "common.hpp"
#include "launch.hpp"

namespace hq {

namespace {

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int BR = 64, BT = 32;  // block tile: rows x tokens
constexpr int NT = 512;          // threads a block: 2 tiles x 4 chains, a wave each


HQ_DEV v16i zero16i() {
  v16i z;
#pragma unroll
  for (int r = 0; r < 16; r++) z[r] = 0;
  return z;
}
HQ_DEV v16f zero16f() {
  v16f z;
#pragma unroll
  for (int r = 0; r < 16; r++) z[r] = 0.0f;
  return z;
}

// Which tile a block computes.  Blocks are handed to the 8 XCDs in turn (block b to XCD b % 8), and each XCD has
// its own L2: the blocks of one XCD take consecutive tiles, walked in strips of kStrip row tiles with the token tiles
// inside a strip, so that the blocks running on one XCD at a time share their weights' rows and their tokens.
constexpr int kXcds = 8, kStrip = 8;

HQ_DEV void tile_of(int b, int nb, int nrb, int &rb, int &tb) {
  const int q = nb / kXcds, r = nb % kXcds, x = b % kXcds;
  const int t = x * q + min(x, r) + b / kXcds;  // consecutive on one XCD
  const int strip = t / (kStrip * (nb / nrb));
  const int first = strip * kStrip, width = min(kStrip, nrb - first);
  const int in = t - first * (nb / nrb);
  rb = first + in % width;
  tb = in / width;
}

// the 4 chains of a tile added in LDS, ((a0 + a1) + a2) + a3: wave k adds its sum to what waves 0..k-1 left (the
// 16 values of a lane are the same (row, token)s in the four waves of a tile); the sum ends in chain 3's waves.
// `part`: 2 x 64 x 16 floats that no wave reads or writes any more
HQ_DEV void add_chains(float acc[16], float *part, int tile, int chain, int lane) {
  float *p = part + (tile * 64 + lane) * 16;
  for (int k = 0; k < 4; k++) {
    __syncthreads();
    if (chain == k) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        if (k > 0) acc[r] = fadd(p[r], acc[r]);
        if (k < 3) p[r] = acc[r];
      }
    }
  }
}

// Buffer loads: a block's rows, tokens and scales are each one buffer resource (base and size in scalar registers),
// so that a thread's offsets are set once and a stage moves them by a scalar offset alone; a load past the size
// returns zeros and reads nothing (the tiles past the last row or token, groups past the last one: their results are
// never stored).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

HQ_DEV __amdgpu_buffer_rsrc_t resource(const char *base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)min(bytes, (int64_t)0xFFFFFFFF),
                                           0x00020000);
}
HQ_DEV u32x4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0);
}
HQ_DEV u32x2 bload8(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, 0);
}
HQ_DEV uint32_t bload4(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, vo, so, 0);
}
HQ_DEV uint32_t bload2(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, vo, so, 0);
}

// ---------------------------------------------------------------------------------------------------------------
// int8 / int6 weights, relaxed activations (matmul_q8r_tile, matmul_q6r)
// MFMA A = weights (m = row), B = activations less their bias (n = token): lane l holds token l % 32 and rows
// 8 (r / 4) + 4 (l / 32) + r % 4 of its tile's 32 (r = 0..15).
// ---------------------------------------------------------------------------------------------------------------
constexpr int QG = 8;               // groups a stage
constexpr int QROW = QG * 32 + 16;  // an LDS row of a stage's bytes, padded against bank conflicts

struct alignas(16) StageQ {
  char w[BR][QROW];    // the stage's 8 groups of each row, widened to int8
  char x[BT][QROW];    // and of each token, less the bias 64
  float ws[QG][BR];    // the rows' scales, group-major
  int32_t dc[QG][BR];  // delta = wc + 64 sum(w) of each row and group (with the caller's wc only)
  float xs[QG][BT];    // the tokens' scales, group-major
  int32_t nz;          // the number of the last stage held here with a delta not 0 (-1: none)
};

// q - 64 of four 7-bit activations (0..127) in a word, byte by byte: q + 64 has no carry out of its byte, and
// flipping its top bit takes 128 off again
HQ_DEV uint32_t unbias(uint32_t q) { return (q + 0x40404040u) ^ 0x80808080u; }

// the block's view of a job: resources and each thread's offsets into them (thread i: weights of row i / 8, group
// i % 8 of a stage; waves 0..3 also the activations of token i / 8, group i % 8, and their scale; waves 4..7 the
// scales of row (i - 256) / 4, groups 2 ((i - 256) % 4) and + 1)
template <int PACK, bool WC>
struct LoaderQ {
  static constexpr int GB = PACK == 8 ? 32 : 24;  // bytes of a group of weights
  __amdgpu_buffer_rsrc_t rw, rx, rxs, rws, rwc;
  uint32_t ow, ox, oxs, ows, owc;
  uint32_t v[8], x[8];
  int32_t dc;
  float f[2];

  HQ_DEV LoaderQ(const Job &J, int row0, int tok0, int M, int wave) {
    const int i = threadIdx.x, ng = J.n >> 5;
    const int64_t rb = (int64_t)ng * GB;
    rw = resource(J.wq + row0 * rb, (J.r1 - row0) * rb);
    rws = resource(J.ws + (int64_t)row0 * ng * 4, (int64_t)(J.r1 - row0) * ng * 4);
    rwc = resource(J.wc + (int64_t)row0 * ng * 4, WC ? (int64_t)(J.r1 - row0) * ng * 4 : 0);
    rx = resource(J.xq + tok0 * J.frame, (M - 1 - tok0) * J.frame + J.n);
    rxs = resource(J.xs + tok0 * J.sframe, (M - 1 - tok0) * J.sframe + 4 * ng);
    ow = (uint32_t)((i >> 3) * rb + (i & 7) * GB);
    owc = (uint32_t)(((i >> 3) * ng + (i & 7)) * 4);
    ox = (uint32_t)((i >> 3) * J.frame + (i & 7) * 32);
    oxs = (uint32_t)((i >> 3) * J.sframe + (i & 7) * 4);
    ows = (uint32_t)((((i - 256) >> 2) * ng + 2 * ((i - 256) & 3)) * 4);
    (void)wave;
  }

  HQ_DEV void load(int g0, int wave) {
    if (PACK == 8) {
      const u32x4 a = bload16(rw, ow, g0 * GB), b = bload16(rw, ow + 16, g0 * GB);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
      const u32x2 a = bload8(rw, ow, g0 * GB), b = bload8(rw, ow + 8, g0 * GB), c = bload8(rw, ow + 16, g0 * GB);
      const uint32_t d[6] = {a.x, a.y, b.x, b.y, c.x, c.y};
      six_widen(d, v);
    }
    if (WC) dc = (int32_t)bload4(rwc, owc, g0 * 4);
    if (wave < 4) {
      const u32x4 a = bload16(rx, ox, g0 * 32), b = bload16(rx, ox + 16, g0 * 32);
      x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
      f[0] = __uint_as_float(bload4(rxs, oxs, g0 * 4));
    } else {
      f[0] = __uint_as_float(bload4(rws, ows, g0 * 4));
      f[1] = __uint_as_float(bload4(rws, ows + 4, g0 * 4));
    }
  }

  // into S; `number`: the stage's number, kept in S.nz when a delta of it is not 0
  HQ_DEV void store(StageQ &S, int wave, int number) {
    const int i = threadIdx.x;
    {
      const int r = i >> 3, gi = i & 7;
      uint4 *d = (uint4 *)(S.w[r] + 32 * gi);
      d[0] = make_uint4(v[0], v[1], v[2], v[3]);
      d[1] = make_uint4(v[4], v[5], v[6], v[7]);
      if (WC) {
        int32_t s = 0;
#pragma unroll
        for (int q = 0; q < 8; q++) s = sdot4((int32_t)v[q], 0x01010101, s);
        const int32_t delta = (int32_t)((uint32_t)dc + 64u * (uint32_t)s);
        S.dc[gi][r] = delta;
        if (__builtin_amdgcn_ballot_w64(delta != 0) != 0 && (i & 63) == 0) S.nz = number;
      }
    }
    if (wave < 4) {
      const int t = i >> 3, gi = i & 7;
      uint4 *d = (uint4 *)(S.x[t] + 32 * gi);
      d[0] = make_uint4(unbias(x[0]), unbias(x[1]), unbias(x[2]), unbias(x[3]));
      d[1] = make_uint4(unbias(x[4]), unbias(x[5]), unbias(x[6]), unbias(x[7]));
      S.xs[gi][t] = f[0];
    } else {
      const int r = (i - 256) >> 2, gp = (i - 256) & 3;
      S.ws[2 * gp][r] = f[0];
      S.ws[2 * gp + 1][r] = f[1];
    }
  }
};

// group gi of the stage for the lane's tile: its exact integers C (MFMA) and the scales' products (the outer-product
// MFMA: A lane l < 32 the scale of row l, B lane l < 32 the scale of token l, the K = 1 half zero)
struct QTerm {
  v16i c;
  v16f s;
};

template <bool DELTA>
HQ_DEV QTerm q_term(const StageQ &S, int gi, int trow, int lane) {
  QTerm t;
  const v4i A = *(const v4i *)(S.w[trow + (lane & 31)] + 32 * gi + 16 * (lane >> 5));
  const v4i B = *(const v4i *)(S.x[lane & 31] + 32 * gi + 16 * (lane >> 5));
  v16i c0;
  if (DELTA) {
    const int rbase = trow + 4 * (lane >> 5);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int4 c4 = *(const int4 *)&S.dc[gi][rbase + 8 * q];
      c0[4 * q] = c4.x; c0[4 * q + 1] = c4.y; c0[4 * q + 2] = c4.z; c0[4 * q + 3] = c4.w;
    }
  } else {
    c0 = zero16i();
  }
  t.c = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, c0, 0, 0, 0);
  const float wsv = S.ws[gi][trow + (lane & 31)], xsv = S.xs[gi][lane & 31];
  t.s = __builtin_amdgcn_mfma_f32_32x32x2f32(lane < 32 ? wsv : 0.0f, lane < 32 ? xsv : 0.0f, zero16f(), 0, 0, 0);
  return t;
}

HQ_DEV void q_add(float acc[16], const QTerm &t) {
#pragma unroll
  for (int r = 0; r < 16; r++) acc[r] = fadd(acc[r], fmul((float)t.c[r], t.s[r]));
}

// this wave's groups of a stage: gi = chain and chain + 4 (the second only in a full stage), in that order; with the
// deltas (a caller's own corrections, never int8_sums') one group at a time, in fewer registers
template <bool DELTA>
HQ_DEV void q_stage(float acc[16], const StageQ &S, int chain, bool full, int trow, int lane) {
  if (DELTA) {
    q_add(acc, q_term<true>(S, chain, trow, lane));
    if (full) q_add(acc, q_term<true>(S, chain + 4, trow, lane));
    return;
  }
  const QTerm t0 = q_term<false>(S, chain, trow, lane);
  if (full) {
    const QTerm t1 = q_term<false>(S, chain + 4, trow, lane);
    q_add(acc, t0);
    q_add(acc, t1);
  } else {
    q_add(acc, t0);
  }
}

template <int PACK, bool WC>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4))) void gemm_relaxed(Job J) {
  __shared__ StageQ stage[2];
  const int M = J.count;
  const int ng = J.n >> 5, ng4 = ng & ~3;
  int rb, tb;
  tile_of(blockIdx.x, gridDim.x, (J.r1 - J.r0 + BR - 1) / BR, rb, tb);
  const int row0 = J.r0 + rb * BR, tok0 = tb * BT;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = wave >> 2, chain = wave & 3;
  const int trow = 32 * tile;

  float acc[16];
#pragma unroll
  for (int r = 0; r < 16; r++) acc[r] = 0.0f;

  LoaderQ<PACK, WC> L(J, row0, tok0, M, wave);
  if (WC) {
    if (threadIdx.x == 0) stage[0].nz = stage[1].nz = -1;
    __syncthreads();
  }
  const int stages = (ng4 + QG - 1) / QG;  // the last one holds only 4 groups where ng4 % 8 == 4
  if (stages > 0) {
    L.load(0, wave);
    L.store(stage[0], wave, 0);
  }
  __syncthreads();
  for (int j = 0; j < stages; ++j) {
    const StageQ &S = stage[j & 1];
    if (j + 1 < stages) L.load((j + 1) * QG, wave);
    // groups 8 j + chain and 8 j + 4 + chain (relaxed/int8.ts:26-39)
    const bool full = QG * j + 4 < ng4;
    if (WC && __builtin_amdgcn_readfirstlane(S.nz) == j) q_stage<true>(acc, S, chain, full, trow, lane);
    else q_stage<false>(acc, S, chain, full, trow, lane);
    if (j + 1 < stages) L.store(stage[(j + 1) & 1], wave, j + 1);
    __syncthreads();
  }
  add_chains(acc, (float *)&stage[0], tile, chain, lane);
  if (ng4 < ng) {  // the groups past the fours, one at a time, after the four chains' sum (relaxed/int8.ts:40-47)
    L.load(ng4, wave);
    L.store(stage[1], wave, stages);
    __syncthreads();
    if (chain == 3) {
      const StageQ &S = stage[1];
      const bool delta = WC && __builtin_amdgcn_readfirstlane(S.nz) == stages;
      for (int gi = 0; gi < ng - ng4; gi++) {
        if (delta) q_add(acc, q_term<true>(S, gi, trow, lane));
        else q_add(acc, q_term<false>(S, gi, trow, lane));
      }
    }
  }
  if (chain == 3) {
    const int t = tok0 + (lane & 31);
    if (t < M) {
      float *out = (float *)(J.out + t * J.os);
      const int rbase = row0 + trow + 4 * (lane >> 5);
#pragma unroll
      for (int q = 0; q < 4; q++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int row = rbase + 8 * q + e;
          if (row < J.r1) out[row] = acc[4 * q + e];
        }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// ternary (matmul_t2r_tile)
// MFMA A = activations (m = token), B = codes (n = row): lane l holds row l % 32 and tokens 8 (r / 4) + 4 (l / 32)
// + r % 4.  Part k of a group of 128 (block h = k / 2, bytes c = 8 (k % 2) .. + 7 of it) as 32 K values in the order
// plane-major: K-half kh of a lane is planes 2 kh, 2 kh + 1, eight c's each, for the codes and for interleave()'s
// activation bytes 64 h + 16 p + 8 (k % 2) .. + 7 alike.
// ---------------------------------------------------------------------------------------------------------------
constexpr int TG = 2;                 // groups of 128 a stage
constexpr int TWROW = TG * 32 + 16;   // an LDS row of a stage's code bytes
constexpr int TXROW = TG * 128 + 16;  // and of a token's activation bytes

struct alignas(16) StageT {
  char w[BR][TWROW];         // the stage's groups' 32 bytes of each row
  char x[BT][TXROW];         // the stage's groups' 128 interleaved activations of each token
  float xs[TG * 4][BT];      // the tokens' scales of each (group, part)
  int32_t sums[TG * 4][BT];  // and their sums
  float d[TG][BR];           // the rows' group scales, widened
};

// waves 0..3: 16 code bytes (row i / 4, group (i / 2) % 2, half i % 2) and 32 activation bytes (token i / 8, bytes
// 32 (i % 8) of the stage's 256); waves 4..7: the scale and sum of (token (i - 256) / 8, group and part
// (i - 256) % 8), and waves 4, 5 a row's group scale (row (i - 256) / 2, group i % 2)
struct LoaderT {
  __amdgpu_buffer_rsrc_t rw, rx, rxs, rws;
  uint32_t ow, ox, oxs, osu, ows;
  uint4 w, x[2];
  float sc;
  int32_t su;
  uint32_t h;

  HQ_DEV LoaderT(const Job &J, int row0, int tok0, int M) {
    const int i = threadIdx.x, groups = J.n >> 7;
    rw = resource(J.wq + (int64_t)row0 * groups * 32, (int64_t)(J.r1 - row0) * groups * 32);
    rws = resource(J.ws + (int64_t)row0 * groups * 2, (int64_t)(J.r1 - row0) * groups * 2);
    rx = resource(J.xq + tok0 * J.frame, (M - 1 - tok0) * J.frame + J.n);
    rxs = resource(J.xs + tok0 * J.sframe, (M - 1 - tok0) * J.sframe + 8 * (J.n >> 5));
    ow = (uint32_t)((i >> 2) * groups * 32 + ((i >> 1) & 1) * 32 + (i & 1) * 16);
    ox = (uint32_t)((i >> 3) * J.frame + ((i & 7) >> 2) * 128 + 32 * (i & 3));
    const int q = i - 256;
    oxs = (uint32_t)((q >> 3) * J.sframe + (q & 7) * 4);
    osu = oxs + 4 * (J.n >> 5);
    ows = (uint32_t)(((q >> 1) * groups + (q & 1)) * 2);
  }

  HQ_DEV void load(int g0, int wave) {
    if (wave < 4) {
      const u32x4 c = bload16(rw, ow, g0 * 32);
      w = make_uint4(c.x, c.y, c.z, c.w);
      const u32x4 a = bload16(rx, ox, g0 * 128), b = bload16(rx, ox + 16, g0 * 128);
      x[0] = make_uint4(a.x, a.y, a.z, a.w);
      x[1] = make_uint4(b.x, b.y, b.z, b.w);
    } else {
      sc = __uint_as_float(bload4(rxs, oxs, g0 * 16));
      su = (int32_t)bload4(rxs, osu, g0 * 16);
      if (wave < 6) h = bload2(rws, ows, g0 * 2);
    }
  }
  HQ_DEV void store(StageT &S, int wave) const {
    const int i = threadIdx.x;
    if (wave < 4) {
      *(uint4 *)(S.w[i >> 2] + 32 * ((i >> 1) & 1) + 16 * (i & 1)) = w;
      uint4 *d = (uint4 *)(S.x[i >> 3] + 32 * (i & 7));
      d[0] = x[0];
      d[1] = x[1];
    } else {
      const int q = i - 256;
      S.xs[q & 7][q >> 3] = sc;
      S.sums[q & 7][q >> 3] = su;
      if (wave < 6) S.d[q & 1][q >> 1] = half_to_float(h);
    }
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

// part k of group gi of the stage for the lane's tile: its exact integers, starting at interleave()'s sums of the
// lane's 16 tokens
HQ_DEV v16i t_mfma(const StageT &S, int gi, int k, int trow, int lane) {
  const int h = k >> 1, s = k & 1, kh = lane >> 5;
  const char *xp = S.x[lane & 31] + 128 * gi + 64 * h + 8 * s + 32 * kh;
  const uint2 a0 = *(const uint2 *)xp, a1 = *(const uint2 *)(xp + 16);
  v4i A;
  A[0] = (int32_t)a0.x; A[1] = (int32_t)a0.y; A[2] = (int32_t)a1.x; A[3] = (int32_t)a1.y;
  const uint2 wv = *(const uint2 *)(S.w[trow + (lane & 31)] + 32 * gi + 16 * h + 8 * s);
  const v4i B = kh == 0 ? plane_pair<0>(wv.x, wv.y) : plane_pair<2>(wv.x, wv.y);
  const int tbase = 4 * kh;
  v16i C;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int4 c4 = *(const int4 *)&S.sums[4 * gi + k][tbase + 8 * q];
    C[4 * q] = c4.x; C[4 * q + 1] = c4.y; C[4 * q + 2] = c4.z; C[4 * q + 3] = c4.w;
  }
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, C, 0, 0, 0);
}

// f(f(whole * xs) * d) into the part's chain (relaxed/signs.ts:206)
HQ_DEV void t_add(float acc[16], const v16i &C, const StageT &S, int gi, int k, int trow, int lane) {
  const float d = S.d[gi][trow + (lane & 31)];
  const int tbase = 4 * (lane >> 5);
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const float4 x4 = *(const float4 *)&S.xs[4 * gi + k][tbase + 8 * q];
    const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
    for (int e = 0; e < 4; e++) acc[4 * q + e] = fadd(acc[4 * q + e], fmul(fmul((float)C[4 * q + e], xv[e]), d));
  }
}

__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4))) void gemm_ternary(Job J) {
  __shared__ StageT stage[2];
  const int M = J.count;
  const int groups = J.n >> 7;
  int rb, tb;
  tile_of(blockIdx.x, gridDim.x, (J.r1 - J.r0 + BR - 1) / BR, rb, tb);
  const int row0 = J.r0 + rb * BR, tok0 = tb * BT;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = wave >> 2, part = wave & 3;
  const int trow = 32 * tile;

  float acc[16];
#pragma unroll
  for (int r = 0; r < 16; r++) acc[r] = 0.0f;

  LoaderT L(J, row0, tok0, M);
  const int stages = (groups + TG - 1) / TG;
  L.load(0, wave);
  L.store(stage[0], wave);
  __syncthreads();
  for (int j = 0; j < stages; ++j) {
    const StageT &S = stage[j & 1];
    if (j + 1 < stages) L.load((j + 1) * TG, wave);
    // part `part` of groups 2 j and 2 j + 1 (relaxed/signs.ts:198-207)
    const v16i c0 = t_mfma(S, 0, part, trow, lane);
    if (TG * j + 1 < groups) {
      const v16i c1 = t_mfma(S, 1, part, trow, lane);
      t_add(acc, c0, S, 0, part, trow, lane);
      t_add(acc, c1, S, 1, part, trow, lane);
    } else {
      t_add(acc, c0, S, 0, part, trow, lane);
    }
    if (j + 1 < stages) L.store(stage[(j + 1) & 1], wave);
    __syncthreads();
  }
  add_chains(acc, (float *)&stage[0], tile, part, lane);
  if (part == 3) {
    const int rw = row0 + trow + (lane & 31);
    if (rw < J.r1) {
      const int tbase = tok0 + 4 * (lane >> 5);
#pragma unroll
      for (int q = 0; q < 4; q++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int t = tbase + 8 * q + e;
          if (t < M) ((float *)(J.out + t * J.os))[rw] = acc[4 * q + e];
        }
    }
  }
}

}  // namespace

bool gemm_supported(Kind kind) { return kind == Q8R || kind == Q6R || kind == T2R || kind == T2; }

hipError_t launch_gemm(Kind kind, const Job &job, hipStream_t s) {
  const int rows = job.r1 - job.r0;
  if (rows <= 0 || job.count <= 0) return hipSuccess;
  dim3 grid(((rows + BR - 1) / BR) * ((job.count + BT - 1) / BT)), block(NT);
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
