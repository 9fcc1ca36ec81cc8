// blocks.hip — llama.cpp's blocks of 256 weights (kernels/blocks/: types.ts, token.ts, row.ts, tile.ts), the ten
// types Q2_K, Q4_K, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M, IQ4_XS:
//   sb_tables (types.ts:323-348), sums_x (token.ts:149-165), matmul_sbr / matmul_sb (token.ts:111-147: the same
//   numbers), their tile for a prompt (tile.ts:144-147; matmul_sbw_tile's numbers too), sb_row (row.ts), signed_dots
//   (tile.ts:158-162).
//
// A weight is F S W - Fm M (types.ts:32-47).  Every block is decoded 16 weights at a time (a "chunk" h = 0..15) into
// four dwords of W's bytes and its unit's integers, in registers, as the reference reads it (the type's grid and
// the sign table from sb_tables's area, copied into LDS; IQ4_XS's 16 values in registers).  A chunk's integer is
// exact in int32:
//   signed grids:  dot(|W|, a) - 2 dot(|W| of the negative weights, a)  (the sign on the weight, not on a byte add)
//   IQ4_XS, K:     dot(W, a)  (IQ4_XS's W signed, the K types' 0..3 / 0..15)
//   IQ1:           8 dot(code, a) - (7 or 9) (the sum of each 8 activations), by the shift of the 8 (token.ts:93-110)
// then G[k] += S (chunk), M[k] += M (sum of the chunk's 16 activations) for the K types, k = h / 2 the group of 32.
// Float32 (types.ts:48-57, token.ts:100-110): lane k of the reference adds, for every block in order,
//   f(f(f(G[k] xs[k]) + f(G[k+4] xs[k+4])) F), less f(f(f(M[k] xs[k]) + f(M[k+4] xs[k+4])) Fm) for the K types,
// and the four lanes are added in order at the end: a lane of a row here takes a block a step, and the parts go
// through fold.hpp's LDS fold, lane k adding part k of the step's blocks in order, as the ternary kernels do.
// A prompt of fewer than kSbTileMin tokens goes 4 tokens at a time through the same kernel; a longer one through
// the matrix-core tile below (gemm_sb): every (row, token) the token kernel's number either way.
#include "common.hpp"
#include "launch.hpp"
#include "fold.hpp"

namespace hq {

namespace {

// sb_tables's area (types.ts:88-92)
constexpr int T_IQ2XS = 2048, T_IQ2S = 6144, T_IQ3XXS = 14336, T_IQ3S = 15360, T_IQ1S = 17408, T_SIGNS = 33792,
              T_IQ4 = 34816, T_VECTORS = 34864, GRIDS = 33792;
constexpr int Q2_K = 10, Q4_K = 12, IQ2_XXS = 16, IQ2_XS = 17, IQ3_XXS = 18, IQ1_S = 19, IQ3_S = 21, IQ2_S = 22,
              IQ4_XS = 23, IQ1_M = 29;

template <int TY> constexpr bool has_signs() {
  return TY == IQ2_XXS || TY == IQ2_XS || TY == IQ2_S || TY == IQ3_XXS || TY == IQ3_S;
}
template <int TY> constexpr bool has_minimums() { return TY == Q2_K || TY == Q4_K; }
template <int TY> constexpr bool is_iq1() { return TY == IQ1_S || TY == IQ1_M; }

// a block's bytes (its start 2-byte aligned: every type's size is even) as dwords from its first byte.  The aligned
// dwords read are only those holding a byte of the block, so no read leaves the block's own 4-byte words.
template <int BYTES>
struct BlockBytes {
  static constexpr int N = (BYTES + 3) / 4;
  static constexpr int M = (BYTES + 2 + 3) / 4;  // the aligned dwords of a block that starts 2 bytes into one
  uint32_t d[N];
  HQ_DEV void load(const char *p) {
    const uintptr_t a = (uintptr_t)p;
    const uint32_t *q = (const uint32_t *)(a & ~(uintptr_t)3);
    const bool odd = (a & 2) != 0;
    uint32_t r[M];
#pragma unroll
    for (int i = 0; i < M; i++) r[i] = (i < N || odd) ? q[i] : 0u;
#pragma unroll
    for (int i = 0; i < N; i++) d[i] = odd ? __builtin_amdgcn_alignbit(i + 1 < M ? r[i + 1] : 0u, r[i], 16) : r[i];
  }
  // the same from a buffer whose byte `start` (even) is the block's first: M dwords always loaded (past the buffer's
  // end they read 0), the funnel shift 0 or 16 bits: no branch
  HQ_DEV void load(__amdgpu_buffer_rsrc_t r, uint32_t start) {
    const uint32_t a = start & ~3u, shift = (start & 2u) * 8u;
    uint32_t q[M];
#pragma unroll
    for (int i = 0; i < M; i++) q[i] = __builtin_amdgcn_raw_buffer_load_b32(r, (int)(a + 4u * i), 0, 0);
#pragma unroll
    for (int i = 0; i < N; i++) d[i] = __builtin_amdgcn_alignbit(i + 1 < M ? q[i + 1] : 0u, q[i], shift);
  }
  HQ_DEV uint32_t u8(int x) const { return (d[x >> 2] >> (8 * (x & 3))) & 0xffu; }
  HQ_DEV uint32_t u16(int x) const { return (d[x >> 2] >> (8 * (x & 3))) & 0xffffu; }  // x even
  HQ_DEV uint32_t u32(int x) const {                                                  // x even
    return (x & 3) == 0 ? d[x >> 2] : __builtin_amdgcn_alignbit(d[(x >> 2) + 1], d[x >> 2], 16);
  }
};

// 16 bits -> 16 bytes of 0xff where a bit is set, the lowest first (bytesOfBits, types.ts:181-184): dword j of them
HQ_DEV uint32_t bit_bytes(uint32_t bits, int j) {
  uint32_t x = (bits >> (4 * j)) & 15u;
  x = (x | (x << 7) | (x << 14) | (x << 21)) & 0x01010101u;
  return x * 0xffu;
}

HQ_DEV uint2 entry8(const uint8_t *tab, int at) { return *(const uint2 *)(tab + at); }
HQ_DEV uint32_t entry4(const uint8_t *tab, int at) { return *(const uint32_t *)(tab + at); }

// chunk h of a block: W's bytes (magnitudes where the sign is apart, IQ1's codes), 0xff where a weight is negative,
// the unit's S (and M), IQ1's shifts of the two 8s (1: down)
struct Chunk {
  uint32_t mag[4], neg[4];
  int32_t S, M;
  uint32_t down0, down1;
};

// the grid a type reads (its offset in sb_tables's area and its bytes) and whether it reads the sign table
template <int TY> constexpr int grid_at() {
  return TY == IQ2_XXS ? 0 : TY == IQ2_XS ? T_IQ2XS : TY == IQ2_S ? T_IQ2S : TY == IQ3_XXS ? T_IQ3XXS
       : TY == IQ3_S ? T_IQ3S : is_iq1<TY>() ? T_IQ1S : 0;
}
template <int TY> constexpr int grid_bytes() {
  return TY == IQ2_XXS ? 2048 : TY == IQ2_XS ? 4096 : TY == IQ2_S ? 8192 : TY == IQ3_XXS ? 1024 : TY == IQ3_S ? 2048
       : is_iq1<TY>() ? 16384 : 0;
}
template <int TY> constexpr bool reads_signs() { return TY == IQ2_XXS || TY == IQ2_XS || TY == IQ3_XXS; }

// a block's bytes in LDS (its first byte p even: the 2-byte loads are aligned): the same reads as BlockBytes's
struct LdsBytes {
  const uint8_t *p;
  HQ_DEV uint32_t u8(int x) const { return p[x]; }
  HQ_DEV uint32_t u16(int x) const { return *(const uint16_t *)(p + x); }  // x even
  HQ_DEV uint32_t u32(int x) const { return u16(x) | (u16(x + 2) << 16); }   // x even
};

// grid: the type's grid (grid_at's bytes of the area, in LDS or in global memory); signs: the sign table (T_SIGNS);
// B: the block's bytes (BlockBytes in registers, or LdsBytes)
template <int TY, class BB>
HQ_DEV void chunk(const BB &B, int h, const uint8_t *grid, const uint8_t *signs, const uint32_t iq4[4], Chunk &c) {
  const int g = h >> 1;
  c.M = 0;
  c.down0 = c.down1 = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) c.neg[j] = 0;
  if (TY == IQ2_XXS) {  // types.ts:197-200, 227-230, 277
    const int at = 2 + 8 * (h >> 1) + 2 * (h & 1);
    const uint2 e0 = entry8(grid, 8 * (int)B.u8(at)), e1 = entry8(grid, 8 * (int)B.u8(at + 1));
    c.mag[0] = e0.x; c.mag[1] = e0.y; c.mag[2] = e1.x; c.mag[3] = e1.y;
    const uint32_t word = B.u32(6 + 8 * (h >> 1)), aux = word >> (14 * (h & 1));
    const uint2 s0 = entry8(signs, 8 * (int)(aux & 127)), s1 = entry8(signs, 8 * (int)((aux >> 7) & 127));
    c.neg[0] = s0.x; c.neg[1] = s0.y; c.neg[2] = s1.x; c.neg[3] = s1.y;
    c.S = (int32_t)((word >> 27) | 1);
  } else if (TY == IQ2_XS) {  // types.ts:201-204, 232-235, 279
    const uint32_t w0 = B.u16(2 + 4 * h), w1 = B.u16(4 + 4 * h);
    const uint2 e0 = entry8(grid, 8 * (int)(w0 & 511)), e1 = entry8(grid, 8 * (int)(w1 & 511));
    c.mag[0] = e0.x; c.mag[1] = e0.y; c.mag[2] = e1.x; c.mag[3] = e1.y;
    const uint2 s0 = entry8(signs, 8 * (int)(w0 >> 9)), s1 = entry8(signs, 8 * (int)(w1 >> 9));
    c.neg[0] = s0.x; c.neg[1] = s0.y; c.neg[2] = s1.x; c.neg[3] = s1.y;
    c.S = (int32_t)((((B.u8(66 + g) >> (4 * (h & 1))) & 15) << 1) | 1);
  } else if (TY == IQ2_S) {  // types.ts:205-208, 237, 280
    const uint32_t high = B.u8(66 + (h >> 1)) >> (4 * (h & 1));
    const uint32_t i0 = B.u8(2 + 2 * h) | ((high & 3) << 8), i1 = B.u8(3 + 2 * h) | ((high & 12) << 6);
    const uint2 e0 = entry8(grid, 8 * (int)i0), e1 = entry8(grid, 8 * (int)i1);
    c.mag[0] = e0.x; c.mag[1] = e0.y; c.mag[2] = e1.x; c.mag[3] = e1.y;
    const uint32_t bits = B.u16(34 + 2 * h);
#pragma unroll
    for (int j = 0; j < 4; j++) c.neg[j] = bit_bytes(bits, j);
    c.S = (int32_t)((((B.u8(74 + g) >> (4 * (h & 1))) & 15) << 1) | 1);
  } else if (TY == IQ3_XXS) {  // types.ts:209-212, 227-230, 278
#pragma unroll
    for (int j = 0; j < 4; j++) c.mag[j] = entry4(grid, 4 * (int)B.u8(2 + 4 * h + j));
    const uint32_t word = B.u32(66 + 4 * (h >> 1)), aux = word >> (14 * (h & 1));
    const uint2 s0 = entry8(signs, 8 * (int)(aux & 127)), s1 = entry8(signs, 8 * (int)((aux >> 7) & 127));
    c.neg[0] = s0.x; c.neg[1] = s0.y; c.neg[2] = s1.x; c.neg[3] = s1.y;
    c.S = (int32_t)((word >> 27) | 1);
  } else if (TY == IQ3_S) {  // types.ts:213-217, 238, 281
    const uint32_t high = B.u8(66 + (h >> 1)) >> (4 * (h & 1));
#pragma unroll
    for (int j = 0; j < 4; j++)
      c.mag[j] = entry4(grid, 4 * (int)(B.u8(2 + 4 * h + j) | (((high >> j) & 1) << 8)));
    const uint32_t bits = B.u16(74 + 2 * h);
#pragma unroll
    for (int j = 0; j < 4; j++) c.neg[j] = bit_bytes(bits, j);
    c.S = (int32_t)((((B.u8(106 + (h >> 2)) >> (4 * ((h >> 1) & 1))) & 15) << 1) | 1);
  } else if (TY == IQ1_S) {  // types.ts:218-221, 260-261, 282
    const uint32_t word = B.u16(34 + 2 * (h >> 1)), high = word >> (6 * (h & 1));
    const uint32_t i0 = B.u8(2 + 2 * h) | ((high & 7) << 8), i1 = B.u8(3 + 2 * h) | ((high & 56) << 5);
    const uint2 e0 = entry8(grid, 8 * (int)i0), e1 = entry8(grid, 8 * (int)i1);
    c.mag[0] = e0.x; c.mag[1] = e0.y; c.mag[2] = e1.x; c.mag[3] = e1.y;
    c.down0 = c.down1 = word >> 15;
    c.S = (int32_t)((((word >> 12) & 7) << 1) | 1);
  } else if (TY == IQ1_M) {  // types.ts:222-225, 262-264, 283
    const uint32_t high = B.u8(32 + h);
    const uint32_t i0 = B.u8(2 * h) | ((high & 7) << 8), i1 = B.u8(2 * h + 1) | ((high & 0x70) << 4);
    const uint2 e0 = entry8(grid, 8 * (int)i0), e1 = entry8(grid, 8 * (int)i1);
    c.mag[0] = e0.x; c.mag[1] = e0.y; c.mag[2] = e1.x; c.mag[3] = e1.y;
    c.down0 = (high >> 3) & 1;
    c.down1 = high >> 7;
    c.S = (int32_t)((((B.u16(48 + 2 * (h >> 2)) >> (3 * (h & 3))) & 7) << 1) | 1);
  } else if (TY == Q2_K) {  // bits 2 s, 2 s + 1 of byte c of a half's 32 are weight 32 s + c (types.ts:226-229)
    const int at = 16 + 32 * (h >> 3) + 16 * (h & 1), s = (h & 7) >> 1;
#pragma unroll
    for (int j = 0; j < 4; j++) c.mag[j] = (B.u32(at + 4 * j) >> (2 * s)) & 0x03030303u;
    c.S = (int32_t)(B.u8(h) & 15);
    c.M = (int32_t)(B.u8(h) >> 4);
  } else if (TY == Q4_K) {  // of every 32 bytes the low halves are 32 weights, the high halves the next (230-232)
    const int at = 16 + 32 * (h >> 2) + 16 * (h & 1), hi = (h >> 1) & 1;
#pragma unroll
    for (int j = 0; j < 4; j++) c.mag[j] = (B.u32(at + 4 * j) >> (4 * hi)) & 0x0f0f0f0fu;
    c.S = (int32_t)(h < 8 ? (B.u8(4 + g) & 63) : ((B.u8(8 + g) & 15) | ((B.u8(g) >> 6) << 4)));
    c.M = (int32_t)(h < 8 ? (B.u8(8 + g) & 63) : ((B.u8(8 + g) >> 4) | ((B.u8(4 + g) >> 6) << 4)));
  } else {  // IQ4_XS: a group's 16 bytes, low halves its first 16 weights, as IQ4_XS's values (types.ts:233-234)
    const int at = 8 + 16 * (h >> 1), hi = h & 1;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t nb = (B.u32(at + 4 * j) >> (4 * hi)) & 0x0f0f0f0fu;
      const uint32_t sel = nb & 0x07070707u, upper = ((nb >> 3) & 0x01010101u) * 0xffu;
      const uint32_t low = __builtin_amdgcn_perm(iq4[1], iq4[0], sel), high = __builtin_amdgcn_perm(iq4[3], iq4[2], sel);
      c.mag[j] = (low & ~upper) | (high & upper);
    }
    c.S = (int32_t)((((B.u8(4 + (h >> 2)) >> (4 * ((h >> 1) & 1))) & 15) | (((B.u16(2) >> (2 * (h >> 1))) & 3) << 4)) - 32);
  }
}

// the block's F (blockScale, types.ts:302-310) and Fm (blockMinimum, 318-320); d: the block's own float16 (IQ1_M's
// put together from its four words' tops, wholeScale 312-316)
template <int TY, class BB>
HQ_DEV float block_d(const BB &B) {
  if (TY == IQ1_M)
    return half_to_float((B.u16(48) >> 12) | ((B.u16(50) >> 8) & 0xf0u) | ((B.u16(52) >> 4) & 0xf00u) | (B.u16(54) & 0xf000u));
  return half_to_float(B.u16(TY == Q2_K ? 80 : 0));
}
template <int TY, class BB>
HQ_DEV float block_f(const BB &B) {
  const float d = block_d<TY>(B);
  if (TY == IQ2_XXS || TY == IQ2_XS || TY == IQ2_S || TY == IQ1_S || TY == IQ1_M) return fmul(d, 0.125f);
  if (TY == IQ3_XXS) return fmul(d, 0.25f);
  return d;
}
template <int TY, class BB>
HQ_DEV float block_fm(const BB &B) {
  return has_minimums<TY>() ? half_to_float(B.u16(TY == Q2_K ? 82 : 2)) : 0.0f;
}

// ---------------------------------------------------------------------------------------------------------------
// the products (matmul_sbr == matmul_sb): rows of L lanes (16, 4 rows a wave; 64 for rows of 32 blocks or more,
// a row a wave), a block of 256 weights a lane a step.
// The blocks of a launch are persistent: each copies its type's grid and sign table (at most 17 KB) into LDS once,
// and its waves take units (a wave's 64 / L rows) in turn.
// ---------------------------------------------------------------------------------------------------------------
struct SbBatch {
  Job job[kMaxJobs];
  int32_t unit0[kMaxJobs + 1];  // the first group of 4 rows of each job; unit0[njobs]: the groups of the launch
  int32_t njobs;
};

// the job of a unit (the units of the jobs one after the other): counted, not searched, so that no branch comes
// between a wave's loads and their use
HQ_DEV int sb_job_of(const SbBatch &b, int unit) {
  int j = 0;
#pragma unroll
  for (int i = 1; i < kMaxJobs; i++) j += (i < b.njobs && unit >= b.unit0[i]) ? 1 : 0;
  return j;
}

// the lanes of a row: 16, or 64 for rows of kSbLongRow blocks or more (the down projections: four times the waves,
// a step a row)
// lane `lane`'s block of step `it` of unit `unit` (a unit: the R = 64 / L rows of a wave; past the row's blocks,
// its block 0; past the job's rows, its last row), row slot `slot`, loaded through a buffer over the job's rows: its
// base the 4-byte word the weights start in, its size the whole words they take (a word holding a byte of them lies
// in their allocation's pages), so that a load of a word past them reads zeros (the host refuses a matrix of 4 GiB
// or more)
template <int BYTES, int L>
HQ_DEV void sb_load_block(BlockBytes<BYTES> &B, const SbBatch &b, int unit, int it, int slot, int lane) {
  const int jb = sb_job_of(b, unit);
  const Job &J = b.job[jb];
  const int row_u = J.r0 + (unit - b.unit0[jb]) * (64 / L) + slot;
  const int row = row_u < J.r1 ? row_u : J.r1 - 1;
  const int blocks = J.n >> 8, blk = it * L + lane;
  const uintptr_t at = (uintptr_t)J.wq;
  const uint32_t delta = (uint32_t)(at & 3u);
  const int64_t end = delta + (int64_t)J.r1 * blocks * BYTES;
  B.load(resource((const char *)(at - delta), (end + 3) & ~(int64_t)3),
         delta + (uint32_t)(((int64_t)row * blocks + (blk < blocks ? blk : 0)) * BYTES));
}

// COAL (the types of blocks of 128 bytes or more and a multiple of 8, every row of the launch starting on 16 bytes,
// one token staged): a wave's step read as coalesced 16-byte loads instead of a lane's block at a time, then passed
// through LDS to the lanes.  The step is four quarters of 16 blocks, each 16 BYTES contiguous bytes: slot q's row
// (L = 16) or the row's blocks 16 q .. 16 q + 15 of the step (L = 64).  Piece p (16 bytes) of a quarter is loaded by
// lane p % 64 as its load p / 64, a step ahead; at the step the wave writes a quarter's pieces to its LDS buffer and
// that quarter's 16 lanes read their blocks back, quarter after quarter.
// (A lane's own block read directly is 144 bytes from its neighbour's: each of its 37 load instructions touched ~72
// lines.  Measured on the 8B MLP shapes: Q4_K 2.73 -> 3.34 TB/s, IQ4_XS 2.59 -> 2.92; the 2-byte aligned types,
// whose LDS reads take a funnel shift and share the LDS with their grids, 3-13 % slower, so they keep their loads.)
template <int TY> constexpr bool coalesced_type() { return sb_block_bytes(TY) % 8 == 0 && sb_block_bytes(TY) >= 128; }
template <int BYTES>
struct Pieces {
  static constexpr int K = (BYTES + 63) / 64;  // loads a lane a quarter
  uint32_t v[4][K][4];
};
template <int BYTES, int L>
HQ_DEV void sb_load_pieces(Pieces<BYTES> &P, const SbBatch &b, int unit, int it, int wl) {
  constexpr int R = 64 / L;
  const int jb = sb_job_of(b, unit);
  const Job &J = b.job[jb];
  const int blocks = J.n >> 8;
  const __amdgpu_buffer_rsrc_t rs = resource(J.wq, (int64_t)J.r1 * blocks * BYTES);
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int ru = J.r0 + (unit - b.unit0[jb]) * R + (L == 16 ? q : 0);
    const int row = ru < J.r1 ? ru : J.r1 - 1;
    const int first = L == 16 ? it * 16 : it * 64 + 16 * q;
    const uint32_t seg = (uint32_t)(((int64_t)row * blocks + first) * BYTES);
#pragma unroll
    for (int k = 0; k < Pieces<BYTES>::K; k++) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(seg + 16u * (uint32_t)(64 * k + wl)), 0, 0);
#pragma unroll
      for (int e = 0; e < 4; e++) P.v[q][k][e] = (uint32_t)v[e];
    }
  }
}
// the step's pieces to the lanes' blocks through the wave's buffer of 16 BYTES bytes
template <int BYTES>
HQ_DEV void sb_transpose(const Pieces<BYTES> &P, char *buf, BlockBytes<BYTES> &B, int wl) {
  constexpr int N = BlockBytes<BYTES>::N;
  const int mine = wl >> 4;
  const uint32_t start = (uint32_t)(BYTES * (wl & 15));
#pragma unroll
  for (int q = 0; q < 4; q++) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int k = 0; k < Pieces<BYTES>::K; k++) {
      const int p = 64 * k + wl;
      if (p < BYTES) *(uint4 *)(buf + 16 * p) = make_uint4(P.v[q][k][0], P.v[q][k][1], P.v[q][k][2], P.v[q][k][3]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (mine == q) {
      if constexpr (BYTES % 16 == 0) {
#pragma unroll
        for (int i = 0; i < N; i += 4) {
          const uint4 v = *(const uint4 *)(buf + start + 4 * i);
          B.d[i] = v.x; B.d[i + 1] = v.y; B.d[i + 2] = v.z; B.d[i + 3] = v.w;
        }
      } else if constexpr (BYTES % 8 == 0) {
#pragma unroll
        for (int i = 0; i < N; i += 2) {
          const uint2 v = *(const uint2 *)(buf + start + 4 * i);
          B.d[i] = v.x; B.d[i + 1] = v.y;
        }
      } else if constexpr (BYTES % 4 == 0) {
#pragma unroll
        for (int i = 0; i < N; i++) B.d[i] = *(const uint32_t *)(buf + start + 4 * i);
      } else {
        constexpr int M = BlockBytes<BYTES>::M;
        const uint32_t a = start & ~3u, shift = (start & 2u) * 8u;
        uint32_t r[M];
#pragma unroll
        for (int i = 0; i < M; i++) r[i] = *(const uint32_t *)(buf + a + 4 * i);
#pragma unroll
        for (int i = 0; i < N; i++) B.d[i] = __builtin_amdgcn_alignbit(i + 1 < M ? r[i + 1] : 0u, r[i], shift);
      }
    }
  }
}

constexpr int kSbLongRow = 32;
// The staged activations: the 16 lanes of a row read the same bytes of 16 consecutive blocks, which 256 bytes apart
// would all fall in one bank (a 16-way conflict on every read).  A block's 256 bytes take kSbPitch (16 bytes of
// padding: 16 different bank quads), the scales and sums following all the blocks; or, for the types that read the
// sums of 16 or 8 too (the K types, IQ1), a block's activations, 8 scales, 16 sums of 16 and 32 sums of 8 together
// in kSbPitchSums bytes (their reads as far apart: Q4_K 7 % faster, IQ1_S 4 %, the others' 1-2 % slower)
constexpr int kSbPitch = 272, kSbPitchSums = 400;
template <int TY> constexpr bool stages_sums() { return has_minimums<TY>() || is_iq1<TY>(); }
constexpr bool stages_sums(int ty) { return ty == Q2_K || ty == Q4_K || ty == IQ1_S || ty == IQ1_M; }
constexpr size_t sb_stage_bytes(int ty, int n) {
  return stages_sums(ty) ? (size_t)(n >> 8) * kSbPitchSums : (size_t)(n >> 8) * kSbPitch + n / 2;
}
// the most a launch stages of a token's activations (n up to 32768)
constexpr size_t kSbStageMax = 52 * 1024;
constexpr int sb_lanes(int blocks) { return blocks >= kSbLongRow ? 64 : 16; }

template <int TY> constexpr int lds_table_bytes() {
  return grid_bytes<TY>() + (reads_signs<TY>() ? 1024 : 0) > 0 ? grid_bytes<TY>() + (reads_signs<TY>() ? 1024 : 0)
                                                                : 16;
}

// STAGE (one token, and every job of the launch the same activations): the block copies the token's n bytes and
// its n/2 bytes of scales and sums into LDS first, so a step's activations are LDS reads, which the next step's block
// loads in flight do not hold up (a vector memory load waits for every one issued before it).  sb_waves<T>() waves a
// block: the fewer the blocks a CU, the fewer copies of the tables and the activations its LDS is filled with
// (one token: 16 against 4, 3-10 % faster for every type); 2..4 tokens keep 4 (their registers: 16 waves a block
// leave a wave 128)
template <int T> constexpr int sb_waves() { return T == 1 ? 16 : 4; }
template <int TY, int T, int L, bool STAGE, bool COAL>
__global__ __launch_bounds__(64 * sb_waves<T>()) void gemv_sb(SbBatch batch) {
  constexpr int kSbWaves = sb_waves<T>();
  constexpr int R = 64 / L;  // rows a wave
  constexpr int BYTES = sb_block_bytes(TY);
  constexpr int GRID = grid_bytes<TY>();
  __shared__ FoldL<T, L> fold[kSbWaves];
  __shared__ __align__(16) char qbuf[COAL ? kSbWaves * 16 * BYTES : 16];  // COAL: a wave's quarter of a step
  __shared__ __align__(16) uint8_t table[lds_table_bytes<TY>()];
  extern __shared__ __align__(16) char staged[];
  const uint8_t *tab = (const uint8_t *)batch.job[0].ws;  // every job of a launch has the same tables' area
  {
    const uint4 *from = (const uint4 *)(tab + grid_at<TY>());
    for (int i = threadIdx.x; i < GRID / 16; i += 64 * kSbWaves) ((uint4 *)table)[i] = from[i];
    if (reads_signs<TY>())
      for (int i = threadIdx.x; i < 1024 / 16; i += 64 * kSbWaves)
        ((uint4 *)(table + GRID))[i] = ((const uint4 *)(tab + T_SIGNS))[i];
  }
  if (STAGE) {
    const Job &J0 = batch.job[0];
    const int per = J0.n + J0.n / 2, acts = (J0.n >> 8) * kSbPitch, n8 = J0.n >> 3;
    for (int i = threadIdx.x; i < per / 16; i += 64 * kSbWaves) {
      const int o = 16 * i, r = o - J0.n;
      int at;
      if (stages_sums<TY>()) {  // block b's activations, scales, sums of 16, sums of 8 at b kSbPitchSums + 0, 256, 288, 320
        if (o < J0.n) at = (o >> 8) * kSbPitchSums + (o & 255);
        else if (r < n8) at = (r >> 5) * kSbPitchSums + 256 + (r & 31);
        else if (r < 2 * n8) at = ((r - n8) >> 5) * kSbPitchSums + 288 + ((r - n8) & 31);
        else at = ((r - 2 * n8) >> 6) * kSbPitchSums + 320 + ((r - 2 * n8) & 63);
      } else {
        at = o < J0.n ? (o >> 8) * kSbPitch + (o & 255) : acts + r;
      }
      *(uint4 *)(staged + at) = *(const uint4 *)(o < J0.n ? J0.xq + o : J0.xs + r);
    }
  }
  uint32_t iq4[4] = {0u, 0u, 0u, 0u};
  if (TY == IQ4_XS) {
    const uint4 v = *(const uint4 *)(tab + T_IQ4);
    iq4[0] = v.x; iq4[1] = v.y; iq4[2] = v.z; iq4[3] = v.w;
  }
  __syncthreads();
  const int lane = threadIdx.x & (L - 1);
  // the wave's number as a scalar: its units, jobs and buffers are then the wave's own (scalar registers)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), slot = (threadIdx.x & 63) / L;
  FoldL<T, L> &f = fold[wave];
  const int units = batch.unit0[batch.njobs], stride = gridDim.x * kSbWaves;
  int unit = blockIdx.x * kSbWaves + wave, it = 0, count = 0;
  if (unit >= units) return;  // (no barrier follows)
  // a wave's steps one after the other (a step: a unit's rows, a block a lane), the next step's blocks loaded before
  // this one is decoded; past the wave's last step it loads this step's blocks again, so every step issues the same
  // loads and a step's decode waits only for its own
  BlockBytes<BYTES> B;
  Pieces<BYTES> P;
  const int wl = threadIdx.x & 63;
  if (COAL) sb_load_pieces<BYTES, L>(P, batch, unit, it, wl);
  else sb_load_block<BYTES, L>(B, batch, unit, it, slot, lane);
  float acc[T];
#pragma unroll
  for (int t = 0; t < T; t++) acc[t] = 0.0f;
  for (;;) {
    const int jb = sb_job_of(batch, unit);
    const Job &J = batch.job[jb];
    const int row_u = J.r0 + (unit - batch.unit0[jb]) * R + slot;
    const bool live = row_u < J.r1;
    const int row = live ? row_u : J.r1 - 1;
    const int blocks = J.n >> 8, steps = (blocks + L - 1) / L;
    const bool last = it + 1 >= steps;
    const int next_unit = last ? unit + stride : unit, next_it = last ? 0 : it + 1;
    const bool more = next_unit < units;
    BlockBytes<BYTES> Bn;
    if (COAL) {  // this step's blocks out of the pieces, then the next step's pieces in flight
      sb_transpose<BYTES>(P, qbuf + wave * 16 * BYTES, B, wl);
      sb_load_pieces<BYTES, L>(P, batch, more ? next_unit : unit, more ? next_it : it, wl);
    } else {
      sb_load_block<BYTES, L>(Bn, batch, more ? next_unit : unit, more ? next_it : it, slot, lane);
    }
    // token t's activations (n int8), its scales (n / 32 float32), its sums of 16 and of 8 (int16)
    const int8_t *xq[T];
    const float *xs[T];
    const int16_t *s16[T], *s8[T];
#pragma unroll
    for (int t = 0; t < T; t++) {
      xq[t] = STAGE ? (const int8_t *)staged : (const int8_t *)(J.xq + t * J.frame);
      xs[t] = STAGE && !stages_sums<TY>() ? (const float *)(staged + (J.n >> 8) * kSbPitch)
                                          : (const float *)(J.xs + t * J.sframe);
      s16[t] = (const int16_t *)(xs[t] + (J.n >> 5));
      s8[t] = s16[t] + (J.n >> 4);
    }
    const int b = it * L + lane;
    const bool valid = b < blocks;
    const int bl = valid ? b : 0;
    // the staged copy of block bl's activations, and of its scales and sums (stages_sums)
    constexpr int PITCH = STAGE ? (stages_sums<TY>() ? kSbPitchSums : kSbPitch) : 256;
    const char *sblk = staged + PITCH * bl;
    int32_t G[T][8], Mi[T][8];
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
      for (int k = 0; k < 8; k++) G[t][k] = Mi[t][k] = 0;
#pragma unroll
    for (int h = 0; h < 16; h++) {
      Chunk c;
      chunk<TY>(B, h, table, table + GRID, iq4, c);
      uint32_t signed_part[4];
#pragma unroll
      for (int j = 0; j < 4; j++) signed_part[j] = c.mag[j] & c.neg[j];
#pragma unroll
      for (int t = 0; t < T; t++) {
        const uint4 av = *(const uint4 *)((const char *)xq[t] + PITCH * bl + 16 * h);
        const int32_t a[4] = {(int32_t)av.x, (int32_t)av.y, (int32_t)av.z, (int32_t)av.w};
        int32_t d = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) d = sdot4((int32_t)c.mag[j], a[j], d);
        if (has_signs<TY>()) {
          int32_t e = 0;
#pragma unroll
          for (int j = 0; j < 4; j++) e = sdot4((int32_t)signed_part[j], a[j], e);
          d -= 2 * e;
        }
        if (is_iq1<TY>()) {  // 8 dot(code, a) - (7 + 2 down) sum of each 8 (token.ts:93-99, 117-127)
          const int16_t *s8b = STAGE ? (const int16_t *)(sblk + 320) : s8[t] + 32 * bl;
          const int32_t e0 = s8b[2 * h], e1 = s8b[2 * h + 1];
          d = 8 * d - (7 + 2 * (int32_t)c.down0) * e0 - (7 + 2 * (int32_t)c.down1) * e1;
        }
        G[t][h >> 1] += c.S * d;
        if (has_minimums<TY>())
          Mi[t][h >> 1] += c.M * (int32_t)(STAGE ? (const int16_t *)(sblk + 288) : s16[t] + 16 * bl)[h];
      }
    }
    const float F = block_f<TY>(B), Fm = block_fm<TY>(B);
#pragma unroll
    for (int t = 0; t < T; t++) {
      const float *xsb = STAGE && stages_sums<TY>() ? (const float *)(sblk + 256) : xs[t] + 8 * bl;
      const float4 x0 = *(const float4 *)xsb, x1 = *(const float4 *)(xsb + 4);
      const float sl[4] = {x0.x, x0.y, x0.z, x0.w}, sh[4] = {x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int k = 0; k < 4; k++) {
        float part = fmul(fadd(fmul((float)G[t][k], sl[k]), fmul((float)G[t][k + 4], sh[k])), F);
        if (has_minimums<TY>())
          part = fsub(part, fmul(fadd(fmul((float)Mi[t][k], sl[k]), fmul((float)Mi[t][k + 4], sh[k])), Fm));
        f.v[count & 1][slot][t][k][lane] = valid ? part : 0.0f;  // +0 leaves a lane as it is: a lane is never -0
      }
    }
    fold_step_l<T, L>(f, count & 1, slot, lane, acc);
    ++count;
    if (last) {
      // lanes 0..3 hold the four lanes' sums: ((l0 + l1) + l2) + l3 in lane 0 (math.ts:7-9)
      float sum[T];
#pragma unroll
      for (int t = 0; t < T; t++)
        sum[t] = fadd(fadd(fadd(acc[t], from_lane_plus<1>(acc[t])), from_lane_plus<2>(acc[t])),
                      from_lane_plus<3>(acc[t]));
      if (live && lane == 0) {
#pragma unroll
        for (int t = 0; t < T; t++) ((float *)(J.out + t * J.os))[row] = sum[t];
      }
#pragma unroll
      for (int t = 0; t < T; t++) acc[t] = 0.0f;
    }
    if (!more) break;
    unit = next_unit;
    it = next_it;
    if (!COAL) B = Bn;
  }
}

// a launch's blocks: as many as stay resident together (at most the units over the waves a block); lds: the staged
// activations' bytes (0: none)
template <int TY, int T, int L, bool STAGE, bool COAL>
hipError_t launch_tt(const SbBatch &b, size_t lds, hipStream_t s) {
  static int per_cu[64][16];  // by device and 4 KB of staged bytes
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  const int slot = (int)(lds / 4096) < 16 ? (int)(lds / 4096) : 15;
  if (per_cu[dev][slot] == 0) {
    int k = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&k, gemv_sb<TY, T, L, STAGE, COAL>, 64 * sb_waves<T>(),
                                                     4096 * (slot + 1)) !=
            hipSuccess || k < 1)
      k = 1;
    per_cu[dev][slot] = k;
  }
  constexpr int W = sb_waves<T>();
  const int want = (b.unit0[b.njobs] + W - 1) / W, cap = per_cu[dev][slot] * cu_count();
  hipLaunchKernelGGL((gemv_sb<TY, T, L, STAGE, COAL>), dim3(want < cap ? want : cap), dim3(64 * W), lds, s, b);
  return hipGetLastError();
}

template <int TY>
hipError_t launch_type(const SbBatch &b, int T, int L, size_t lds, hipStream_t s) {
  switch (T) {
  case 1:
    if (lds) {
      if constexpr (coalesced_type<TY>()) {
        bool coal = true;  // every job's rows start on 16 bytes: the weights' base and a row's bytes
        for (int j = 0; j < b.njobs; j++) {
          const int64_t row_bytes = (int64_t)(b.job[j].n >> 8) * sb_block_bytes(TY);
          coal = coal && ((uintptr_t)b.job[j].wq & 15u) == 0 && row_bytes % 16 == 0;
        }
        if (coal)
          return L == 64 ? launch_tt<TY, 1, 64, true, true>(b, lds, s) : launch_tt<TY, 1, 16, true, true>(b, lds, s);
      }
      return L == 64 ? launch_tt<TY, 1, 64, true, false>(b, lds, s) : launch_tt<TY, 1, 16, true, false>(b, lds, s);
    }
    return L == 64 ? launch_tt<TY, 1, 64, false, false>(b, 0, s) : launch_tt<TY, 1, 16, false, false>(b, 0, s);
  case 2: return launch_tt<TY, 2, 16, false, false>(b, 0, s);
  case 3: return launch_tt<TY, 3, 16, false, false>(b, 0, s);
  case 4: return launch_tt<TY, 4, 16, false, false>(b, 0, s);
  default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------------------------------------------
// the prompt tile (matmul_sbr_tile / matmul_sbw_tile for kSbTileMin tokens or more): a block takes 32 rows x NT
// tokens (NT 32, 64 or 128).  For each block of 256 weights it stages the tokens' activations (with their scales and
// sums) and the rows' raw blocks into LDS, decodes the 32 blocks once (two chunks of 16 a thread, the token kernel's
// decoder reading the LDS copy) into int8 tiles, and multiplies them on the matrix cores:
// v_mfma_i32_32x32x32_i8, A = 32 tokens, B = the 32 rows, K = 32 = a group, so a lane holds one row (l % 32) and 16
// tokens (8 (r / 4) + 4 (l / 32) + r % 4).  The integers are exactly the token kernel's:
//   signed grids: W ^ neg (W where the sign is plus, ~W = -W - 1 where it is minus: always an int8) and neg's 0 / 1
//   in two tiles, d = C(W ^ neg) + C(neg & 1), the second product added in the first's accumulator;
//   a scale S for each 16 (IQ2_XS, IQ2_S, IQ1_M): two products a group, B zero in one half of the lanes (K 0..15
//   is lanes 0..31's, K 16..31 lanes 32..63's), G = S_lo d_lo + S_hi d_hi; Q2_K's S W (at most 45) is its tile;
//   IQ1: C of the codes and C of a second tile holding -(7 + 2 down) for each 8 weights, d = 8 C + C(corr) = 8
//   dot(code, a) - (7 + 2 down) (sum of each 8); the K types' M against the sums of 16 (an f32 outer product on the
//   matrix core, K = 2: the two chunks of the group);
// then each (row, token) adds f(f(f(G_k xs_k) + f(G_{k+4} xs_{k+4})) F) (less the minimums') to its lane k in block
// order, and ((l0 + l1) + l2) + l3 at the end (types.ts:48-57): every (row, token) the token kernel's number.
// The four waves split the tokens and the lanes k: NT = 128, 32 tokens and all four lanes a wave; NT = 64, two token
// halves x two pairs of lanes; NT = 32, a lane k a wave; the lanes meet in LDS at the end in that order.  The next
// block's bytes are loaded into registers while this one is decoded and multiplied, and stored into LDS after.
// ---------------------------------------------------------------------------------------------------------------
typedef int32_t v4i_t __attribute__((ext_vector_type(4)));
typedef int32_t v16i_t __attribute__((ext_vector_type(16)));
typedef float v16f_t __attribute__((ext_vector_type(16)));

constexpr int SBT_R = 32;            // a block's rows
constexpr int SBT_PITCH = 256 + 16;  // an LDS row of a block's 256 bytes (16 more: 16-byte reads of rows apart)

template <int TY> constexpr bool tile_signed() { return has_signs<TY>(); }
template <int TY> constexpr bool tile_split() { return TY == IQ2_XS || TY == IQ2_S || TY == IQ1_M; }
template <int TY> constexpr bool tile_sums16() { return has_minimums<TY>(); }
// a second int8 tile: neg's 0 / 1 (signed grids) or IQ1's -(7 + 2 down) for each 8 weights
template <int TY> constexpr bool tile_second() { return has_signs<TY>() || is_iq1<TY>(); }
// the types with a 128-token tile (one scale a group, no sums: two waves a SIMD still fit; the others measured
// slower at 128 than at 64)
template <int TY> constexpr bool tile_wide() { return !tile_sums16<TY>() && !tile_split<TY>(); }

template <int TY, int NT>
struct SbTileLayout {
  static constexpr int BYTES = sb_block_bytes(TY);
  static constexpr int WORDS = (BYTES + 2 + 3) / 4;  // the aligned words that hold a block
  static constexpr int RAWP = 4 * WORDS;
  static constexpr int X = 0;                                              // int8 [NT][SBT_PITCH]
  static constexpr int XS = X + NT * SBT_PITCH;                            // float [8][NT]
  static constexpr int S16 = XS + 8 * NT * 4;                              // int32 [16][NT] (K)
  static constexpr int RAW = S16 + (tile_sums16<TY>() ? 16 * NT * 4 : 0);  // bytes [SBT_R][RAWP]
  static constexpr int WM = RAW + SBT_R * RAWP;                            // int8 [SBT_R][SBT_PITCH]
  static constexpr int WN = WM + SBT_R * SBT_PITCH;                        // int8 [SBT_R][SBT_PITCH] (tile_second)
  static constexpr int RS = WN + (tile_second<TY>() ? SBT_R * SBT_PITCH : 0);  // int8 [SBT_R][16] S
  static constexpr int RM = RS + SBT_R * 16;                               // int8 [SBT_R][16] M
  static constexpr int FF = RM + SBT_R * 16;                               // float [SBT_R] F, then [SBT_R] Fm
  static constexpr int GRIDS = FF + 2 * SBT_R * 4;                         // the type's grid and sign table
  static constexpr int SIZE = GRIDS + lds_table_bytes<TY>();
  // the lanes' sums at the end, over X .. : NT = 64, l0 + l1 [SBT_R][NT]; NT = 32, l0, l1, l2 [3][SBT_R][NT]
  static constexpr int LANES = (NT == 128 ? 0 : NT == 64 ? 1 : 3) * SBT_R * NT * 4;
  static_assert(LANES <= GRIDS, "the lanes' sums fit below the grids");
  // the loads of a block a thread: the tokens' bytes (16 a load), their scales and sums (16 bytes a load), the raw
  // blocks' words
  static constexpr int XU = NT * 16 / 256;
  static constexpr int AUX = NT * (2 + (tile_sums16<TY>() ? 2 : 0));
  static constexpr int AU = (AUX + 255) / 256;
  static constexpr int RU = (SBT_R * WORDS + 255) / 256;
};

HQ_DEV int32_t sbyte(uint32_t w, int i) { return (int32_t)(int8_t)(uint8_t)(w >> (8 * i)); }

// a block's loads in flight: block b's bytes of the tile's tokens and rows, in registers
template <int TY, int NT>
struct TileLoads {
  using Lay = SbTileLayout<TY, NT>;
  v4i_t x[Lay::XU], aux[Lay::AU];
  uint32_t raw[Lay::RU];
};

template <int TY, int NT>
HQ_DEV void tile_load(TileLoads<TY, NT> &L, int tid, int b, __amdgpu_buffer_rsrc_t rq, __amdgpu_buffer_rsrc_t ra,
                      __amdgpu_buffer_rsrc_t rw, int64_t frame, int64_t sframe, int n, int blocks, int r0, int r1,
                      uint32_t wdelta) {
  using Lay = SbTileLayout<TY, NT>;
  constexpr int BYTES = Lay::BYTES, WORDS = Lay::WORDS;
#pragma unroll
  for (int u = 0; u < Lay::XU; u++) {
    const int idx = tid + 256 * u, tok = idx >> 4, q = idx & 15;
    L.x[u] = __builtin_amdgcn_raw_buffer_load_b128(rq, (int)(tok * frame + 256 * b + 16 * q), 0, 0);
  }
#pragma unroll
  for (int u = 0; u < Lay::AU; u++) {
    // a < 2 NT: the scales (token a / 2, half a % 2); then the K types' sums of 16
    const int a0 = tid + 256 * u, a = a0 < Lay::AUX ? a0 : Lay::AUX - 1;
    const int off = a < 2 * NT ? (a >> 1) * (int)sframe + 32 * b + 16 * (a & 1)
                               : ((a - 2 * NT) >> 1) * (int)sframe + 4 * (n >> 5) + 32 * b + 16 * (a & 1);
    L.aux[u] = __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0);
  }
#pragma unroll
  for (int u = 0; u < Lay::RU; u++) {
    const int i0 = tid + 256 * u, idx = i0 < SBT_R * WORDS ? i0 : SBT_R * WORDS - 1;
    const int r = idx / WORDS, w = idx - r * WORDS;
    const int row = r0 + r < r1 ? r0 + r : r1 - 1;
    const uint32_t start = wdelta + (uint32_t)(((int64_t)row * blocks + b) * BYTES);
    L.raw[u] = __builtin_amdgcn_raw_buffer_load_b32(rw, (int)((start & ~3u) + 4u * w), 0, 0);
  }
}

template <int TY, int NT>
HQ_DEV void tile_store(const TileLoads<TY, NT> &L, int tid, char *lds) {
  using Lay = SbTileLayout<TY, NT>;
  constexpr int WORDS = Lay::WORDS;
  int8_t *x = (int8_t *)(lds + Lay::X);
  float *xsT = (float *)(lds + Lay::XS);
  int32_t *s16T = (int32_t *)(lds + Lay::S16);
#pragma unroll
  for (int u = 0; u < Lay::XU; u++) {
    const int idx = tid + 256 * u, tok = idx >> 4, q = idx & 15;
    *(v4i_t *)(x + tok * SBT_PITCH + 16 * q) = L.x[u];
  }
#pragma unroll
  for (int u = 0; u < Lay::AU; u++) {
    const int a = tid + 256 * u;  // (the kinds change at multiples of 64: a wave takes one)
    const v4i_t v = L.aux[u];
    if (a < 2 * NT) {
      const int tok = a >> 1, half = a & 1;
#pragma unroll
      for (int i = 0; i < 4; i++) xsT[(4 * half + i) * NT + tok] = __int_as_float(v[i]);
    } else if (a < Lay::AUX) {
      const int tok = (a - 2 * NT) >> 1, half = a & 1;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        s16T[(8 * half + 2 * i) * NT + tok] = (int32_t)(int16_t)(v[i] & 0xffff);
        s16T[(8 * half + 2 * i + 1) * NT + tok] = (int32_t)(int16_t)((uint32_t)v[i] >> 16);
      }
    }
  }
  uint8_t *raw = (uint8_t *)(lds + Lay::RAW);
#pragma unroll
  for (int u = 0; u < Lay::RU; u++) {
    const int idx = tid + 256 * u;
    if (idx < SBT_R * WORDS) {
      const int r = idx / WORDS, w = idx - r * WORDS;
      *(uint32_t *)(raw + r * Lay::RAWP + 4 * w) = L.raw[u];
    }
  }
}

template <int TY, int NT>
__global__ __launch_bounds__(256) void gemm_sb(Job J) {
  using Lay = SbTileLayout<TY, NT>;
  constexpr int BYTES = Lay::BYTES, GRID = grid_bytes<TY>();
  constexpr int TH = NT / 32;  // the waves' token slices; also the lanes k a wave
  extern __shared__ __align__(16) char lds[];
  const int8_t *x = (const int8_t *)(lds + Lay::X);
  const float *xsT = (const float *)(lds + Lay::XS);
  const int32_t *s16T = (const int32_t *)(lds + Lay::S16);
  const uint8_t *raw = (const uint8_t *)(lds + Lay::RAW);
  int8_t *wm = (int8_t *)(lds + Lay::WM), *wn = (int8_t *)(lds + Lay::WN);
  int8_t *rs = (int8_t *)(lds + Lay::RS), *rm = (int8_t *)(lds + Lay::RM);
  float *ff = (float *)(lds + Lay::FF);
  uint8_t *table = (uint8_t *)(lds + Lay::GRIDS);

  const int tid = threadIdx.x;
  const int nrt = (J.r1 - J.r0 + SBT_R - 1) / SBT_R;
  const int rt = blockIdx.x % nrt, tt = blockIdx.x / nrt;
  const int r0 = J.r0 + SBT_R * rt, t0 = NT * tt;
  const int blocks = J.n >> 8;
  // the type's grid and sign table, and IQ4_XS's values
  const uint8_t *tab = (const uint8_t *)J.ws;
  for (int i = tid; i < GRID / 16; i += 256) ((uint4 *)table)[i] = ((const uint4 *)(tab + grid_at<TY>()))[i];
  if (reads_signs<TY>())
    for (int i = tid; i < 1024 / 16; i += 256) ((uint4 *)(table + GRID))[i] = ((const uint4 *)(tab + T_SIGNS))[i];
  uint32_t iq4[4] = {0u, 0u, 0u, 0u};
  if (TY == IQ4_XS) {
    const uint4 v = *(const uint4 *)(tab + T_IQ4);
    iq4[0] = v.x; iq4[1] = v.y; iq4[2] = v.z; iq4[3] = v.w;
  }
  // buffers: the tile's tokens (a token past the prompt reads zeros) and the weights (the aligned words of rows
  // 0 .. r1 - 1)
  const int64_t tokens_left = (int64_t)J.count - t0;
  const __amdgpu_buffer_rsrc_t rq = resource(J.xq + t0 * J.frame, tokens_left * J.frame);
  const __amdgpu_buffer_rsrc_t ra = resource(J.xs + t0 * J.sframe, tokens_left * J.sframe);
  const uintptr_t wat = (uintptr_t)J.wq;
  const uint32_t wdelta = (uint32_t)(wat & 3u);
  const int64_t wend = wdelta + (int64_t)J.r1 * blocks * BYTES;
  const __amdgpu_buffer_rsrc_t rw = resource((const char *)(wat - wdelta), (wend + 3) & ~(int64_t)3);
  // this thread's row for the decode: tile row tid / 8 (past the job's rows: its last), chunks 2 (tid % 8), + 1
  const int dr = tid >> 3, dq = tid & 7;
  const int drow = r0 + dr < J.r1 ? r0 + dr : J.r1 - 1;
  // the wave's tokens 32 th .. and lanes k0 .. k0 + TH - 1; the lane's row, and its 16 tokens' first of each four
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, kh = lane >> 5, l32 = lane & 31;
  const int th = wave % TH, k0 = (wave / TH) * TH;
  const int mrow = l32, mtok = 32 * th + l32;
  float acc[TH][16];
#pragma unroll
  for (int kk = 0; kk < TH; kk++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[kk][r] = 0.0f;

  TileLoads<TY, NT> loads;
  tile_load<TY, NT>(loads, tid, 0, rq, ra, rw, J.frame, J.sframe, J.n, blocks, r0, J.r1, wdelta);
  for (int b = 0; b < blocks; b++) {
    __syncthreads();  // (the last block's tiles read)
    tile_store<TY, NT>(loads, tid, lds);
    // the next block's loads (the last block's again at the end: not used)
    tile_load<TY, NT>(loads, tid, b + 1 < blocks ? b + 1 : b, rq, ra, rw, J.frame, J.sframe, J.n, blocks, r0, J.r1,
                      wdelta);
    __syncthreads();
    // ---- decode: this thread's two chunks of its row's block into the tiles
    {
      const uint32_t start = wdelta + (uint32_t)(((int64_t)drow * blocks + b) * BYTES);
      const LdsBytes B{raw + dr * Lay::RAWP + (start & 2u)};
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int h = 2 * dq + u;
        Chunk c;
        chunk<TY>(B, h, table, table + GRID, iq4, c);
        uint32_t m4[4];
#pragma unroll
        for (int j = 0; j < 4; j++) m4[j] = TY == Q2_K ? c.mag[j] * (uint32_t)c.S : c.mag[j];  // (S W <= 45)
        if (tile_signed<TY>()) {
          *(uint4 *)(wm + dr * SBT_PITCH + 16 * h) =
              make_uint4(c.mag[0] ^ c.neg[0], c.mag[1] ^ c.neg[1], c.mag[2] ^ c.neg[2], c.mag[3] ^ c.neg[3]);
          *(uint4 *)(wn + dr * SBT_PITCH + 16 * h) = make_uint4(c.neg[0] & 0x01010101u, c.neg[1] & 0x01010101u,
                                                                c.neg[2] & 0x01010101u, c.neg[3] & 0x01010101u);
        } else {
          *(uint4 *)(wm + dr * SBT_PITCH + 16 * h) = make_uint4(m4[0], m4[1], m4[2], m4[3]);
        }
        if (is_iq1<TY>()) {  // -(7 + 2 down) for each 8 weights of the chunk
          const uint32_t e0 = (uint32_t)(uint8_t)(int8_t)(-7 - 2 * (int32_t)c.down0) * 0x01010101u;
          const uint32_t e1 = (uint32_t)(uint8_t)(int8_t)(-7 - 2 * (int32_t)c.down1) * 0x01010101u;
          *(uint4 *)(wn + dr * SBT_PITCH + 16 * h) = make_uint4(e0, e0, e1, e1);
        }
        rs[dr * 16 + h] = (int8_t)c.S;
        rm[dr * 16 + h] = (int8_t)c.M;
      }
      if (dq == 0) {
        ff[dr] = block_f<TY>(B);
        ff[SBT_R + dr] = block_fm<TY>(B);
      }
    }
    __syncthreads();
    // ---- the products: the wave's 32 x 32 for its lanes k, group pairs (k, k + 4)
    const float F = ff[mrow], Fm = ff[SBT_R + mrow];
    const uint4 S4 = *(const uint4 *)(rs + mrow * 16), M4 = *(const uint4 *)(rm + mrow * 16);
    const uint32_t Sw[4] = {S4.x, S4.y, S4.z, S4.w}, Mw[4] = {M4.x, M4.y, M4.z, M4.w};
#pragma unroll
    for (int kk = 0; kk < TH; kk++) {
      const int k = k0 + kk;
      float q0[16], qm0[16];  // group k's f(G xs) and f(M xs)
#pragma unroll
      for (int e = 0; e < 2; e++) {
        const int gg = k + 4 * e, c0 = 2 * gg, c1 = 2 * gg + 1;
        const v4i_t A = *(const v4i_t *)(x + mtok * SBT_PITCH + 32 * gg + 16 * kh);
        const v4i_t Bm = *(const v4i_t *)(wm + mrow * SBT_PITCH + 32 * gg + 16 * kh);
        const v16i_t zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
        const int32_t S0 = sbyte(Sw[c0 >> 2], c0 & 3), S1 = sbyte(Sw[c1 >> 2], c1 & 3);
        int32_t G[16];
        if (tile_split<TY>()) {
          const v4i_t z4 = {0, 0, 0, 0};
          v16i_t lo = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, kh == 0 ? Bm : z4, zero, 0, 0, 0);
          v16i_t hi = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, kh == 1 ? Bm : z4, zero, 0, 0, 0);
          if (tile_signed<TY>()) {
            const v4i_t Bn = *(const v4i_t *)(wn + mrow * SBT_PITCH + 32 * gg + 16 * kh);
            lo = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, kh == 0 ? Bn : z4, lo, 0, 0, 0);
            hi = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, kh == 1 ? Bn : z4, hi, 0, 0, 0);
          }
          if (is_iq1<TY>()) {  // 8 dot(code, a) - (7 + 2 down) (sum of each 8), for each of the two 16s
            const v4i_t Bc = *(const v4i_t *)(wn + mrow * SBT_PITCH + 32 * gg + 16 * kh);
            const v16i_t clo = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, kh == 0 ? Bc : z4, zero, 0, 0, 0);
            const v16i_t chi = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, kh == 1 ? Bc : z4, zero, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; r++) {
              lo[r] = 8 * lo[r] + clo[r];
              hi[r] = 8 * hi[r] + chi[r];
            }
          }
#pragma unroll
          for (int r = 0; r < 16; r++) G[r] = __mul24(S0, lo[r]) + __mul24(S1, hi[r]);  // (|lo|, |hi| < 2^23)
        } else {
          v16i_t C = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, Bm, zero, 0, 0, 0);
          if (tile_signed<TY>()) {
            const v4i_t Bn = *(const v4i_t *)(wn + mrow * SBT_PITCH + 32 * gg + 16 * kh);
            C = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, Bn, C, 0, 0, 0);
          }
          if (is_iq1<TY>()) {  // IQ1_S: one shift for the 32, against the sum of the 32
            const v4i_t Bc = *(const v4i_t *)(wn + mrow * SBT_PITCH + 32 * gg + 16 * kh);
            const v16i_t Cc = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, Bc, zero, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; r++) C[r] = 8 * C[r] + Cc[r];
          }
#pragma unroll
          for (int r = 0; r < 16; r++) G[r] = TY == Q2_K ? C[r] : __mul24(S0, C[r]);
        }
        v16f_t Mf;  // M0 v0 + M1 v1 (the K types' minimums against the sums of 16), exact in float32: |.| < 2^18
        if (has_minimums<TY>()) {  // an outer product with K = 2: A the tokens' sums of chunks c0 (lanes 0..31) and
                                   // c1 (32..63), B the row's M of the same chunks
          const int c = kh ? c1 : c0;
          const v16f_t z = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
          Mf = __builtin_amdgcn_mfma_f32_32x32x2f32((float)s16T[c * NT + mtok], (float)sbyte(Mw[c >> 2], c & 3), z, 0,
                                                    0, 0);
        }
        // group gg's scales: f(G xs) (and f(M xs)); the second group of the pair completes the part
#pragma unroll
        for (int m = 0; m < 4; m++) {
          const int tk = 32 * th + 8 * m + 4 * kh;
          const float4 s4 = *(const float4 *)(xsT + gg * NT + tk);
          const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const int r = 4 * m + i;
            if (e == 0) {
              q0[r] = fmul((float)G[r], sv[i]);
              if (has_minimums<TY>()) qm0[r] = fmul(Mf[r], sv[i]);
            } else {
              float part = fmul(fadd(q0[r], fmul((float)G[r], sv[i])), F);
              if (has_minimums<TY>()) part = fsub(part, fmul(fadd(qm0[r], fmul(Mf[r], sv[i])), Fm));
              acc[kk][r] = fadd(acc[kk][r], part);
            }
          }
        }
      }
    }
  }
  // ((l0 + l1) + l2) + l3 (math.ts:7-9) through LDS (the tiles are free): the lane's row, its 16 tokens
  __syncthreads();
  float *lanes = (float *)(lds + Lay::X);
  const int row = r0 + mrow;
  if (NT == 128) {  // a wave holds the four lanes
    if (row < J.r1) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int t = 32 * th + 8 * (r >> 2) + 4 * kh + (r & 3);
        if (t0 + t < J.count)
          ((float *)(J.out + (t0 + t) * J.os))[row] =
              fadd(fadd(fadd(acc[0][r], acc[1 % TH][r]), acc[2 % TH][r]), acc[3 % TH][r]);
      }
    }
  } else if (NT == 64) {  // waves 0, 1 (lanes 0, 1) leave l0 + l1; waves 2, 3 add l2, then l3
    if (k0 == 0) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int t = 32 * th + 8 * (r >> 2) + 4 * kh + (r & 3);
        lanes[t * SBT_R + mrow] = fadd(acc[0][r], acc[TH - 1][r]);
      }
    }
    __syncthreads();
    if (k0 != 0 && row < J.r1) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int t = 32 * th + 8 * (r >> 2) + 4 * kh + (r & 3);
        if (t0 + t < J.count)
          ((float *)(J.out + (t0 + t) * J.os))[row] = fadd(fadd(lanes[t * SBT_R + mrow], acc[0][r]), acc[TH - 1][r]);
      }
    }
  } else {  // a lane a wave: waves 0..2 leave l0, l1, l2; wave 3 adds them in order, then l3
    if (k0 < 3) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int t = 8 * (r >> 2) + 4 * kh + (r & 3);
        lanes[(k0 * NT + t) * SBT_R + mrow] = acc[0][r];
      }
    }
    __syncthreads();
    if (k0 == 3 && row < J.r1) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int t = 8 * (r >> 2) + 4 * kh + (r & 3);
        if (t0 + t < J.count) {
          const float l0 = lanes[t * SBT_R + mrow], l1 = lanes[(NT + t) * SBT_R + mrow],
                      l2 = lanes[(2 * NT + t) * SBT_R + mrow];
          ((float *)(J.out + (t0 + t) * J.os))[row] = fadd(fadd(fadd(l0, l1), l2), acc[0][r]);
        }
      }
    }
  }
}

template <int TY, int NT>
hipError_t launch_tile_nt(const Job &j, int nrt, hipStream_t s) {
  static bool sized[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (!sized[dev]) {  // (more than 64 KB of LDS a block)
    const hipError_t e = hipFuncSetAttribute((const void *)gemm_sb<TY, NT>,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, SbTileLayout<TY, NT>::SIZE);
    if (e != hipSuccess) return e;
    sized[dev] = true;
  }
  const int ntt = (j.count + NT - 1) / NT;
  constexpr int lds = SbTileLayout<TY, NT>::SIZE;
  hipLaunchKernelGGL((gemm_sb<TY, NT>), dim3(nrt * ntt), dim3(256), lds, s, j);
  return hipGetLastError();
}

// the widest tile (128 for the tile_wide types, 64, 32 tokens) that still makes at least two blocks a compute unit:
// a wider one decodes each block of weights for more tokens, a narrower one has more blocks to hide a block's waits
template <int TY>
hipError_t launch_tile_type(const Job &j, hipStream_t s) {
  const int nrt = (j.r1 - j.r0 + SBT_R - 1) / SBT_R;
  const int64_t want = 2 * (int64_t)cu_count();
  const int nt = tile_wide<TY>() && (int64_t)nrt * ((j.count + 127) / 128) >= want ? 128
               : (int64_t)nrt * ((j.count + 63) / 64) >= want ? 64 : 32;
  if constexpr (tile_wide<TY>())
    if (nt == 128) return launch_tile_nt<TY, 128>(j, nrt, s);
  return nt == 64 ? launch_tile_nt<TY, 64>(j, nrt, s) : launch_tile_nt<TY, 32>(j, nrt, s);
}

// ---------------------------------------------------------------------------------------------------------------
// sb_row: a row as float32 (row.ts), a chunk of 16 weights a thread
// ---------------------------------------------------------------------------------------------------------------
template <int TY>
__global__ __launch_bounds__(256) void sb_row_kernel(float *out, const char *w, const uint8_t *tab, int32_t n) {
  constexpr int BYTES = sb_block_bytes(TY);
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // chunk: block i / 16, h = i % 16
  if (i >= (int64_t)(n >> 4)) return;
  const int b = (int)(i >> 4), h = (int)(i & 15);
  BlockBytes<BYTES> B;
  B.load(w + (int64_t)b * BYTES);
  uint32_t iq4[4] = {0u, 0u, 0u, 0u};
  if (TY == IQ4_XS) {
    const uint4 v = *(const uint4 *)(tab + T_IQ4);
    iq4[0] = v.x; iq4[1] = v.y; iq4[2] = v.z; iq4[3] = v.w;
  }
  Chunk c;
  // h is not a constant here: the chunk is decoded for each h and the one of this thread kept
#pragma unroll
  for (int hh = 0; hh < 16; hh++)
    if (hh == h) chunk<TY>(B, hh, tab + grid_at<TY>(), tab + T_SIGNS, iq4, c);
  const float d = block_d<TY>(B), fm = block_fm<TY>(B);
  // floatScale (row.ts:9-17): d (s + 1/2) / 4 (IQ2), d (s + 1/2) / 2 (IQ3_XXS), d S otherwise
  const float s = (float)(c.S >> 1);
  const float scale = (TY == IQ2_XXS || TY == IQ2_XS || TY == IQ2_S) ? fmul(fmul(d, fadd(0.5f, s)), 0.25f)
                    : TY == IQ3_XXS ? fmul(fmul(d, fadd(0.5f, s)), 0.5f) : fmul(d, (float)c.S);
  const float least = has_minimums<TY>() ? fmul(fm, (float)c.M) : 0.0f;
  float *to = out + 16 * i;
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const int32_t byte = (int32_t)(int8_t)((c.mag[j >> 2] >> (8 * (j & 3))) & 0xff);
    // W as an int8: the reference puts the signs on the magnitudes and takes IQ1's 1 off with byte subtractions that
    // wrap (row.ts:24, 32-37); only a grid byte of -128 (outside the converter's grids) shows it
    float v;
    if (is_iq1<TY>()) {  // the grid's -1, 0, 1 and an eighth more or less (row.ts:22-31)
      const uint32_t down = j < 8 ? c.down0 : c.down1;
      v = fadd((float)(int8_t)(byte - 1), down ? -0.125f : 0.125f);
    } else if (has_signs<TY>()) {
      const bool negative = ((c.neg[j >> 2] >> (8 * (j & 3))) & 0xff) != 0;
      v = (float)(int8_t)(negative ? -byte : byte);
    } else {
      v = (float)byte;
    }
    float x = fmul(scale, v);
    if (has_minimums<TY>()) x = fsub(x, least);
    to[j] = x;
  }
}

// ---------------------------------------------------------------------------------------------------------------
// sb_tables, sums_x, signed_dots
// ---------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void sb_tables_kernel(uint8_t *area, const uint8_t *codebooks) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < GRIDS) area[i] = (uint8_t)(codebooks[i] + (i >= T_IQ1S ? 1 : 0));
  if (i < 128 * 8) {  // the signs of 8 weights by a 7-bit index; the eighth makes the count of minus signs even
    const int idx = i >> 3, j = i & 7;
    const int held = idx | ((__builtin_popcount(idx) & 1) << 7);
    area[T_SIGNS + i] = ((held >> j) & 1) ? 255 : 0;
  }
  if (i < 16) {
    const int8_t v = (int8_t)codebooks[GRIDS + i];
    area[T_IQ4 + i] = (uint8_t)v;
    area[T_IQ4 + 16 + i] = (uint8_t)(int8_t)(v < 0 ? -v : v);
    area[T_IQ4 + 32 + i] = v < 0 ? 255 : 0;
    uint8_t *vec = area + T_VECTORS;
    vec[0 + i] = (uint8_t)(1u << (i & 7));
    vec[16 + i] = (uint8_t)(i >> 3);
    vec[32 + i] = 3;
    vec[48 + i] = 15;
    vec[80 + i] = 7;
    vec[96 + i] = 1;
  }
  if (i < 4) {
    ((int32_t *)(area + T_VECTORS + 64))[i] = 512 >> (3 * i);
    ((int32_t *)(area + T_VECTORS + 112))[i] = 4096 >> (4 * i);
  }
}

// a thread per 16 activations of a token: its two sums of 8 and its sum of 16 (int16)
__global__ __launch_bounds__(256) void sums_x_kernel(char *xs, const char *xq, int32_t n, int64_t total, int64_t frame) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int32_t per = n >> 4;
  const int64_t t = i / per;
  const int32_t u = (int32_t)(i - t * per);
  const int8_t *a = (const int8_t *)(xq + t * frame) + 16 * u;
  int32_t s0 = 0, s1 = 0;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    s0 += a[j];
    s1 += a[8 + j];
  }
  int16_t *s16 = (int16_t *)(xs + t * frame + 4 * (n >> 5)), *s8 = s16 + (n >> 4);
  s16[u] = (int16_t)(s0 + s1);
  s8[2 * u] = (int16_t)s0;
  s8[2 * u + 1] = (int16_t)s1;
}

__global__ void signed_dots_kernel(int32_t *out, const int8_t *a, const int8_t *b) {
  const int k = threadIdx.x;
  if (k < 4) {
    int32_t s = 0;
    for (int j = 0; j < 4; j++) s += (int32_t)a[4 * k + j] * (int32_t)b[4 * k + j];
    out[k] = s;
  }
}

}  // namespace

hipError_t launch_sb_tables(uint8_t *area, const uint8_t *codebooks, hipStream_t s) {
  hipLaunchKernelGGL(sb_tables_kernel, dim3((GRIDS + 255) / 256), dim3(256), 0, s, area, codebooks);
  return hipGetLastError();
}

hipError_t launch_sums_x(char *xs, const char *xq, int32_t n, int32_t count, int64_t frame, hipStream_t s) {
  const int64_t total = (int64_t)count * (n >> 4);
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL(sums_x_kernel, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, s, xs, xq, n, total, frame);
  return hipGetLastError();
}

hipError_t launch_signed_dots(int32_t *out, const int8_t *a, const int8_t *b, hipStream_t s) {
  hipLaunchKernelGGL(signed_dots_kernel, dim3(1), dim3(64), 0, s, out, a, b);
  return hipGetLastError();
}

hipError_t launch_sb_row(float *out, const char *w, const uint8_t *tab, int32_t n, int32_t type, hipStream_t s) {
  const int64_t chunks = n >> 4;
  if (chunks <= 0) return hipSuccess;
  const dim3 grid((uint32_t)((chunks + 255) / 256)), block(256);
  switch (type) {
  case Q2_K: hipLaunchKernelGGL(sb_row_kernel<Q2_K>, grid, block, 0, s, out, w, tab, n); break;
  case Q4_K: hipLaunchKernelGGL(sb_row_kernel<Q4_K>, grid, block, 0, s, out, w, tab, n); break;
  case IQ2_XXS: hipLaunchKernelGGL(sb_row_kernel<IQ2_XXS>, grid, block, 0, s, out, w, tab, n); break;
  case IQ2_XS: hipLaunchKernelGGL(sb_row_kernel<IQ2_XS>, grid, block, 0, s, out, w, tab, n); break;
  case IQ2_S: hipLaunchKernelGGL(sb_row_kernel<IQ2_S>, grid, block, 0, s, out, w, tab, n); break;
  case IQ3_XXS: hipLaunchKernelGGL(sb_row_kernel<IQ3_XXS>, grid, block, 0, s, out, w, tab, n); break;
  case IQ3_S: hipLaunchKernelGGL(sb_row_kernel<IQ3_S>, grid, block, 0, s, out, w, tab, n); break;
  case IQ1_S: hipLaunchKernelGGL(sb_row_kernel<IQ1_S>, grid, block, 0, s, out, w, tab, n); break;
  case IQ1_M: hipLaunchKernelGGL(sb_row_kernel<IQ1_M>, grid, block, 0, s, out, w, tab, n); break;
  case IQ4_XS: hipLaunchKernelGGL(sb_row_kernel<IQ4_XS>, grid, block, 0, s, out, w, tab, n); break;
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// a prompt (kSbTileMin tokens or more) of one job through the tile
hipError_t launch_sb_tile(const Job &j, hipStream_t s) {
  if (j.r1 <= j.r0 || j.count <= 0) return hipSuccess;
  switch (j.type) {
  case Q2_K: return launch_tile_type<Q2_K>(j, s);
  case Q4_K: return launch_tile_type<Q4_K>(j, s);
  case IQ2_XXS: return launch_tile_type<IQ2_XXS>(j, s);
  case IQ2_XS: return launch_tile_type<IQ2_XS>(j, s);
  case IQ2_S: return launch_tile_type<IQ2_S>(j, s);
  case IQ3_XXS: return launch_tile_type<IQ3_XXS>(j, s);
  case IQ3_S: return launch_tile_type<IQ3_S>(j, s);
  case IQ1_S: return launch_tile_type<IQ1_S>(j, s);
  case IQ1_M: return launch_tile_type<IQ1_M>(j, s);
  case IQ4_XS: return launch_tile_type<IQ4_XS>(j, s);
  default: return hipErrorInvalidValue;
  }
}

// jobs: one block type, one token count (1..4), one tables' area
hipError_t launch_sb(const Job *jobs, int32_t njobs, hipStream_t s) {
  if (njobs < 1 || njobs > kMaxJobs) return hipErrorInvalidValue;
  SbBatch b{};
  int longest = 0;
  for (int j = 0; j < njobs; j++) longest = (jobs[j].n >> 8) > longest ? (jobs[j].n >> 8) : longest;
  // (a prompt's slices of 2..4 tokens keep 16 lanes: their steps are long enough)
  const int L = jobs[0].count == 1 ? sb_lanes(longest) : 16, R = 64 / L;
  int units = 0;
  for (int j = 0; j < njobs; j++) {
    if (jobs[j].type != jobs[0].type || jobs[j].count != jobs[0].count || jobs[j].ws != jobs[0].ws)
      return hipErrorInvalidValue;
    b.job[j] = jobs[j];
    b.unit0[j] = units;
    units += (jobs[j].r1 - jobs[j].r0 + R - 1) / R;
  }
  b.unit0[njobs] = units;
  b.njobs = njobs;
  if (units == 0) return hipSuccess;
  const int T = jobs[0].count;
  // one token's activations, the same for every job: staged in LDS (sb_stage_bytes) when they fit (every type:
  // with the padded pitch, 20-51 % faster than reading them through the L1 for the types that gather from a grid)
  bool same = T == 1;
  for (int j = 1; j < njobs; j++)
    same = same && jobs[j].xq == jobs[0].xq && jobs[j].xs == jobs[0].xs && jobs[j].n == jobs[0].n;
  const size_t stage_bytes = sb_stage_bytes(jobs[0].type, jobs[0].n);
  const size_t lds = same && stage_bytes <= kSbStageMax ? stage_bytes : 0;
  switch (jobs[0].type) {
  case Q2_K: return launch_type<Q2_K>(b, T, L, lds, s);
  case Q4_K: return launch_type<Q4_K>(b, T, L, lds, s);
  case IQ2_XXS: return launch_type<IQ2_XXS>(b, T, L, lds, s);
  case IQ2_XS: return launch_type<IQ2_XS>(b, T, L, lds, s);
  case IQ2_S: return launch_type<IQ2_S>(b, T, L, lds, s);
  case IQ3_XXS: return launch_type<IQ3_XXS>(b, T, L, lds, s);
  case IQ3_S: return launch_type<IQ3_S>(b, T, L, lds, s);
  case IQ1_S: return launch_type<IQ1_S>(b, T, L, lds, s);
  case IQ1_M: return launch_type<IQ1_M>(b, T, L, lds, s);
  case IQ4_XS: return launch_type<IQ4_XS>(b, T, L, lds, s);
  default: return hipErrorInvalidValue;
  }
}

}  // namespace hq
