// gemv.hip — the token kernels (decode, 1..4 tokens a launch, the weights read once for all of them):
//   matmul_q8r / matmul_q6r   (kernels/relaxed/int8.ts:17-50, relaxed/six.ts:16-39; the tile's numbers for
//                              2..4 tokens, relaxed/int8.ts:52-166)
//   matmul_q8 / matmul_q6     (kernels/kernel/matmul.ts:77-104, 227-244)
//   matmul_t2r / matmul_t2    (kernels/relaxed/signs.ts:35-55, 117-119, kernel/matmul.ts:196-220; the same numbers)
//   matmul_b1r / matmul_b1    (relaxed/signs.ts:123-125, kernel/matmul.ts:222-224: the ternary kernels on binary
//                              weights, kernels/binary.ts; ternary's numbers for the same signs)
//
// Layout: a row is 16 lanes (relaxed: 16 or 32 by the launch's shape; ternary: 8, 16 or 32 by the row's length), a
// wave 4 rows (2 of 32 lanes); a block is 2 waves (8 rows, or 4 of 32 lanes) for the relaxed kinds, 4 waves for the
// others.  Lane l of a row of L lanes takes the groups L i + l (i = 0, 1, ...): a group's bytes (32 int8, 24 int6 or
// 32 ternary) are one lane's, so its integer sum is exact in that lane (v_dot4_i32_i8) and a row's lanes read
// 32 L (24 L) contiguous bytes a step.  One token of int8 (RelaxedChunk::PAIRED) instead reads each step as whole
// cache lines with non-temporal loads: a group's two 16-byte halves are in lanes 2 i and 2 i + 1, which add their
// integers by a DPP swap.
//
// The float32 order is the reference's, so every output is its number to the bit:
//   relaxed int8 / int6: lane k (k = 0..3) of the reference's accumulator adds the groups 4 j + k in order.  Those
//     are lanes k, k + 4, k + 8, k + 12 of a step here (of a 32-lane row's step, then k + 16, ..., k + 28): lane k
//     adds them in that order with DPP moves (no LDS; the upper 16 lanes brought down by v_permlane16_swap), then
//     lane 0 adds the four lanes ((l0 + l1) + l2) + l3 and the groups past the last four one at a time (one token
//     of int8: chain k in lane 2 k, the four in lanes 0, 2, 4, 6).
//   plain int8 / int6 and ternary: the reference's lane k adds part k of EVERY group in order (matmul_q8: the
//     products 2k, 2k+1, 2k+8, 2k+9 of each half; ternary: the k-th 32 of each 128).  A step's 16 groups x 4 parts
//     are written to LDS and lane k of the row adds its part of the 16 groups in order.
// Rows past r1 in a block compute on a clamped row and store nothing (DPP needs the whole row of lanes live).
#include <algorithm>
#include <numeric>

#include "common.hpp"
#include "launch.hpp"
#include "fold.hpp"

#define HQ_HOST_DEV __host__ __device__

namespace hq {

namespace {

struct GemvBatch {
  Job job[kMaxJobs];
  int32_t block0[kMaxJobs + 1];  // the first block of each job
  int32_t njobs;
};

// how a batch is launched: by (a job a grid row) with pieces of `rows` rows; lead_r1 the end of the rows of the job
// whose pieces come first
struct JobPieces {
  bool by;
  int32_t rows, lead_r1, lead_pieces;  // lead_pieces: how many of the pieces are that job's
};

// where a kernel's activations come from: the caller's xq / xs in global memory (read through the L1), or a copy
// of them the block makes in LDS
enum Src { GLOBAL = 0, STAGED = 1 };

// the LDS a block needs for T tokens of n activations (bytes, then float32 scales)
HQ_HOST_DEV constexpr int64_t act_lds_bytes(int T, int n) { return (int64_t)T * (n + 4 * (n / 32)); }

// STAGED: fill the block's LDS with the activations of T tokens: bytes of token t at lq + t n, scales at
// ls + t (n / 32).  Every thread takes groups of 32 in turn; the block synchronizes after.
template <int T>
HQ_DEV void fill_acts(const Job &J, char *lq, float *ls) {
  const int n = J.n, ng = n >> 5;
  for (int idx = threadIdx.x; idx < T * ng; idx += blockDim.x) {
    const int t = idx / ng, g = idx - t * ng;
    const char *src = J.xq + t * J.frame + g * GS;
    uint4 *dst = (uint4 *)(lq + t * n + g * GS);
    dst[0] = *(const uint4 *)src;
    dst[1] = *(const uint4 *)(src + 16);
    ls[t * ng + g] = ((const float *)(J.xs + t * J.sframe))[g];
  }
  __syncthreads();
}

constexpr int kRowsPerBlock = 16;
// the relaxed kinds' blocks: 128 threads, 8 rows of 16 lanes or 4 of 32 (fewer rows a block: more blocks, a finer
// balance of the last ones over the CUs; 8 rows of 16 measured faster than 16 rows at the 8B decode); 2..4 tokens
// staged in LDS take 512 (one staged copy for four times the rows: the 8B decode's products at M = 4 2.02 ms with
// 256 threads, 1.96 with 512; 1024 threads, whose waves get 128 registers, 2.26)
constexpr int kRelaxedThreads = 128;
HQ_HOST_DEV constexpr int relaxed_threads(int T, bool staged) { return T > 1 && staged ? 512 : kRelaxedThreads; }
// One token's launches whose blocks of kRelaxedThreads come short of whole rounds of the compute units take blocks of
// one wave where those fill them better (relaxed_block_threads)
constexpr int kOneTokenSmall = 64;
// Lanes a relaxed row: 32 lanes give a launch twice the waves, each lane half the steps.  Measured phase by phase
// streaming from HBM (configs 1-4's decode shapes, int8 and int6, 16 against 32 lanes): one int8 token, 32 lanes are
// faster where a row is 4096 or 8192 bytes (8B q/k/v 7.7 -> 7.1 us, o 6.2 -> 5.8, gate+up 25.3 -> 23.5, lm-head 97 ->
// 94; 1B down 6.8 -> 6.3) and slower at 1024, 2048 and 5120 (LFM2's lm-head 18.1 -> 25.7), and at 14336 in chunks of
// four steps (8B down 14.0 -> 14.6; in chunks of two, below, faster); int6 shows no consistent gain (16 lanes); 2..4
// tokens gain on rows past 8192 (four tokens' 8B down 19.8 -> 18.8 us, int6 30.4 -> 20.7) and lose below (gate+up
// 29.6 -> 31.9).
constexpr int kRelaxedLongRow = 8192;
// One token of int8 past 8192 takes 32 lanes where a row is an even number of 32-lane steps, not a multiple of four
// (10240, 14336, ...), in chunks of 2 steps: none past the row's end (8B down 12.73 -> 12.55 us; with chunks of 4,
// half a chunk of loads wasted at each row's end, 13.45).
HQ_HOST_DEV constexpr bool relaxed_pairs_of_steps(Kind kind, int T, int n) {
  return T == 1 && kind == Q8R && n > kRelaxedLongRow && (n / 1024) % 4 == 2 && n % 1024 == 0;
}
HQ_HOST_DEV constexpr int relaxed_lanes(Kind kind, int T, int n) {
  if (T > 1) return n > kRelaxedLongRow ? 32 : 16;
  return kind == Q8R && ((n % 4096 == 0 && n <= kRelaxedLongRow) || relaxed_pairs_of_steps(kind, T, n)) ? 32 : 16;
}

// the job of block `blk`: block0's entries past the batch's jobs are INT32_MAX, so that every entry is compared
// without a loop, all read in one round of scalar loads
HQ_DEV int job_of(const GemvBatch &b, int blk) {
  int j = 0;
#pragma unroll
  for (int i = 1; i < kMaxJobs; i++) j += blk >= b.block0[i] ? 1 : 0;
  return j;
}
// a block's job and its place among the job's blocks.  BY (the batch's jobs cut into pieces of gridDim.x blocks, one
// a grid row): the job is blockIdx.y, so its fields are read in the kernel's first round of scalar loads; else it is
// found through block0 and its fields read in a second round
template <bool BY>
HQ_DEV void block_job(const GemvBatch &b, int &jb, int &blk) {
  if (BY) {
    jb = (int)blockIdx.y;
    blk = (int)blockIdx.x;
  } else {
    jb = job_of(b, (int)blockIdx.x);
    blk = (int)blockIdx.x - b.block0[jb];
  }
}

HQ_DEV uint4 ld16(const char *p) { return *(const uint4 *)p; }
HQ_DEV uint2 ld8(const char *p) { return *(const uint2 *)p; }

HQ_DEV uint4 ldw16(const char *p) { return *(const uint4 *)p; }
// a weight load that is not kept in the caches (each weight byte is read once); for whole cache lines only: a line
// read in halves by two such loads is fetched twice
HQ_DEV uint4 ldw16_nt(const char *p) {
  typedef uint32_t u4v __attribute__((ext_vector_type(4)));
  const u4v q = __builtin_nontemporal_load((const u4v *)p);
  return make_uint4(q.x, q.y, q.z, q.w);
}
// streamed (non-temporal) unless CACHED: a launch's weights small enough to stay in the caches from one step to the
// next are read through them (relaxed_cached)
template <bool CACHED> HQ_DEV uint4 ldw16_as(const char *p) { return CACHED ? ldw16(p) : ldw16_nt(p); }
template <bool CACHED, typename V> HQ_DEV V ld_as(const V *p) { return CACHED ? *p : __builtin_nontemporal_load(p); }

// the 32 weight bytes of group g of a row, as eight dwords of int8 (int6 groups widened, kernels/six.ts)
template <int PACK>
HQ_DEV void load_group(const char *wrow, int g, uint32_t w[8]) {
  if (PACK == 8) {
    const uint4 a = ldw16(wrow + g * 32), b = ldw16(wrow + g * 32 + 16);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  } else {
    const char *p = wrow + g * 24;
    const uint2 a = ld8(p), b = ld8(p + 8), c = ld8(p + 16);
    const uint32_t d[6] = {a.x, a.y, b.x, b.y, c.x, c.y};
    six_widen(d, w);
  }
}

HQ_DEV void load_acts(const char *xq, int g, uint32_t x[8]) {
  const uint4 a = ld16(xq + g * 32), b = ld16(xq + g * 32 + 16);
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
  x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

// ---------------------------------------------------------------------------------------------------------------
// relaxed int8 / int6 (matmul_q8r, matmul_q6r; T tokens of the tile)
// ---------------------------------------------------------------------------------------------------------------
// Memory-level parallelism: a lane's steps are taken U at a time (a chunk: its weights and scales, and from global
// memory its activations, loaded into registers together), and the next chunk's loads are issued before the current
// chunk is computed, so a wave keeps two chunks of loads in flight.  The compiler cannot unroll the step loop itself
// (the DPP moves are convergent), so the two chunk buffers alternate by hand.  With 2..4 tokens staged in LDS (LATE)
// a chunk holds only the weights of 2 steps and the fold reads each step's activations from LDS as it goes, so
// the registers that 4 tokens' activations would take hold more weights in flight (one step a chunk with the
// activations in it: 8 % slower at M = 4; 4 or 8 steps a chunk: slower still).
template <int T, int SRC>
struct ActSource {
  const char *xq[T];
  const char *xs[T];
  const char *lq;  // LDS: token t's bytes at lq + t n, scales at ls + t ng
  const float *ls;
  int n, ng;
  HQ_DEV void get(int t, int g, uint32_t x[8]) const {
    const char *p = SRC == GLOBAL ? xq[t] + g * 32 : lq + t * n + g * 32;
    const uint4 a = *(const uint4 *)p, b = *(const uint4 *)(p + 16);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  }
  HQ_DEV float scale(int t, int g) const { return SRC == GLOBAL ? ((const float *)xs[t])[g] : ls[t * ng + g]; }
};

template <int PACK, int T, bool WC, int SRC, int RL, int U1, bool CACHED>
struct RelaxedChunk {
  static constexpr bool LATE = T > 1 && SRC == STAGED;
  static constexpr int U = T == 1 ? U1 : (LATE || T == 2 ? 2 : 1);  // U1: 4, or 2 (relaxed_pairs_of_steps)
  static constexpr int UX = LATE ? 1 : U;  // steps of activations a chunk holds (none read when LATE)
  // One token of int8 (PAIRED): a step's weights are read as whole cache lines by non-temporal loads (ordinary
  // loads when CACHED).  Lane j of a row takes the 16 bytes at 16 j of the step's first half (group j / 2's half
  // j % 2) and at RL 16 + 16 j of its second (group RL / 2 + j / 2's), so that each load instruction reads a row's
  // RL 16 contiguous bytes; a group's integer is its two halves' (lanes 2 i and 2 i + 1) added by a DPP swap.
  // Half-lines read by two loads would be fetched twice past the caches.
  static constexpr bool PAIRED = T == 1 && SRC == GLOBAL && PACK == 8;
  uint32_t w[U][8];   // PAIRED: w[u][0..3] the first half's 16 bytes, [4..7] the second's
  uint32_t x[UX][T][8];
  float ws[U], xs[UX][T];  // PAIRED: the scales (and wc the correction) of group 2 i's lane's own group: an even
  int32_t wc[U];           // lane's of the first half, an odd lane's of the second (the pair swaps them by DPP)

  // PAIRED: steps it0 .. it0 + U - 1, weights, activations and scales of the lane's two half-groups (a group past
  // the row's fours: group 0's bytes, its term dropped)
  // (wb, sb, cb: the wave's first row's weights, scales and corrections, the same in every lane; rb: the lane's row's
  // byte offset from wb, gb its offset from sb and cb: every address a scalar base plus a 32-bit offset)
  HQ_DEV void load_paired(const char *wb, const float *sb, const int32_t *cb, uint32_t rb, uint32_t gb,
                          const ActSource<T, SRC> &A, int it0, int lane, int ng4) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int g0 = (it0 + u) * RL + (lane >> 1), g1 = g0 + RL / 2;
      const uint32_t h = 16u * (uint32_t)(lane & 1);
      const uint32_t c0 = (uint32_t)(g0 < ng4 ? g0 : 0), c1 = (uint32_t)(g1 < ng4 ? g1 : 0);
      const uint4 a = ldw16_as<CACHED>(wb + (rb + c0 * 32u + h)), b = ldw16_as<CACHED>(wb + (rb + c1 * 32u + h));
      w[u][0] = a.x; w[u][1] = a.y; w[u][2] = a.z; w[u][3] = a.w;
      w[u][4] = b.x; w[u][5] = b.y; w[u][6] = b.z; w[u][7] = b.w;
      const uint4 xa = ld16(A.xq[0] + (c0 * 32u + h)), xb = ld16(A.xq[0] + (c1 * 32u + h));
      x[u][0][0] = xa.x; x[u][0][1] = xa.y; x[u][0][2] = xa.z; x[u][0][3] = xa.w;
      x[u][0][4] = xb.x; x[u][0][5] = xb.y; x[u][0][6] = xb.z; x[u][0][7] = xb.w;
      // the row's scales and corrections, like its weights, streamed once (a row's 32 lanes read one whole line;
      // through the caches when CACHED)
      const uint32_t own = (lane & 1) ? c1 : c0;
      ws[u] = ld_as<CACHED>((const float *)((const char *)sb + (gb + own * 4u)));
      xs[u][0] = *(const float *)(A.xs[0] + own * 4u);
      if (WC) wc[u] = ld_as<CACHED>((const int32_t *)((const char *)cb + (gb + own * 4u)));
    }
  }
  // PAIRED: the chunk's terms folded into the chains: chain k of the reference (groups 4 j + k) lives in lane 2 k, and
  // a step's groups k, k + 4, .. of its first half are lanes 2 k, 2 k + 8 (then 2 k + 16, 2 k + 24 of a 32-lane row,
  // brought down by v_permlane16_swap), then the same of its second half (relaxed/int8.ts:26-39)
  HQ_DEV void fold_paired(float acc[T], int it0, int lane, int ng4) const {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int g0 = (it0 + u) * RL + (lane >> 1), g1 = g0 + RL / 2;
      // an even lane's scale product of its first group, and (swapped in from the odd lane) of its second
      const float sown = fmul(ws[u], xs[u][0]);
      const float sc[2] = {sown, __int_as_float(swap_pair(__float_as_int(sown)))};
      const int32_t cw[2] = {WC ? wc[u] : 0, WC ? swap_pair(wc[u]) : 0};
      float q[2];
#pragma unroll
      for (int s2 = 0; s2 < 2; s2++) {
        int32_t d = 0;
        if (!WC) {
          int32_t wsum = 0;
#pragma unroll
          for (int i = 0; i < 4; i++) wsum = sdot4((int32_t)w[u][4 * s2 + i], 0x01010101, wsum);
          d = -64 * wsum;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) d = sdot4((int32_t)w[u][4 * s2 + i], (int32_t)x[u][0][4 * s2 + i], d);
        d += swap_pair(d);  // the group's two halves (wrapping int32 adds, as the reference's i32x4.add)
        if (WC) d += cw[s2];
        const float p = fmul((float)d, sc[s2]);  // (an odd lane's terms are never read)
        q[s2] = (s2 ? g1 : g0) < ng4 ? p : 0.0f;  // +0 leaves a lane as it is: a lane is never -0
      }
      float a = acc[0];
#pragma unroll
      for (int s2 = 0; s2 < 2; s2++) {
        a = fadd(a, q[s2]);
        a = fadd(a, from_lane_plus<8>(q[s2]));
        if (RL == 32) {
          const float qh = upper_row(q[s2]);
          a = fadd(a, qh);
          a = fadd(a, from_lane_plus<8>(qh));
        }
      }
      acc[0] = a;
    }
  }

  // steps it0 .. it0 + U - 1 of this lane (its group RL it + lane of each; a lane past the row's fours reads group
  // 0 again, whose term it drops): the weights, their scales and corrections
  HQ_DEV void load_w(const char *wrow, const float *srow, const int32_t *crow, int it0, int lane, int ng4) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int g = (it0 + u) * RL + lane;
      const int gl = g < ng4 ? g : 0;
      load_group<PACK>(wrow, gl, w[u]);
      ws[u] = srow[gl];
      if (WC) wc[u] = crow[gl];
    }
  }
  // ... and the activations of the same groups (from global memory or the block's LDS)
  HQ_DEV void load_x(const ActSource<T, SRC> &A, int it0, int lane, int ng4) {
    if (LATE) return;
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int g = (it0 + u) * RL + lane;
      const int gl = g < ng4 ? g : 0;
#pragma unroll
      for (int t = 0; t < T; t++) {
        A.get(t, gl, x[u][t]);
        xs[u][t] = A.scale(t, gl);
      }
    }
  }
  // both, a group at a time
  HQ_DEV void load(const char *wrow, const float *srow, const int32_t *crow, const ActSource<T, SRC> &A, int it0,
                   int lane, int ng4) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int g = (it0 + u) * RL + lane;
      const int gl = g < ng4 ? g : 0;
      load_group<PACK>(wrow, gl, w[u]);
      ws[u] = srow[gl];
      if (WC) wc[u] = crow[gl];
      if (!LATE) {
#pragma unroll
        for (int t = 0; t < T; t++) {
          A.get(t, gl, x[u][t]);
          xs[u][t] = A.scale(t, gl);
        }
      }
    }
  }

  // the chunk's terms, folded into the lanes' sums: lane k takes groups RL it + k, + 4, + 8, ... in order
  // (relaxed/int8.ts:26-39); a 32-lane row's second 16 groups come to lanes 0..15 by v_permlane16_swap
  HQ_DEV void fold(float acc[T], int it0, int lane, int ng4, const ActSource<T, SRC> &A) const {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int g = (it0 + u) * RL + lane;
      const bool valid = g < ng4;
      uint32_t xl[T][8];  // LATE: the step's activations, read here
      float xsl[T];
      if (LATE) {
#pragma unroll
        for (int t = 0; t < T; t++) {
          A.get(t, valid ? g : 0, xl[t]);
          xsl[t] = A.scale(t, valid ? g : 0);
        }
      }
      int32_t wsum = 0;
      if (!WC) {
#pragma unroll
        for (int i = 0; i < 8; i++) wsum = sdot4((int32_t)w[u][i], 0x01010101, wsum);
      }
#pragma unroll
      for (int t = 0; t < T; t++) {
        int32_t d = WC ? wc[u] : -64 * wsum;
#pragma unroll
        for (int i = 0; i < 8; i++) d = sdot4((int32_t)w[u][i], (int32_t)(LATE ? xl[t][i] : x[LATE ? 0 : u][t][i]), d);
        const float p = fmul((float)d, fmul(ws[u], LATE ? xsl[t] : xs[LATE ? 0 : u][t]));
        const float q = valid ? p : 0.0f;  // +0 leaves a lane as it is: a lane is never -0
        float a = fadd(acc[t], q);
        a = fadd(a, from_lane_plus<4>(q));
        a = fadd(a, from_lane_plus<8>(q));
        a = fadd(a, from_lane_plus<12>(q));
        if (RL == 32) {
          const float qh = upper_row(q);
          a = fadd(a, qh);
          a = fadd(a, from_lane_plus<4>(qh));
          a = fadd(a, from_lane_plus<8>(qh));
          a = fadd(a, from_lane_plus<12>(qh));
        }
        acc[t] = a;
      }
    }
  }
};

// the relaxed_threads / RL rows of tile `blk` of job `jb` (its row range cut into tiles in order).  STAGED: first
// make the block's LDS copy of the activations, while the first weights are in flight
template <int PACK, int T, bool WC, int SRC, int RL, int U1, int NT, bool CACHED>
HQ_DEV void relaxed_tile(const Job &J, int blk, char *lds) {
  const int lane = threadIdx.x & (RL - 1);
  constexpr int rows = NT / RL;
  const int row_u = J.r0 + blk * rows + (int)(threadIdx.x / RL);
  const bool live = row_u < J.r1;
  const int row = live ? row_u : J.r1 - 1;
  const int ng = J.n >> 5, ng4 = ng & ~3;
  constexpr int GB = PACK == 8 ? 32 : 24;
  const char *wrow = J.wq + (int64_t)row * ng * GB;
  const float *srow = (const float *)J.ws + (int64_t)row * ng;
  const int32_t *crow = WC ? (const int32_t *)J.wc + (int64_t)row * ng : nullptr;
  // the wave's first row (lane 0's: the rows of a wave ascend, and a clamped row is the job's last) as scalar bases
  const int row0 = __builtin_amdgcn_readfirstlane(row);
  const char *wb = J.wq + (int64_t)row0 * ng * GB;
  const float *sb = (const float *)J.ws + (int64_t)row0 * ng;
  const int32_t *cb = WC ? (const int32_t *)J.wc + (int64_t)row0 * ng : nullptr;
  const uint32_t rb = (uint32_t)(row - row0) * (uint32_t)(ng * GB), gb = (uint32_t)(row - row0) * (uint32_t)(ng * 4);
  ActSource<T, SRC> A;
#pragma unroll
  for (int t = 0; t < T; t++) {
    A.xq[t] = J.xq + t * J.frame;
    A.xs[t] = J.xs + t * J.sframe;
  }
  A.lq = lds;
  A.ls = (const float *)(lds + T * J.n);
  A.n = J.n;
  A.ng = ng;

  float acc[T];
#pragma unroll
  for (int t = 0; t < T; t++) acc[t] = 0.0f;
  using Chunk = RelaxedChunk<PACK, T, WC, SRC, RL, U1, CACHED>;
  constexpr int U = Chunk::U;
  const int steps = (ng4 + RL - 1) / RL;
  Chunk a, b;
  if (SRC == STAGED) {
    if (steps > 0) a.load_w(wrow, srow, crow, 0, lane, ng4);  // the first weights in flight during the staging
    fill_acts<T>(J, lds, (float *)(lds + T * J.n));
    if (steps > 0) a.load_x(A, 0, lane, ng4);
  } else if (Chunk::PAIRED) {
    if (steps > 0) a.load_paired(wb, sb, cb, rb, gb, A, 0, lane, ng4);
  } else if (steps > 0) {
    a.load(wrow, srow, crow, A, 0, lane, ng4);
  }
  if (Chunk::PAIRED) {
    for (int it = 0; it < steps; it += 2 * U) {
      if (it + U < steps) b.load_paired(wb, sb, cb, rb, gb, A, it + U, lane, ng4);
      a.fold_paired(acc, it, lane, ng4);
      if (it + U < steps) {
        if (it + 2 * U < steps) a.load_paired(wb, sb, cb, rb, gb, A, it + 2 * U, lane, ng4);
        b.fold_paired(acc, it + U, lane, ng4);
      }
    }
  } else if (T == 1) {
    for (int it = 0; it < steps; it += 2 * U) {
      if (it + U < steps) b.load(wrow, srow, crow, A, it + U, lane, ng4);
      a.fold(acc, it, lane, ng4, A);
      if (it + U < steps) {
        if (it + 2 * U < steps) a.load(wrow, srow, crow, A, it + 2 * U, lane, ng4);
        b.fold(acc, it + U, lane, ng4, A);
      }
    }
  } else {
    // each fold in the block of the loads issued before it, so that its wait counts only the chunk it folds: where
    // paths with and without those loads met, the fold also waited for the next chunk's first loads (one chunk in
    // flight instead of two; a chunk of M = 1 is 24 loads, so only one of them, and it keeps the loop above)
    for (int it = 0; steps > 0; it += 2 * U) {
      if (it + U >= steps) {
        a.fold(acc, it, lane, ng4, A);
        break;
      }
      b.load(wrow, srow, crow, A, it + U, lane, ng4);
      a.fold(acc, it, lane, ng4, A);
      if (it + 2 * U >= steps) {
        b.fold(acc, it + U, lane, ng4, A);
        break;
      }
      a.load(wrow, srow, crow, A, it + 2 * U, lane, ng4);
      b.fold(acc, it + U, lane, ng4, A);
    }
  }
  // lane 0: ((l0 + l1) + l2) + l3 (math.ts:7-9), then the groups past the fours one at a time (int8.ts:40-47); the
  // paired layout's chains are in lanes 0, 2, 4, 6
  float sum[T];
#pragma unroll
  for (int t = 0; t < T; t++) {
    if (Chunk::PAIRED)
      sum[t] = fadd(fadd(fadd(acc[t], from_lane_plus<2>(acc[t])), from_lane_plus<4>(acc[t])), from_lane_plus<6>(acc[t]));
    else
      sum[t] = fadd(fadd(fadd(acc[t], from_lane_plus<1>(acc[t])), from_lane_plus<2>(acc[t])), from_lane_plus<3>(acc[t]));
  }
  const int tail = ng - ng4;
  if (tail > 0) {
    const int g = ng4 + (lane < tail ? lane : 0);
    uint32_t w[8];
    load_group<PACK>(wrow, g, w);
    int32_t wsum = 0;
    if (!WC) {
#pragma unroll
      for (int i = 0; i < 8; i++) wsum = sdot4((int32_t)w[i], 0x01010101, wsum);
    }
    const float ws = srow[g];
#pragma unroll
    for (int t = 0; t < T; t++) {
      uint32_t x[8];
      A.get(t, g, x);
      int32_t d = WC ? crow[g] : -64 * wsum;
#pragma unroll
      for (int i = 0; i < 8; i++) d = sdot4((int32_t)w[i], (int32_t)x[i], d);
      const float p = fmul((float)d, fmul(ws, A.scale(t, g)));
      sum[t] = fadd(sum[t], p);
      if (tail > 1) sum[t] = fadd(sum[t], from_lane_plus<1>(p));
      if (tail > 2) sum[t] = fadd(sum[t], from_lane_plus<2>(p));
    }
  }
  if (live && lane == 0) {
#pragma unroll
    for (int t = 0; t < T; t++) ((float *)(J.out + t * J.os))[row] = sum[t];
  }
}

// a tile a block
// PRE (a job a grid row): the batch's first job is also the first arguments, which the command processor puts in the
// waves' scalar registers before they start (gemv.hip is built with kernel-argument preloading: the 13 dwords up to
// frame fit the 14 user registers left), so the blocks of its pieces (rows r0 + pr y .. of grid row y) make no scalar
// load before their first weight and activation loads (out, os and wc, read late, follow as ordinary arguments); the
// other jobs' pieces read theirs.  PRE 2: every piece is the first job's (no other path in the kernel: measured
// 0.05 us a launch shorter than PRE 1).  The activations and their scales are `frame` bytes a token apart (the tile
// kinds' one stride).
template <int PACK, int T, bool WC, int SRC, int RL, bool BY, int PRE, int U1, int NT, bool CACHED>
__global__ __launch_bounds__(NT) void gemv_relaxed(
    const char *xq, const char *xs, const char *wq, const char *ws, int32_t n, int32_t r0, int32_t r1, int32_t pr,
    int32_t frame, char *out, int64_t os, const char *wc, GemvBatch batch) {
  extern __shared__ __align__(16) char lds[];
  if (PRE) {
    const int a = r0 + (int)blockIdx.y * pr;
    if (PRE == 2 || a < r1) {
      const Job J{out, xq, xs, wq, ws, wc, n, a, min(a + pr, r1), T, os, frame, frame, 0};
      relaxed_tile<PACK, T, WC, SRC, RL, U1, NT, CACHED>(J, (int)blockIdx.x, lds);
      return;
    }
  }
  int jb, blk;
  block_job<BY>(batch, jb, blk);
  relaxed_tile<PACK, T, WC, SRC, RL, U1, NT, CACHED>(batch.job[jb], blk, lds);
}

// ---------------------------------------------------------------------------------------------------------------
// the LDS fold of the kinds whose four lanes take part of every group
// ---------------------------------------------------------------------------------------------------------------
// per wave: 4 rows x T tokens x 4 parts x 16 groups, twice (a step's and the next one's)
template <int T>
struct Fold {
  float v[2][4][T][4][16];
};

// after the wave wrote its step's parts: lane k (k < 4) of each row adds part k of the 16 groups in order
template <int T>
HQ_DEV void fold_step(const Fold<T> &f, int buf, int slot, int lane, float acc[T]) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int k = lane & 3;
#pragma unroll
  for (int t = 0; t < T; t++) {
    const float4 *src = (const float4 *)f.v[buf][slot][t][k];
    float a = acc[t];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const float4 v = src[q];
      a = fadd(fadd(fadd(fadd(a, v.x), v.y), v.z), v.w);
    }
    acc[t] = a;
  }
}

// ---------------------------------------------------------------------------------------------------------------
// plain int8 / int6 (matmul_q8, matmul_q6)
// ---------------------------------------------------------------------------------------------------------------
// dot32's lanes (kernel/matmul.ts:60-72): part k of a group is the products at 2k, 2k+1, 2k+8, 2k+9 of each half.
// In dwords: part 0 is bytes 0-1 of dwords 0 and 2, part 1 bytes 2-3 of them, part 2 bytes 0-1 of dwords 1 and 3,
// part 3 bytes 2-3 of those (and the same of dwords 4..7).  v_perm_b32 gathers a part's four bytes of each half.
HQ_DEV void parts_of(const uint32_t v[8], uint32_t out[8]) {
#pragma unroll
  for (int h = 0; h < 2; h++) {
    out[0 + h] = perm(v[4 * h + 2], v[4 * h + 0], 0x05040100u);
    out[2 + h] = perm(v[4 * h + 2], v[4 * h + 0], 0x07060302u);
    out[4 + h] = perm(v[4 * h + 3], v[4 * h + 1], 0x05040100u);
    out[6 + h] = perm(v[4 * h + 3], v[4 * h + 1], 0x07060302u);
  }
}

template <int PACK, int T>
__global__ __launch_bounds__(256) void gemv_plain(GemvBatch batch) {
  __shared__ Fold<T> fold[4];
  const int jb = job_of(batch, blockIdx.x);
  const Job &J = batch.job[jb];
  const int lane = threadIdx.x & 15;
  const int wave = threadIdx.x >> 6, slot = (threadIdx.x >> 4) & 3;
  const int row_u = J.r0 + (blockIdx.x - batch.block0[jb]) * kRowsPerBlock + (threadIdx.x >> 4);
  const bool live = row_u < J.r1;
  const int row = live ? row_u : J.r1 - 1;
  const int ng = J.n >> 5;
  constexpr int GB = PACK == 8 ? 32 : 24;
  const char *wrow = J.wq + (int64_t)row * ng * GB;
  const float *srow = (const float *)J.ws + (int64_t)row * ng;
  Fold<T> &f = fold[wave];

  float acc[T];
#pragma unroll
  for (int t = 0; t < T; t++) acc[t] = 0.0f;
  const int steps = (ng + 15) >> 4;
  // a step's loads (group 16 it + lane of the row, and of every token's activations; past the row's groups, group 0
  // again), issued a step ahead of its use on every path, so that using a step waits for its own loads alone
  struct Step {
    uint32_t w[8], x[T][8];
    float ws, xs[T];
  };
  const auto load = [&](Step &p, int it) {
    const int g = it * 16 + lane, gl = g < ng ? g : 0;
    load_group<PACK>(wrow, gl, p.w);
    p.ws = srow[gl];
#pragma unroll
    for (int t = 0; t < T; t++) {
      load_acts(J.xq + t * J.frame, gl, p.x[t]);
      p.xs[t] = ((const float *)(J.xs + t * J.sframe))[gl];
    }
  };
  const auto step = [&](const Step &p, int it) {
    const bool valid = it * 16 + lane < ng;
    uint32_t wp[8];
    parts_of(p.w, wp);
    const int buf = it & 1;
#pragma unroll
    for (int t = 0; t < T; t++) {
      uint32_t xp[8];
      parts_of(p.x[t], xp);
      const float s = fmul(p.ws, p.xs[t]);
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int32_t d = sdot4((int32_t)wp[2 * k + 1], (int32_t)xp[2 * k + 1], sdot4((int32_t)wp[2 * k], (int32_t)xp[2 * k], 0));
        f.v[buf][slot][t][k][lane] = valid ? fmul((float)d, s) : 0.0f;
      }
    }
    fold_step<T>(f, buf, slot, lane, acc);
  };
  Step a, b;
  if (steps > 0) load(a, 0);
  for (int it = 0; it < steps; it += 2) {
    load(b, it + 1);
    step(a, it);
    if (it + 1 >= steps) break;  // uniform
    load(a, it + 2);
    step(b, it + 1);
  }
  // lanes 0..3 hold the four parts' sums: ((l0 + l1) + l2) + l3 in lane 0
  float sum[T];
#pragma unroll
  for (int t = 0; t < T; t++)
    sum[t] = fadd(fadd(fadd(acc[t], from_lane_plus<1>(acc[t])), from_lane_plus<2>(acc[t])), from_lane_plus<3>(acc[t]));
  if (live && lane == 0) {
#pragma unroll
    for (int t = 0; t < T; t++) ((float *)(J.out + t * J.os))[row] = sum[t];
  }
}

// ---------------------------------------------------------------------------------------------------------------
// ternary (matmul_t2r == matmul_t2) and binary (matmul_b1r == matmul_b1)
// ---------------------------------------------------------------------------------------------------------------
// A group of 128 weights is 32 bytes: block h (bytes 16h..16h+15) holds the codes of weights 64h + 4c + p in byte c,
// bits 2p.  The activations are interleave()'s: byte 16p + c of block (2g + h) is activation 4c + p of it.  Part k
// (the reference's lane k: activations 32k..32k+31 of the group) is block h = k / 2, c in 8 (k % 2) .. + 7: weight
// dwords 4h + 2(k%2) + {0,1} and, for every plane p, activation dwords 4p + 2(k%2) + {0,1} of the block.  Its
// integer is sum(code * a) + (minus the sum of its 32 activations) = sum((code - 1) a) exactly (ternary.ts:6-12).
// Binary (BIN, kernels/binary.ts): a group is 16 bytes, weight 64h + 4c + p at bit 4h + p of byte c, its code twice
// the bit (0 or 2: the weight + 1 again), so part k takes dwords 2(k%2) + {0,1} for both blocks and plane p of block
// h is ((dword >> (4h + p)) & 0x01010101) << 1 (binary.ts:19-22); everything after the codes is ternary's.
//
// A lane reads 32 bytes of codes a group but 128 bytes of activations (and 32 of their scales and sums): the block
// copies the activations of its T tokens into LDS once (STAGE), so that only the codes stream from memory, U steps
// at a time with the next U steps' loads in flight.  In LDS a group's 128 bytes take 144 (16 bytes of padding), so
// that the 16 lanes of a row, which read the same 16 bytes of 16 consecutive groups, hit 16 different bank quads.
constexpr int kTernarySteps = 1;  // steps a chunk (two chunks of loads in flight)
constexpr int kTernaryPitch = 144;  // LDS bytes a group of 128 activations

HQ_HOST_DEV constexpr int ternary_token_bytes(int n) { return (n >> 7) * kTernaryPitch + n / 4; }

template <int T, bool STAGE>
struct TernaryActs {
  const char *xq[T], *xs[T];  // global (not STAGE)
  const char *lds;            // STAGE: token t's groups at lds + t * ternary_token_bytes(n), its scales after them
  int n;
  HQ_DEV const char *group(int t, int g) const {
    return STAGE ? lds + t * ternary_token_bytes(n) + g * kTernaryPitch : xq[t] + (int64_t)g * 128;
  }
  HQ_DEV const char *area(int t) const { return STAGE ? lds + t * ternary_token_bytes(n) + (n >> 7) * kTernaryPitch : xs[t]; }
};

// plane p of block h of a group's dword of codes: ternary's 2-bit codes, or binary's bit 4h + p doubled
template <bool BIN, int H, int P>
HQ_DEV uint32_t plane_codes(uint32_t w) {
  if (BIN) return ((w >> (4 * H + P)) & 0x01010101u) << 1;
  return codes<P>(w);
}

// Ternary activations staged in nibbles (NIB: ternary weights, activations in LDS).  A code dword w (bytes c0..c0+3
// of a block, plane p at bits 2p of each byte) gives two words of eight 4-bit codes with one AND each: w & 0x33333333
// (nibble 2j: plane 0 of byte c0 + j, nibble 2j + 1: plane 2) and (w >> 2) & 0x33333333 (planes 1 and 3).  The
// staging writes each activation a = 16 hi + lo (hi = a >> 4 in -8..7, lo = a & 15 in 0..15) into the same nibble
// places, so that sum(code a) = 16 v_dot8_i32_i4(codes, hi) + v_dot8_u32_u4(codes, lo): the same integer, from two
// dot instructions and three to take a dword's codes apart instead of four and seven.  A staged block of 64 bytes
// holds for each dword column j (bytes c0 = 4 j ..) the words {lo of planes 0 / 2, hi of 0 / 2, lo of 1 / 3, hi of
// 1 / 3}; from the interleaved block's plane dwords P0..P3 of column j:
HQ_DEV uint4 nibble_column(uint32_t p0, uint32_t p1, uint32_t p2, uint32_t p3) {
  constexpr uint32_t M = 0x0f0f0f0fu;
  return make_uint4((p0 & M) | ((p2 << 4) & ~M), ((p0 >> 4) & M) | (p2 & ~M), (p1 & M) | ((p3 << 4) & ~M),
                    ((p1 >> 4) & M) | (p3 & ~M));
}
HQ_DEV int32_t nibble_dot(uint32_t w, const uint4 &a, int32_t lo_in, int32_t &hi) {
  const uint32_t n02 = w & 0x33333333u, n13 = (w >> 2) & 0x33333333u;
  uint32_t lo = __builtin_amdgcn_udot8(n02, a.x, (uint32_t)lo_in, false);
  lo = __builtin_amdgcn_udot8(n13, a.z, lo, false);
  hi = __builtin_amdgcn_sdot8((int32_t)n02, (int32_t)a.y, hi, false);
  hi = __builtin_amdgcn_sdot8((int32_t)n13, (int32_t)a.w, hi, false);
  return (int32_t)lo;
}

template <int T, bool STAGE, int L, bool BIN>
HQ_DEV void ternary_step(FoldL<T, L> &f, const TernaryActs<T, STAGE> &A, const uint32_t w[8], float d, int g,
                         bool valid, int buf, int slot, int lane, float acc[T]) {
  constexpr bool NIB = STAGE && !BIN;
  if constexpr (NIB) {
#pragma unroll
    for (int t = 0; t < T; t++) {
      const char *xb = A.group(t, g);
      const float *xs = (const float *)A.area(t);
      const float4 sc = *(const float4 *)(xs + 4 * g);
      const int4 su = *(const int4 *)((const int32_t *)(xs + (A.n >> 5)) + 4 * g);
      const float scale[4] = {sc.x, sc.y, sc.z, sc.w};
      const int32_t sums[4] = {su.x, su.y, su.z, su.w};
#pragma unroll
      for (int k = 0; k < 4; k++) {  // part k: block k / 2, columns 2 (k % 2), + 1 (code dwords 2k, 2k + 1)
        const uint4 a0 = ld16(xb + 32 * k), a1 = ld16(xb + 32 * k + 16);
        int32_t hi = 0;
        int32_t lo = nibble_dot(w[2 * k], a0, sums[k], hi);
        lo = nibble_dot(w[2 * k + 1], a1, lo, hi);
        const int32_t dot = (int32_t)((uint32_t)lo + ((uint32_t)hi << 4));  // wrapping, as the dot4 chain adds
        f.v[buf][slot][t][k][lane] = valid ? fmul(fmul((float)dot, scale[k]), d) : 0.0f;
      }
    }
    fold_step_l<T, L>(f, buf, slot, lane, acc);
    return;
  }
#pragma unroll
  for (int t = 0; t < T; t++) {
    const char *xb = A.group(t, g);
    const float *xs = (const float *)A.area(t);
    const float4 sc = *(const float4 *)(xs + 4 * g);
    const int4 su = *(const int4 *)((const int32_t *)(xs + (A.n >> 5)) + 4 * g);
    const float scale[4] = {sc.x, sc.y, sc.z, sc.w};
    const int32_t sums[4] = {su.x, su.y, su.z, su.w};
#pragma unroll
    for (int h = 0; h < 2; h++) {
      uint32_t a[16];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint4 v = ld16(xb + 64 * h + 16 * q);
        a[4 * q] = v.x; a[4 * q + 1] = v.y; a[4 * q + 2] = v.z; a[4 * q + 3] = v.w;
      }
#pragma unroll
      for (int s = 0; s < 2; s++) {
        const int wi = BIN ? 2 * s : 4 * h + 2 * s;
        const uint32_t w0 = w[wi], w1 = w[wi + 1];
        int32_t dot = sums[2 * h + s];
        if (h == 0) {
          dot = sdot4((int32_t)plane_codes<BIN, 0, 0>(w0), (int32_t)a[0 + 2 * s], dot);
          dot = sdot4((int32_t)plane_codes<BIN, 0, 0>(w1), (int32_t)a[1 + 2 * s], dot);
          dot = sdot4((int32_t)plane_codes<BIN, 0, 1>(w0), (int32_t)a[4 + 2 * s], dot);
          dot = sdot4((int32_t)plane_codes<BIN, 0, 1>(w1), (int32_t)a[5 + 2 * s], dot);
          dot = sdot4((int32_t)plane_codes<BIN, 0, 2>(w0), (int32_t)a[8 + 2 * s], dot);
          dot = sdot4((int32_t)plane_codes<BIN, 0, 2>(w1), (int32_t)a[9 + 2 * s], dot);
          dot = sdot4((int32_t)plane_codes<BIN, 0, 3>(w0), (int32_t)a[12 + 2 * s], dot);
          dot = sdot4((int32_t)plane_codes<BIN, 0, 3>(w1), (int32_t)a[13 + 2 * s], dot);
        } else {
          dot = sdot4((int32_t)plane_codes<BIN, 1, 0>(w0), (int32_t)a[0 + 2 * s], dot);
          dot = sdot4((int32_t)plane_codes<BIN, 1, 0>(w1), (int32_t)a[1 + 2 * s], dot);
          dot = sdot4((int32_t)plane_codes<BIN, 1, 1>(w0), (int32_t)a[4 + 2 * s], dot);
          dot = sdot4((int32_t)plane_codes<BIN, 1, 1>(w1), (int32_t)a[5 + 2 * s], dot);
          dot = sdot4((int32_t)plane_codes<BIN, 1, 2>(w0), (int32_t)a[8 + 2 * s], dot);
          dot = sdot4((int32_t)plane_codes<BIN, 1, 2>(w1), (int32_t)a[9 + 2 * s], dot);
          dot = sdot4((int32_t)plane_codes<BIN, 1, 3>(w0), (int32_t)a[12 + 2 * s], dot);
          dot = sdot4((int32_t)plane_codes<BIN, 1, 3>(w1), (int32_t)a[13 + 2 * s], dot);
        }
        const int k = 2 * h + s;
        // f(f(whole * xs) * d) (relaxed/signs.ts:31)
        f.v[buf][slot][t][k][lane] = valid ? fmul(fmul((float)dot, scale[k]), d) : 0.0f;
      }
    }
  }
  fold_step_l<T, L>(f, buf, slot, lane, acc);
}

// the codes and group scales of U steps of a lane (step it: group L it + lane; past the row's groups, group 0):
// 32 bytes a group (ternary) or 16 (binary, in w[u][0..3])
template <int L, bool BIN>
struct TernaryChunk {
  uint32_t w[kTernarySteps][8];
  uint32_t h[kTernarySteps];
  HQ_DEV void load(const char *wrow, const uint16_t *srow, int it0, int lane, int groups) {
#pragma unroll
    for (int u = 0; u < kTernarySteps; u++) {
      const int g = (it0 + u) * L + lane;
      const int gl = g < groups ? g : 0;
      if (BIN) {
        const uint4 a = ldw16(wrow + gl * 16);
        w[u][0] = a.x; w[u][1] = a.y; w[u][2] = a.z; w[u][3] = a.w;
      } else {
        const uint4 a = ldw16(wrow + gl * 32), b = ldw16(wrow + gl * 32 + 16);
        w[u][0] = a.x; w[u][1] = a.y; w[u][2] = a.z; w[u][3] = a.w;
        w[u][4] = b.x; w[u][5] = b.y; w[u][6] = b.z; w[u][7] = b.w;
      }
      h[u] = srow[gl];
    }
  }
  template <int T, bool STAGE>
  HQ_DEV void run(FoldL<T, L> &f, const TernaryActs<T, STAGE> &A, int it0, int steps, int groups, int slot, int lane,
                  float acc[T]) const {
    // every step of the chunk, also those past the row (their lanes' parts are +0, which leaves an accumulator as it
    // is: one is never -0): no branch between a chunk's loads and their use
#pragma unroll
    for (int u = 0; u < kTernarySteps; u++) {
      const int it = it0 + u;
      const int g = it * L + lane;
      const bool valid = g < groups;
      ternary_step<T, STAGE, L, BIN>(f, A, w[u], half_to_float(h[u]), valid ? g : 0, valid, it & 1, slot, lane, acc);
    }
  }
};

// A ternary block is W waves, 64 W / L rows: 4, or for one token 5 or 6, the count chosen a launch by ternary_waves
constexpr int kTernMaxWaves = 6;
// rows of L lanes (16: 16 rows a block; 32 for long rows: twice the waves on the same rows)
template <int T, bool STAGE, int L, bool BIN, int W>
HQ_DEV void ternary_rows(const Job &J, int blk, char *acts, FoldL<T, L> *fold) {
  const int lane = threadIdx.x & (L - 1);
  const int wave = threadIdx.x >> 6, slot = (threadIdx.x & 63) / L;
  constexpr int threads = 64 * W;
  const int row_u = J.r0 + blk * (threads / L) + threadIdx.x / L;
  const bool live = row_u < J.r1;
  const int row = live ? row_u : J.r1 - 1;
  const int groups = J.n >> 7;
  const char *wrow = J.wq + (int64_t)row * groups * (BIN ? 16 : 32);
  const uint16_t *srow = (const uint16_t *)J.ws + (int64_t)row * groups;
  FoldL<T, L> &f = fold[wave];
  TernaryActs<T, STAGE> A;
#pragma unroll
  for (int t = 0; t < T; t++) {
    A.xq[t] = J.xq + t * J.frame;
    A.xs[t] = J.xs + t * J.sframe;
  }
  A.lds = acts;
  A.n = J.n;

  float acc[T];
#pragma unroll
  for (int t = 0; t < T; t++) acc[t] = 0.0f;
  const int steps = (groups + L - 1) / L;
  TernaryChunk<L, BIN> a, b;
  // the first codes in flight during the staging: the staged bytes' stores then wait for them too (the memory
  // counter is in order), but the two round trips overlap instead of following one another
  a.load(wrow, srow, 0, lane, groups);
  if (STAGE && !BIN) {
    // every token's n bytes (a group's 128 in 144) as nibbles (nibble_column: a 64-byte block a thread at a time, two
    // in flight), then its n/32 scales and n/32 sums, 16 bytes a thread at a time
    const int per = ternary_token_bytes(J.n), nb = J.n / 64, gb = groups * kTernaryPitch, area = J.n / 64;
    for (int t = 0; t < T; t++) {
      for (int base = 0; base < nb; base += 2 * threads) {
        uint4 v[2][4];
#pragma unroll
        for (int u = 0; u < 2; u++) {
          const int b = base + u * threads + (int)threadIdx.x;
          if (b < nb)
#pragma unroll
            for (int q = 0; q < 4; q++) v[u][q] = ld16(J.xq + t * J.frame + 64 * b + 16 * q);
        }
#pragma unroll
        for (int u = 0; u < 2; u++) {
          const int b = base + u * threads + (int)threadIdx.x;
          if (b < nb) {
            uint4 *dst = (uint4 *)(acts + t * per + (b >> 1) * kTernaryPitch + 64 * (b & 1));
            dst[0] = nibble_column(v[u][0].x, v[u][1].x, v[u][2].x, v[u][3].x);
            dst[1] = nibble_column(v[u][0].y, v[u][1].y, v[u][2].y, v[u][3].y);
            dst[2] = nibble_column(v[u][0].z, v[u][1].z, v[u][2].z, v[u][3].z);
            dst[3] = nibble_column(v[u][0].w, v[u][1].w, v[u][2].w, v[u][3].w);
          }
        }
      }
      for (int c = (int)threadIdx.x; c < area; c += threads)
        *(uint4 *)(acts + t * per + gb + 16 * c) = ld16(J.xs + t * J.sframe + 16 * c);
    }
  } else if (STAGE) {
    // every token's n bytes (a group's 128 in 144), then its n/32 scales and n/32 sums: 16 bytes a thread at a time,
    // eight loads of a thread in flight before their stores
    const int per = ternary_token_bytes(J.n), chunks = (J.n + J.n / 4) / 16, gb = groups * kTernaryPitch;
    constexpr int K = 8;
    for (int t = 0; t < T; t++)
      for (int base = 0; base < chunks; base += K * threads) {
        uint4 v[K];
#pragma unroll
        for (int u = 0; u < K; u++) {
          const int o = 16 * (base + u * threads + (int)threadIdx.x);
          if (o < J.n) v[u] = ld16(J.xq + t * J.frame + o);
          else if (o < J.n + J.n / 4) v[u] = ld16(J.xs + t * J.sframe + (o - J.n));
        }
#pragma unroll
        for (int u = 0; u < K; u++) {
          const int o = 16 * (base + u * threads + (int)threadIdx.x);
          if (o < J.n) *(uint4 *)(acts + t * per + (o >> 7) * kTernaryPitch + (o & 127)) = v[u];
          else if (o < J.n + J.n / 4) *(uint4 *)(acts + t * per + gb + (o - J.n)) = v[u];
        }
      }
  }
  if (STAGE) __syncthreads();
  // the next step's codes are loaded whether or not the row has that step (past its groups a lane loads its group 0
  // again): the same loads outstanding on every path, so using a step's codes waits for them alone and not for the
  // ones just issued
  for (int it = 0; it < steps; it += 2 * kTernarySteps) {
    b.load(wrow, srow, it + kTernarySteps, lane, groups);
    a.template run<T, STAGE>(f, A, it, steps, groups, slot, lane, acc);
    if (it + kTernarySteps >= steps) break;  // uniform
    a.load(wrow, srow, it + 2 * kTernarySteps, lane, groups);
    b.template run<T, STAGE>(f, A, it + kTernarySteps, steps, groups, slot, lane, acc);
  }
  float sum[T];
#pragma unroll
  for (int t = 0; t < T; t++)
    sum[t] = fadd(fadd(fadd(acc[t], from_lane_plus<1>(acc[t])), from_lane_plus<2>(acc[t])), from_lane_plus<3>(acc[t]));
  if (live && lane == 0) {
#pragma unroll
    for (int t = 0; t < T; t++) ((float *)(J.out + t * J.os))[row] = sum[t];
  }
}

// PRE (one token, a job a grid row), as gemv_relaxed's: the first job's pieces from the preloaded arguments
template <int T, bool STAGE, int L, bool BIN, bool BY, int PRE, int W>
__global__ __launch_bounds__(64 * W) void gemv_ternary(char *out, const char *xq, const char *xs, const char *wq,
                                                       const char *ws, int32_t n, int32_t r0, int32_t r1, int32_t pr,
                                                       GemvBatch batch) {
  extern __shared__ __align__(16) char acts[];
  __shared__ FoldL<T, L> fold[W];
  if (PRE) {
    const int a = r0 + (int)blockIdx.y * pr;
    if (PRE == 2 || a < r1) {
      const Job J{out, xq, xs, wq, ws, nullptr, n, a, min(a + pr, r1), 1, 0, 0, 0, 0};
      ternary_rows<T, STAGE, L, BIN, W>(J, (int)blockIdx.x, acts, fold);
      return;
    }
  }
  int jb, blk;
  block_job<BY>(batch, jb, blk);
  ternary_rows<T, STAGE, L, BIN, W>(batch.job[jb], blk, acts, fold);
}

// the LDS a ternary block stages for T tokens of n activations (beyond: read through the L1)
constexpr size_t kTernaryStageMax = 64 * 1024;
// lanes a row of ternary weights: 32 for rows of at least kTernaryLongRow weights, 8 for rows of an odd number of
// 8-group steps (no lanes idle in the last step), else 16
constexpr int kTernaryLongRow = 8192;
HQ_HOST_DEV constexpr int ternary_lanes(int n) {
  return n >= kTernaryLongRow ? 32 : ((n >> 7) % 16 != 0 && (n >> 7) % 8 == 0) ? 8 : 16;
}
HQ_HOST_DEV constexpr size_t ternary_stage_bytes(int T, int n) { return (size_t)T * ternary_token_bytes(n); }

// lead_r1, pr: the end of the rows of the job whose pieces come first (b.job[0] is its first piece), and the rows a
// piece (the arguments PRE reads).  CACHED kernels exist for 16-lane rows only (relaxed_cached's launches).
template <int PACK, int T, int SRC, bool BY, int PRE, int U1, int NT, bool CACHED>
void launch_relaxed_by(const GemvBatch &b, dim3 grid, int32_t lead_r1, int32_t pr, bool wc, int lanes, size_t lds,
                       hipStream_t s) {
  const dim3 block(NT);
  const Job &J = b.job[0];
  const int32_t frame = (int32_t)J.frame;  // (PRE: J.frame == J.sframe, below 2^31)
  if constexpr (!CACHED) {
    if (lanes == 32) {
      if (wc) hipLaunchKernelGGL((gemv_relaxed<PACK, T, true, SRC, 32, BY, PRE, U1, NT, false>), grid, block, lds, s, J.xq,
                                 J.xs, J.wq, J.ws, J.n, J.r0, lead_r1, pr, frame, J.out, J.os, J.wc, b);
      else hipLaunchKernelGGL((gemv_relaxed<PACK, T, false, SRC, 32, BY, PRE, U1, NT, false>), grid, block, lds, s, J.xq,
                              J.xs, J.wq, J.ws, J.n, J.r0, lead_r1, pr, frame, J.out, J.os, J.wc, b);
      return;
    }
  }
  if (wc) hipLaunchKernelGGL((gemv_relaxed<PACK, T, true, SRC, 16, BY, PRE, U1, NT, CACHED>), grid, block, lds, s, J.xq,
                             J.xs, J.wq, J.ws, J.n, J.r0, lead_r1, pr, frame, J.out, J.os, J.wc, b);
  else hipLaunchKernelGGL((gemv_relaxed<PACK, T, false, SRC, 16, BY, PRE, U1, NT, CACHED>), grid, block, lds, s, J.xq,
                          J.xs, J.wq, J.ws, J.n, J.r0, lead_r1, pr, frame, J.out, J.os, J.wc, b);
}
template <int PACK, int T, int SRC, int NT, bool CACHED>
hipError_t launch_relaxed_nt(const GemvBatch &b, dim3 grid, const JobPieces &p, bool wc, int lanes, size_t lds,
                             hipStream_t s) {
  // PRE takes one stride for a token's activations and scales (the tile kinds' frame; one token: none read)
  const Job &J = b.job[0];
  const bool pre = p.by && (T == 1 || (J.frame == J.sframe && J.frame >= 0 && J.frame <= INT32_MAX));
  if constexpr (!CACHED) {
    if (T == 1 && lanes == 32 && relaxed_pairs_of_steps(PACK == 8 ? Q8R : Q6R, T, J.n)) {
      // (T == 1 ? 2 : 4: the kernels of 2..4 tokens are never made with U1 = 2)
      constexpr int U1 = T == 1 ? 2 : 4;
      if (pre && p.lead_pieces == b.njobs)
        launch_relaxed_by<PACK, T, SRC, true, 2, U1, NT, false>(b, grid, p.lead_r1, p.rows, wc, lanes, lds, s);
      else if (pre)
        launch_relaxed_by<PACK, T, SRC, true, 1, U1, NT, false>(b, grid, p.lead_r1, p.rows, wc, lanes, lds, s);
      else if (p.by) launch_relaxed_by<PACK, T, SRC, true, 0, U1, NT, false>(b, grid, p.lead_r1, p.rows, wc, lanes, lds, s);
      else launch_relaxed_by<PACK, T, SRC, false, 0, U1, NT, false>(b, grid, 0, 0, wc, lanes, lds, s);
      return hipGetLastError();
    }
  }
  if (pre && p.lead_pieces == b.njobs)
    launch_relaxed_by<PACK, T, SRC, true, 2, 4, NT, CACHED>(b, grid, p.lead_r1, p.rows, wc, lanes, lds, s);
  else if (pre)
    launch_relaxed_by<PACK, T, SRC, true, 1, 4, NT, CACHED>(b, grid, p.lead_r1, p.rows, wc, lanes, lds, s);
  else if (p.by) launch_relaxed_by<PACK, T, SRC, true, 0, 4, NT, CACHED>(b, grid, p.lead_r1, p.rows, wc, lanes, lds, s);
  else launch_relaxed_by<PACK, T, SRC, false, 0, 4, NT, CACHED>(b, grid, 0, 0, wc, lanes, lds, s);
  return hipGetLastError();
}
// nt: the block's threads, relaxed_threads' or (one token) kOneTokenSmall; cached: relaxed_cached's choice (one token
// of int8 on 16-lane rows only: the other forms read their weights one way)
template <int PACK, int T, int SRC>
hipError_t launch_relaxed(const GemvBatch &b, dim3 grid, const JobPieces &p, bool wc, int lanes, size_t lds, int nt,
                          bool cached, hipStream_t s) {
  constexpr int big = relaxed_threads(T, SRC == STAGED);
  if constexpr (T == 1 && SRC == GLOBAL && PACK == 8) {  // (RelaxedChunk's PAIRED form)
    if (cached && lanes == 16) {
      if (nt == kOneTokenSmall) return launch_relaxed_nt<PACK, T, SRC, kOneTokenSmall, true>(b, grid, p, wc, lanes, lds, s);
      return launch_relaxed_nt<PACK, T, SRC, big, true>(b, grid, p, wc, lanes, lds, s);
    }
  }
  // (T == 1 ? kOneTokenSmall : big: the kernels of 2..4 tokens are never made with the small blocks)
  if (T == 1 && nt == kOneTokenSmall)
    return launch_relaxed_nt<PACK, T, SRC, T == 1 ? kOneTokenSmall : big, false>(b, grid, p, wc, lanes, lds, s);
  return launch_relaxed_nt<PACK, T, SRC, big, false>(b, grid, p, wc, lanes, lds, s);
}

// ternary / binary: rows of ternary_lanes(n) lanes, the activations staged in LDS when they fit
template <int T, bool BIN, bool BY, int PRE, int W>
void launch_signs_w(const GemvBatch &b, dim3 grid, int32_t lead_r1, int32_t pr, hipStream_t s) {
  const Job &J = b.job[0];
  int nmax = 0;
  for (int j = 0; j < b.njobs; j++) nmax = b.job[j].n > nmax ? b.job[j].n : nmax;
  const size_t bytes = ternary_stage_bytes(T, nmax);
  const bool stage = bytes <= kTernaryStageMax;
  const dim3 block(64 * W);
  switch (ternary_lanes(nmax)) {
  case 32:
    if (stage)
      hipLaunchKernelGGL((gemv_ternary<T, true, 32, BIN, BY, PRE, W>), grid, block, bytes, s, J.out, J.xq, J.xs, J.wq, J.ws,
                         J.n, J.r0, lead_r1, pr, b);
    else
      hipLaunchKernelGGL((gemv_ternary<T, false, 32, BIN, BY, PRE, W>), grid, block, 0, s, J.out, J.xq, J.xs, J.wq, J.ws,
                         J.n, J.r0, lead_r1, pr, b);
    break;
  case 8:
    if (stage)
      hipLaunchKernelGGL((gemv_ternary<T, true, 8, BIN, BY, PRE, W>), grid, block, bytes, s, J.out, J.xq, J.xs, J.wq, J.ws,
                         J.n, J.r0, lead_r1, pr, b);
    else
      hipLaunchKernelGGL((gemv_ternary<T, false, 8, BIN, BY, PRE, W>), grid, block, 0, s, J.out, J.xq, J.xs, J.wq, J.ws,
                         J.n, J.r0, lead_r1, pr, b);
    break;
  default:
    if (stage)
      hipLaunchKernelGGL((gemv_ternary<T, true, 16, BIN, BY, PRE, W>), grid, block, bytes, s, J.out, J.xq, J.xs, J.wq, J.ws,
                         J.n, J.r0, lead_r1, pr, b);
    else
      hipLaunchKernelGGL((gemv_ternary<T, false, 16, BIN, BY, PRE, W>), grid, block, 0, s, J.out, J.xq, J.xs, J.wq, J.ws,
                         J.n, J.r0, lead_r1, pr, b);
  }
}
// (2..4 tokens: 4 waves; the kernels of 5 and 6 are made for one token only)
template <int T, bool BIN, bool BY, int PRE>
void launch_signs_by(const GemvBatch &b, dim3 grid, int threads, int32_t lead_r1, int32_t pr, hipStream_t s) {
  if (threads == 320) launch_signs_w<T, BIN, BY, PRE, T == 1 ? 5 : 4>(b, grid, lead_r1, pr, s);
  else if (threads == 384) launch_signs_w<T, BIN, BY, PRE, T == 1 ? 6 : 4>(b, grid, lead_r1, pr, s);
  else launch_signs_w<T, BIN, BY, PRE, 4>(b, grid, lead_r1, pr, s);
}
template <int T, bool BIN>
hipError_t launch_signs(const GemvBatch &b, dim3 grid, int threads, const JobPieces &p, hipStream_t s) {
  if (T == 1 && p.by && p.lead_pieces == b.njobs)
    launch_signs_by<T, BIN, true, T == 1 ? 2 : 0>(b, grid, threads, p.lead_r1, p.rows, s);
  else if (T == 1 && p.by)
    launch_signs_by<T, BIN, true, T == 1 ? 1 : 0>(b, grid, threads, p.lead_r1, p.rows, s);
  else if (p.by) launch_signs_by<T, BIN, true, 0>(b, grid, threads, p.lead_r1, p.rows, s);
  else launch_signs_by<T, BIN, false, 0>(b, grid, threads, 0, 0, s);
  return hipGetLastError();
}

// grid: (blocks) with the jobs found through block0, or (blocks a piece, pieces) when p.by
template <int T>
hipError_t launch_t(Kind kind, const GemvBatch &b, dim3 grid, const JobPieces &p, bool wc, int src, int lanes,
                    size_t lds, int tern_threads, int relaxed_nt, bool cached, hipStream_t s) {
  const dim3 block(256);
  switch (kind) {
  case Q8R:
  case Q6R:
    if (kind == Q8R) {
      if (src == STAGED) return launch_relaxed<8, T, STAGED>(b, grid, p, wc, lanes, lds, relaxed_nt, cached, s);
      return launch_relaxed<8, T, GLOBAL>(b, grid, p, wc, lanes, 0, relaxed_nt, cached, s);
    }
    if (src == STAGED) return launch_relaxed<6, T, STAGED>(b, grid, p, wc, lanes, lds, relaxed_nt, cached, s);
    return launch_relaxed<6, T, GLOBAL>(b, grid, p, wc, lanes, 0, relaxed_nt, cached, s);
  case Q8: hipLaunchKernelGGL((gemv_plain<8, T>), grid, block, 0, s, b); break;
  case Q6: hipLaunchKernelGGL((gemv_plain<6, T>), grid, block, 0, s, b); break;
  case T2R:
  case T2: return launch_signs<T, false>(b, grid, tern_threads, p, s);
  case B1R:
  case B1: return launch_signs<T, true>(b, grid, tern_threads, p, s);
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

// the largest activations (bytes and scales of all tokens) a block of 2..4 tokens copies into LDS (STAGED) rather
// than reading them through the L1: two blocks a CU.  Four tokens of the 8B down projection (64.5 KB) staged make the
// decode step 2.37 -> 2.29 ms: in a step the activations were just written by quantize_x, and read through the caches
// every wave fetches them anew (with activations left warm by earlier launches the staged form is 2 % slower).  One
// token is read through the caches (measured 9 % faster than staged).
constexpr size_t kGemvStageMax = 80 * 1024;

namespace {
// the fraction of the last round's block slots a launch of `blocks` fills (rounds of one block a compute unit)
double round_fill(int64_t blocks) {
  const int64_t cus = cu_count();
  return blocks <= 0 ? 1.0 : (double)blocks / (double)(((blocks + cus - 1) / cus) * cus);
}
// the blocks of `rpb` rows the jobs take
int64_t blocks_of(const Job *jobs, int32_t njobs, int rpb) {
  int64_t n = 0;
  for (int j = 0; j < njobs; j++) n += (jobs[j].r1 - jobs[j].r0 + rpb - 1) / rpb;
  return n;
}
// A ternary / binary launch's waves a block (one token: 4 to 6; more: 4): the count whose blocks come closest to
// whole rounds of one block a compute unit (the last round's empty slots the fewest, the fewer waves on a tie).
// Measured on the 27B shapes, A/B on one box: the down projection's 5120 rows in 5-wave blocks (512 blocks, two
// rounds) 2.76 -> 2.99 TB/s against 4 waves (640: three rounds, the last a quarter full), gate+up's 2 x 17408 in
// 6-wave blocks (726, three rounds) 4.0 -> 4.18.
int ternary_waves(const Job *jobs, int32_t njobs, int lanes) {
  int best = 4;
  double best_fill = 0.0;
  if (jobs[0].count != 1) return 4;
  for (int w = 4; w <= kTernMaxWaves; w++) {
    const double fill = round_fill(blocks_of(jobs, njobs, 64 * w / lanes));
    if (fill > best_fill + 1e-9) best = w, best_fill = fill;
  }
  return best;
}

// A relaxed launch's threads a block: relaxed_threads', or for one token blocks of one wave where those come closer
// to whole rounds (LFM2-350M's o and down projections, 1024 rows of 16 lanes: 128 blocks of 8 rows fill half the
// compute units, 256 of 4 all of them).  Measured A/B on one box: config 1's step 1.58 -> 1.65 TB/s, the 27B int6
// down projection 4.53 -> 4.63; the 8B shapes' launches fill whole rounds either way and keep 128 threads.
int relaxed_block_threads(const Job *jobs, int32_t njobs, int T, bool staged, int lanes) {
  const int big = relaxed_threads(T, staged);
  if (T != 1) return big;
  const double small = round_fill(blocks_of(jobs, njobs, kOneTokenSmall / lanes));
  return small > round_fill(blocks_of(jobs, njobs, big / lanes)) + 0.02 ? kOneTokenSmall : big;
}

// One token's int8 weights are streamed past the caches (non-temporal loads: on the 8B decode step 1.83 -> 1.77 ms)
// unless the launch's weights come to less than kCachedWeights bytes: a small model's matrices can stay in the caches
// from one step to the next, which streaming them throws away.  Measured A/B on one box: stories15M's 768 x 288
// (config 0, 221 KB a launch) 2.43 us a launch streamed against 2.13 cached; LFM2-350M's phases (config 1, 1 MiB and
// more) 3.53 streamed against 3.64.
constexpr int64_t kCachedWeights = 1 << 20;
bool relaxed_cached(Kind kind, const Job *jobs, int32_t njobs) {
  int64_t bytes = 0;
  for (int j = 0; j < njobs; j++) bytes += (int64_t)(jobs[j].r1 - jobs[j].r0) * jobs[j].n;
  return kind == Q8R && jobs[0].count == 1 && bytes < kCachedWeights;
}

hipError_t launch_batch(Kind kind, const Job *jobs, int32_t njobs, hipStream_t s) {
  if (njobs < 1 || njobs > kMaxJobs) return hipErrorInvalidValue;
  GemvBatch b{};
  int blocks = 0, nmax = 0;
  for (int j = 0; j < njobs; j++) nmax = jobs[j].n > nmax ? jobs[j].n : nmax;
  const int T = jobs[0].count;
  const bool relaxed = kind == Q8R || kind == Q6R;
  const int lanes = relaxed ? relaxed_lanes(kind, T, nmax) : 16;
  const size_t lds = (size_t)act_lds_bytes(T, nmax);
  // staged in LDS for 2..4 tokens (each row's lanes read every token's activations: measured 4 % faster at M = 4)
  const int src = T > 1 && lds <= kGemvStageMax ? STAGED : GLOBAL;
  const int tern_threads = signs_kind(kind) ? 64 * ternary_waves(jobs, njobs, ternary_lanes(nmax)) : 0;
  const int relaxed_nt = relaxed ? relaxed_block_threads(jobs, njobs, T, src == STAGED, lanes) : 0;
  const bool cached = relaxed_cached(kind, jobs, njobs);
  const int rpb = signs_kind(kind) ? tern_threads / ternary_lanes(nmax)
                  : relaxed          ? relaxed_nt / lanes
                                     : kRowsPerBlock;
  for (int j = 0; j < njobs; j++) {
    b.job[j] = jobs[j];
    b.block0[j] = blocks;
    blocks += (jobs[j].r1 - jobs[j].r0 + rpb - 1) / rpb;
  }
  b.block0[njobs] = blocks;
  for (int j = njobs + 1; j <= kMaxJobs; j++) b.block0[j] = INT32_MAX;  // job_of's comparisons past the jobs
  b.njobs = njobs;
  if (blocks == 0) return hipSuccess;
  dim3 grid(blocks);
  // The relaxed and signs kernels take a job a grid row where every job's blocks cut into pieces of g blocks (g the
  // greatest common divisor of the jobs' block counts) make at most kMaxJobs pieces: a block's job is then blockIdx.y,
  // and its fields are read in the kernel's first round of scalar loads instead of a round after the block0 it is
  // found by (measured on the 8B decode: the o and down projections' launches 0.14-0.2 us shorter with one job).
  JobPieces pc{false, 0, 0, 0};
  if (relaxed || signs_kind(kind)) {
    int g = 0;
    for (int j = 0; j < njobs; j++) g = std::gcd(g, b.block0[j + 1] - b.block0[j]);
    if (blocks / g <= kMaxJobs) {
      GemvBatch p{};
      int pieces = 0, lead = -1;
      for (int j = 0; j < njobs; j++)
        for (int r = jobs[j].r0; r < jobs[j].r1; r += g * rpb) {
          if (pieces == 0) lead = j, pc.lead_r1 = jobs[j].r1;
          if (j == lead) ++pc.lead_pieces;
          p.job[pieces] = jobs[j];
          p.job[pieces].r0 = r;
          p.job[pieces].r1 = std::min(r + g * rpb, jobs[j].r1);
          p.block0[pieces] = pieces * g;
          ++pieces;
        }
      for (int j = pieces; j <= kMaxJobs; j++) p.block0[j] = j == pieces ? blocks : INT32_MAX;
      p.njobs = pieces;
      b = p;
      grid = dim3(g, pieces);
      pc.by = true;
      pc.rows = g * rpb;
    }
  }
  const bool wc = jobs[0].wc != nullptr;
  switch (T) {
  case 1: return launch_t<1>(kind, b, grid, pc, wc, src, lanes, lds, tern_threads, relaxed_nt, cached, s);
  case 2: return launch_t<2>(kind, b, grid, pc, wc, src, lanes, lds, tern_threads, relaxed_nt, cached, s);
  case 3: return launch_t<3>(kind, b, grid, pc, wc, src, lanes, lds, tern_threads, relaxed_nt, cached, s);
  case 4: return launch_t<4>(kind, b, grid, pc, wc, src, lanes, lds, tern_threads, relaxed_nt, cached, s);
  default: return hipErrorInvalidValue;
  }
}
}  // namespace

// jobs: one kind, one token count (1..4), one wc-ness (all with corrections or all without)
hipError_t launch_gemv(Kind kind, const Job *jobs, int32_t njobs, hipStream_t s) {
  return launch_batch(kind, jobs, njobs, s);
}

}  // namespace hq
