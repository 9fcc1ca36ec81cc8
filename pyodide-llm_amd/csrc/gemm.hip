// gemm.hip — the prompt kernels on the matrix cores (a prompt's many tokens):
//   matmul_q8r_tile (kernels/relaxed/int8.ts:52-166), matmul_q6r for many tokens (jobs.ts:243-248 runs it a token at
//   a time: every (row, token) is matmul_q6r's number), matmul_t2r_tile (kernels/relaxed/signs.ts:77-114, 120-122).
//
// The matrix core gives each group's exact integer: v_mfma_i32_32x32x32_i8 with K = 32 is one scale group of 32 (for
// ternary, one part of 32 of a group of 128), and the correction rides in its accumulator input:
//   int8 / int6 with the caller's wc: wc itself, so the integer is dot(w, q) + wc as the reference adds it
//     (relaxed/int8.ts:37, wrapping in int32 like i32x4.add);
//   int8 / int6 with wc == NULL: -64 sum(w), made by a second MFMA of the same weights against a constant -64
//     (the value int8_sums would have given, exact for every byte);
//   ternary: interleave()'s sums of the part (one a token), as the reference adds them.
//
// Float32 order: every (row, token) is the token kernel's number to the bit.  The reference's lane k adds groups
// 4 j + k (int8, int6) or part k of every group (ternary), in order, and the four lanes are added
// ((l0 + l1) + l2) + l3 at the end (math.ts:7-9), then (int8, int6) the groups past the last four one at a time
// (relaxed/int8.ts:40-47).  Here a wave IS a lane k of the reference: the 4 waves of one 32-row slice of the tile take
// chain k = 0..3 each, adding their groups / parts in order into registers, and at the end add their sums through LDS
// in that order.  Each term is f(f(C) * f(ws * xs)) (int8, int6) or f(f(f(C) * xs) * d) (ternary), rounded as the
// reference rounds it (-ffp-contract=off).
//
// The scales' product of int8 / int6, f(ws * xs) for every (row, token), is an outer product: four
// v_mfma_f32_4x4x1_16b_f32 (sixteen 4 x 4 outer products each, K = 1) give a 32 x 32 sub-tile's, each product rounded
// once as v_mul_f32 rounds it (subnormals included), on the matrix core.  Roofline: per output element and group the
// epilogue is then 3 VALU operations (convert, multiply, add; ternary 4: f(f(C * xs) * d) has no such product)
// against 32 MACs on the matrix core.  Without packed float32 instructions (this build turns them off) MI355X's VALU
// does 64 float32 lanes a clock a CU (4 SIMDs x 16) against 4096 int8 MACs, so the epilogue, not the MFMA, bounds
// this kernel: at best 32 / (3 x 4096 / 64) = 16.7 % of dense int8 peak, 833 TOP/s (12.5 % for ternary).
//
// A block computes a 128-row x 64-token tile.  int8 / int6: 8 waves, two a SIMD; the waves of pair p (waves 4 p ..
// 4 p + 3) take rows 64 p .. + 63 and chain w % 4, four 32 x 32 sub-tiles each (the weights' operand read once for
// two MFMAs, the tokens' for two slices); a launch of few tiles takes 64-row tiles of one pair (4 waves) instead.
// Ternary: 16 waves; wave w takes rows 32 (w / 4) .. + 31 and chain w % 4, both 32-token halves.  The operands come into LDS by direct buffer-to-LDS loads (no registers on the way), into a
// ring of 4 stage buffers: a stage is 4 groups (int8, int6) or 2 groups of 128 (ternary), and the loads of stages
// s + 1 .. s + 3 are in flight while stage s is computed.  Every wave issues the same number of loads a stage (6 for
// int8 / int6, 3 for ternary; some of them into a scratch area), so that one s_waitcnt vmcnt count means "my loads of
// stage s have landed"; a bare s_barrier then makes them everyone's.  The 16-byte chunks of a row are stored XOR-
// swizzled so that the MFMA operand reads (32 rows or tokens, one chunk each) spread over the LDS banks.  Blocks are
// ordered so that the blocks one XCD runs at a time share their rows and tokens in that XCD's L2.
//
// Measured on MI355X (8B gate+up, 2048 tokens): a stage takes about twice the sum of its MFMA, VALU and LDS time;
// the rest is waiting for the stage's loads, and the parts add up rather than overlap (one wave issues VALU at about
// half a SIMD's rate; the VALU and the matrix core run side by side only part of the time), so the kernel sits
// near 320 int8 TOP/s, well under the bound above.
#include "common.hpp"
#include "launch.hpp"

namespace hq {

namespace {

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int BR = 128, BT = 64;  // block tile: rows x tokens
constexpr int RING = 4;           // stage buffers
constexpr int AHEAD = RING - 1;   // stages loaded beyond the one computed

HQ_DEV v16i zero16i() {
  v16i z;
#pragma unroll
  for (int r = 0; r < 16; r++) z[r] = 0;
  return z;
}
HQ_DEV v4f zero4f() { return (v4f){0.0f, 0.0f, 0.0f, 0.0f}; }

// ---- loads -----------------------------------------------------------------------------------------------------
// A block's rows, tokens and scales are each one buffer resource (common.hpp's resource(): base and size in scalar
// registers): a thread's offsets are set once, a stage moves them by a scalar offset, and a load past the size reads
// nothing and returns zeros (the tiles past the last row or token, the groups past the last one: their results are
// never stored).
// direct loads into LDS: lane l's `size` bytes land at dst + size * l (dst the same in the whole wave, in M0; 2-byte
// loads land zero-extended in 4-byte slots).  Written as the instructions themselves: the compiler, which tracks
// such loads only a few at a time, would otherwise wait for every one in flight before each LDS read; here the
// waits are stage_ready's alone (which only these loads need: the loops issue no other vector memory operation).
HQ_DEV uint32_t lds_address(void *p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)p);
}
HQ_DEV void dma16(__amdgpu_buffer_rsrc_t r, void *dst, uint32_t vo, uint32_t so) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(lds_address(dst)), "v"(vo), "s"(r), "s"(so) : "memory", "m0");
}
HQ_DEV void dma4(__amdgpu_buffer_rsrc_t r, void *dst, uint32_t vo, uint32_t so) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
               :: "s"(lds_address(dst)), "v"(vo), "s"(r), "s"(so) : "memory", "m0");
}
HQ_DEV void dma2(__amdgpu_buffer_rsrc_t r, void *dst, uint32_t vo, uint32_t so) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_ushort %1, %2, %3 offen lds"
               :: "s"(lds_address(dst)), "v"(vo), "s"(r), "s"(so) : "memory", "m0");
}

// the stage's loads have landed: wait until at most N of this wave's loads are outstanding (and its LDS reads are
// done), then the block's barrier, which no memory operation is moved across
template <int N>
HQ_DEV void stage_ready() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((N & 15) | 0x70 | ((N >> 4) << 14));  // vmcnt(N) expcnt(7) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// stage s of `total` loaded stages, N loads a wave a stage: the loads issued after its own are those of the next
// min(AHEAD - 1, ...) stages
template <int N>
HQ_DEV void wait_for(int s, int total) {
  const int later = min(AHEAD - 1, total - 1 - s);
  if (later >= 2) stage_ready<2 * N>();
  else if (later == 1) stage_ready<N>();
  else stage_ready<0>();
}

// the 8 16-byte chunks of a row's 128 stage bytes: chunk c of row r is stored at c ^ swz(r), so that 8 (32 banks) or
// 16 (64 banks) consecutive rows reading the same chunk hit different banks
HQ_DEV int swz(int r) { return (r ^ (r >> 3)) & 7; }

// Which tile a block computes.  Blocks are handed to the 8 XCDs in turn (block b to XCD b % 8), and each XCD has
// its own L2: the blocks of one XCD take consecutive tiles, walked in strips of kStrip row tiles with the token tiles
// inside a strip, so that the blocks running on one XCD at a time share their weights' rows and their tokens.
constexpr int kXcds = 8, kStrip = 4;

HQ_DEV void tile_of(int b, int nb, int nrb, int &rb, int &tb) {
  const int q = nb / kXcds, r = nb % kXcds, x = b % kXcds;
  const int t = x * q + min(x, r) + b / kXcds;  // consecutive on one XCD
  const int ntb = nb / nrb;
  const int strip = t / (kStrip * ntb);
  const int first = strip * kStrip, width = min(kStrip, nrb - first);
  const int in = t - first * ntb;
  rb = first + in % width;
  tb = in / width;
}

// the 4 chains of a slice added in LDS, ((a0 + a1) + a2) + a3, for both token halves: wave k adds its sums to what
// waves 0..k-1 left (the 16 values of a lane are the same (row, token)s in the four waves of a slice); the sums end
// in chain 3's waves.  p0, p1: 4 x 64 x 16 floats each that nothing else uses meanwhile
HQ_DEV void add_chains(float acc0[16], float acc1[16], float *p0, float *p1, int slice, int chain, int lane) {
  float *q0 = p0 + (slice * 64 + lane) * 16, *q1 = p1 + (slice * 64 + lane) * 16;
  for (int k = 0; k < 4; k++) {
    __syncthreads();
    if (chain == k) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        if (k > 0) {
          acc0[r] = fadd(q0[r], acc0[r]);
          acc1[r] = fadd(q1[r], acc1[r]);
        }
        if (k < 3) {
          q0[r] = acc0[r];
          q1[r] = acc1[r];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// int8 / int6 weights, relaxed activations (matmul_q8r_tile, matmul_q6r)
// A block is 8 waves, two waves a SIMD with up to 256 registers each: wave w takes chain w % 4 of rows
// 64 (w / 4) .. + 63 (two 32-row slices) for both 32-token halves, four 32 x 32 sub-tiles, so that the MFMAs of one
// sub-tile run while the epilogue of the one before it does.
// MFMA A = weights (m = row), B = activations (n = token): lane l holds token l % 32 of its half and rows
// 8 (r / 4) + 4 (l / 32) + r % 4 of its slice (r = 0..15); K half l / 32 is bytes 16 (l / 32) .. + 15 of the group.
// ---------------------------------------------------------------------------------------------------------------
constexpr int QG = 4;  // groups a stage
// the rows of a block's tile (BRT 128: 8 waves; 64, for launches of few tiles: 4 waves, twice the blocks), its
// threads and each wave's loads a stage
template <int BRT> constexpr int q_threads() { return 4 * BRT; }
template <int BRT> constexpr int q_loads() { return BRT == 128 ? 6 : 7; }

template <int BRT>
struct alignas(16) StageQ {
  char w[BRT * 128];    // int8: BRT rows x 4 groups x 32 bytes, chunks swizzled; int6: BRT rows x 4 x 24 bytes
  char x[BT * 128];     // 64 tokens x 4 groups x 32 bytes, chunks swizzled
  float ws[QG][BRT];    // the rows' scales, group-major
  int32_t wc[QG][BRT];  // the rows' corrections (with the caller's wc), group-major
  float xs[QG][BT];     // the tokens' scales, group-major; in each 32-token half token 8 m + 4 h + i at 16 h + 4 i + m
};

// K half kh (values 16 kh .. + 15) of an int6 group (24 bytes at p, kernels/six.ts:16-31): value j's low nibble is
// in byte j % 16 (low half for j < 16, high half after), its top two bits at bits 2 (j / 8) of byte 16 + j % 8;
// widened to the int8 4 v as six_widen does
HQ_DEV v4i six_half(const char *p, int kh) {
  const uint2 a = *(const uint2 *)p, b = *(const uint2 *)(p + 8), c = *(const uint2 *)(p + 16);
  const uint32_t lo[4] = {a.x, a.y, b.x, b.y};
  const uint32_t top[2] = {c.x, c.y};
  const int sl = 4 * kh;
  v4i v;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t nib = ((lo[i] >> sl) & 0x0f0f0f0fu) << 2;
    const uint32_t t = top[i & 1] << ((i < 2 ? 6 : 4) - sl);
    v[i] = (int32_t)((t & 0xc0c0c0c0u) | nib);
  }
  return v;
}

// a block's loads of int8 / int6 stages: wave w's q_loads a stage and their offsets
template <int PACK, bool WC, int BRT>
struct Relaxed {
  static constexpr int GB = PACK == 8 ? 32 : 24;  // bytes of a group of weights
  static constexpr int NW = BRT / 16;             // waves
  static constexpr int XPW = 8 / NW;              // 1 KB pieces of the activations a wave
  static constexpr int SPG = BRT / 64;            // 64-row pieces of a group's scales
  __amdgpu_buffer_rsrc_t rw, rx, rws, rwc, rxs;
  uint32_t oa[2], ob[XPW], oc, oe;
  int wave;
  char *junk;

  HQ_DEV Relaxed(const Job &J, int row0, int tok0, int M, int w, char *junk_area) : wave(w), junk(junk_area) {
    const int lane = threadIdx.x & 63, ng = J.n >> 5;
    const int64_t rb = (int64_t)ng * GB;
    rw = resource(J.wq + row0 * rb, (J.r1 - row0) * rb);
    rws = resource(J.ws + (int64_t)row0 * ng * 4, (int64_t)(J.r1 - row0) * ng * 4);
    rwc = resource(J.wc + (int64_t)row0 * ng * 4, WC ? (int64_t)(J.r1 - row0) * ng * 4 : 0);
    rx = resource(J.xq + tok0 * J.frame, (M - 1 - tok0) * J.frame + J.n);
    rxs = resource(J.xs + tok0 * J.sframe, (M - 1 - tok0) * J.sframe + 4 * ng);
    // loads a0, a1: 1 KB pieces 2 w and 2 w + 1 of the stage's weights.  int8: piece c is rows 8 c .. + 7, lane l
    // row 8 c + l / 8, slot l % 8 holding chunk (l % 8) ^ swz(row); int6: 16-byte piece 64 c + l of 128 rows x 96
    // bytes (pieces 0..11)
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int c = 2 * w + i;
      if (PACK == 8) {
        const int row = 8 * c + (lane >> 3), ch = (lane & 7) ^ swz(row);
        oa[i] = (uint32_t)(row * rb + (ch >> 1) * 32 + (ch & 1) * 16);
      } else {
        const int q = 64 * c + lane;
        oa[i] = (uint32_t)((q / 6) * rb + (q % 6) * 16);
      }
    }
    // load b: the activations of tokens 8 c .. + 7 (pieces c = XPW w ..), as the weights
#pragma unroll
    for (int i = 0; i < XPW; i++) {
      const int tok = 8 * (XPW * w + i) + (lane >> 3), ch = (lane & 7) ^ swz(tok);
      ob[i] = (uint32_t)(tok * J.frame + (ch >> 1) * 32 + (ch & 1) * 16);
    }
    // loads c, d: the rows' scales and corrections of group w / SPG, rows 64 (w % SPG) + l
    oc = (uint32_t)(((64 * (w % SPG) + lane) * ng + w / SPG) * 4);
    // load e: waves 0..3 the tokens' scales of group w, the tokens of each 32-token half reordered (entry 16 h + 4 i
    // + m is token 8 m + 4 h + i), so that one 16-byte read gives a lane the four tokens of its 4 x 4 outer products
    {
      const int q = lane & 31;
      const int tok = 32 * (lane >> 5) + 8 * (q & 3) + 4 * (q >> 4) + ((q >> 2) & 3);
      oe = (uint32_t)(tok * J.sframe + (w & 3) * 4);
    }
  }

  // the q_loads of stage s (groups 4 s .. 4 s + 3) into S
  HQ_DEV void load(StageQ<BRT> &S, int s) {
    const int w = wave;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      if (PACK == 8 || 2 * w + i < 12 * BRT / 128) dma16(rw, S.w + (2 * w + i) * 1024, oa[i], s * QG * GB);
      else dma16(rxs, junk, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < XPW; i++) dma16(rx, S.x + (XPW * w + i) * 1024, ob[i], s * QG * 32);
    dma4(rws, &S.ws[w / SPG][64 * (w % SPG)], oc, s * QG * 4);
    if (WC) dma4(rwc, &S.wc[w / SPG][64 * (w % SPG)], oc, s * QG * 4);
    else dma4(rxs, junk, 0, 0);
    if (w < 4) dma4(rxs, &S.xs[w][0], oe, s * QG * 4);
    else dma4(rxs, junk, 0, 0);
  }
};

// group gi of stage S into the chain of the lane's four sub-tiles (slices 2 pair, 2 pair + 1 x both token halves,
// acc[2 slice + half]): the exact integers (MFMA, from the corrections) and the scales' products (outer-product
// MFMAs), each term f(f(C) * f(ws * xs)) (relaxed/int8.ts:26-39).  MFMA A = activations (m = token), B = weights
// (n = row): lane l holds row l % 32 of its slice and tokens 8 (r / 4) + 4 (l / 32) + r % 4 of its half, so a lane's
// correction and row scale are one value each.
template <int PACK, bool WC, int BRT>
HQ_DEV void q_group(float acc[4][16], const StageQ<BRT> &S, int gi, int pair, int lane) {
  const int kh = lane >> 5, l32 = lane & 31;
  v4i X[2];
  float xv[2][4];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int t = l32 + 32 * h;
    X[h] = *(const v4i *)(S.x + t * 128 + ((2 * gi + kh) ^ swz(t)) * 16);
    // the scales of tokens 8 m + 4 kh + lane % 4 (m = 0..3) of the half
    const float4 v = *(const float4 *)&S.xs[gi][32 * h + 16 * kh + 4 * (lane & 3)];
    xv[h][0] = v.x; xv[h][1] = v.y; xv[h][2] = v.z; xv[h][3] = v.w;
  }
#pragma unroll
  for (int sp = 0; sp < 2; sp++) {
    const int row = 64 * pair + 32 * sp + l32;
    v4i W;
    if (PACK == 8) W = *(const v4i *)(S.w + row * 128 + ((2 * gi + kh) ^ swz(row)) * 16);
    else W = six_half(S.w + row * 96 + gi * 24, kh);
    v16i cin;
    if (WC) {  // the caller's correction of the lane's row
      const int32_t c = S.wc[gi][row];
#pragma unroll
      for (int r = 0; r < 16; r++) cin[r] = c;
    } else {  // -64 sum(w) of the row: 32 bytes of -64 against the weights
      const v4i m64 = {(int32_t)0xc0c0c0c0, (int32_t)0xc0c0c0c0, (int32_t)0xc0c0c0c0, (int32_t)0xc0c0c0c0};
      cin = __builtin_amdgcn_mfma_i32_32x32x32_i8(m64, W, zero16i(), 0, 0, 0);
    }
    const float wsv = S.ws[gi][row];
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(X[h], W, cin, 0, 0, 0);
      // f(xs * ws) of the sub-tile: v_mfma_f32_4x4x1_16b_f32 gives lane l, register i the product of lane
      // 4 (l / 4) + i's A and lane l's B, so A = the scale of token 8 m + 4 kh + lane % 4 and B = the row's scale
      // give registers 4 m .. 4 m + 3 the tokens 8 m + 4 kh + i of the i8 MFMA's layout, one product each
      v16f sc;
#pragma unroll
      for (int m = 0; m < 4; m++) {
        const v4f d = __builtin_amdgcn_mfma_f32_4x4x1f32(xv[h][m], wsv, zero4f(), 0, 0, 0);
        sc[4 * m] = d[0]; sc[4 * m + 1] = d[1]; sc[4 * m + 2] = d[2]; sc[4 * m + 3] = d[3];
      }
      float *a = acc[2 * sp + h];
#pragma unroll
      for (int r = 0; r < 16; r++) a[r] = fadd(a[r], fmul((float)c[r], sc[r]));
    }
  }
}

// stage s in `cur`, the loads of stage s + AHEAD into `next` (the buffer of stage s - 1)
template <int PACK, bool WC, int BRT>
HQ_DEV void q_step(Relaxed<PACK, WC, BRT> &L, const StageQ<BRT> &cur, StageQ<BRT> &next, int s, int stages,
                   int total, float acc[4][16], int pair, int chain, int lane) {
  if (s >= stages) return;
  wait_for<q_loads<BRT>()>(s, total);
  if (s + AHEAD < total) L.load(next, s + AHEAD);
  q_group<PACK, WC, BRT>(acc, cur, chain, pair, lane);  // group 4 s + chain
}

// the 4 chains of a pair of slices added in LDS, ((a0 + a1) + a2) + a3, for its four sub-tiles: wave k adds its sums
// to what waves 0..k-1 left (the values of a lane are the same (row, token)s in the four waves of a pair); the sums
// end in chain 3's waves.  p0 (sub-tiles 0, 1) and p1 (2, 3): 2 x 64 x 32 floats each that nothing else uses
HQ_DEV void add_chains4(float acc[4][16], float *p0, float *p1, int pair, int chain, int lane) {
  float *q[2] = {p0 + (pair * 64 + lane) * 32, p1 + (pair * 64 + lane) * 32};
  for (int k = 0; k < 4; k++) {
    __syncthreads();
    if (chain == k) {
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          float *m = q[i >> 1] + 16 * (i & 1) + r;
          if (k > 0) acc[i][r] = fadd(*m, acc[i][r]);
          if (k < 3) *m = acc[i][r];
        }
    }
  }
}

template <int PACK, bool WC, int BRT>
__global__ __launch_bounds__(q_threads<BRT>()) void gemm_relaxed(Job J) {
  __shared__ StageQ<BRT> b0, b1, b2, b3;
  __shared__ __attribute__((aligned(16))) char junk[1024];
  const int M = J.count;
  const int ng = J.n >> 5, ng4 = ng & ~3;
  int rb, tb;
  tile_of(blockIdx.x, gridDim.x, (J.r1 - J.r0 + BRT - 1) / BRT, rb, tb);
  const int row0 = J.r0 + rb * BRT, tok0 = tb * BT;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int pair = wave >> 2, chain = wave & 3;

  float acc[4][16];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[i][r] = 0.0f;

  Relaxed<PACK, WC, BRT> L(J, row0, tok0, M, wave, junk);
  const int stages = ng4 / QG;
  const int total = stages + (ng4 < ng ? 1 : 0);  // stages loaded: the tail's groups are one more
  if (total > 0) L.load(b0, 0);
  if (total > 1) L.load(b1, 1);
  if (total > 2) L.load(b2, 2);
  for (int s = 0; s < stages; s += RING) {
    q_step<PACK, WC, BRT>(L, b0, b3, s, stages, total, acc, pair, chain, lane);
    q_step<PACK, WC, BRT>(L, b1, b0, s + 1, stages, total, acc, pair, chain, lane);
    q_step<PACK, WC, BRT>(L, b2, b1, s + 2, stages, total, acc, pair, chain, lane);
    q_step<PACK, WC, BRT>(L, b3, b2, s + 3, stages, total, acc, pair, chain, lane);
  }
  stage_ready<0>();  // every load has landed (the tail's too) and every wave is done with the stages
  auto ring = [&](int i) -> StageQ<BRT> & { return i == 0 ? b0 : i == 1 ? b1 : i == 2 ? b2 : b3; };
  add_chains4(acc, (float *)&ring((stages + 1) % RING), (float *)&ring((stages + 2) % RING), pair, chain, lane);
  if (chain == 3) {
    // the groups past the fours, one at a time, after the four chains' sum (relaxed/int8.ts:40-47)
    const StageQ<BRT> &T = ring(stages % RING);
    for (int gi = 0; gi < ng - ng4; gi++) q_group<PACK, WC, BRT>(acc, T, gi, pair, lane);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = row0 + 64 * pair + 32 * (i >> 1) + (lane & 31);
      if (row < J.r1) {
        const int tbase = tok0 + 32 * (i & 1) + 4 * (lane >> 5);
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int t = tbase + 8 * q + e;
            if (t < M) ((float *)(J.out + t * J.os))[row] = acc[i][4 * q + e];
          }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// ternary (matmul_t2r_tile)
// MFMA A = activations (m = token), B = codes (n = row): lane l holds row l % 32 of its slice and tokens
// 8 (r / 4) + 4 (l / 32) + r % 4 of its half.  Part k of a group of 128 (block h = k / 2, bytes c = 8 (k % 2) .. + 7
// of it) as 32 K values in the order plane-major: K half kh of a lane is planes 2 kh, 2 kh + 1, eight c's each, for
// the codes and for interleave()'s activation bytes 64 h + 16 p + 8 (k % 2) .. + 7 alike.
// ---------------------------------------------------------------------------------------------------------------
constexpr int TG = 2;       // groups of 128 a stage
constexpr int NT = 1024;    // threads a block: 16 waves, 4 slices of 32 rows x 4 parts
constexpr int TLOADS = 3;   // loads a wave a stage

struct alignas(16) StageT {
  char w[BR * 64];           // 128 rows x 2 groups x 32 code bytes; 16-byte chunk j of row r at j ^ tswz(r)
  char x[BT * 256];          // 64 tokens x 2 groups x 128 activation bytes; chunk c of token t at c ^ (t & 15)
  float xs[TG * 4][BT];      // the tokens' scales of each (group, part)
  int32_t sums[TG * 4][BT];  // and their sums
  uint32_t d[TG][BR];        // the rows' float16 group scales, one a word
};

HQ_DEV int tswz(int r) { return (r >> 2) & 3; }
// binary: a row's two 16-byte groups of a stage, swapped on every other 8 rows
HQ_DEV int bswz(int r) { return (r >> 3) & 1; }

// a block's loads of ternary (binary: BIN) stages: wave w's three loads a stage and their offsets
template <bool BIN>
struct Ternary {
  __amdgpu_buffer_rsrc_t rw, rx, rxs, rws;
  uint32_t oa, ob, oc;
  int wave;
  char *junk;

  HQ_DEV Ternary(const Job &J, int row0, int tok0, int M, int w, char *junk_area) : wave(w), junk(junk_area) {
    const int lane = threadIdx.x & 63, groups = J.n >> 7;
    const int nsc = 4 * (J.n >> 5);  // the bytes of a token's scales: its sums follow them
    constexpr int GB = BIN ? 16 : 32;  // bytes of a group's codes
    rw = resource(J.wq + (int64_t)row0 * groups * GB, (int64_t)(J.r1 - row0) * groups * GB);
    rws = resource(J.ws + (int64_t)row0 * groups * 2, (int64_t)(J.r1 - row0) * groups * 2);
    rx = resource(J.xq + tok0 * J.frame, (M - 1 - tok0) * J.frame + J.n);
    rxs = resource(J.xs + tok0 * J.sframe, (M - 1 - tok0) * J.sframe + 2 * nsc);
    // load a: the activations, tokens 4 w .. + 3, lane l token 4 w + l / 16, slot l % 16 holding chunk
    // (l % 16) ^ (token & 15) of the stage's 256 bytes
    {
      const int tok = 4 * w + (lane >> 4), c = (lane & 15) ^ (tok & 15);
      oa = (uint32_t)(tok * J.frame + c * 16);
    }
    // load b: waves 0..7 the codes (rows 16 w .. + 15, lane l row 16 w + l / 4, slot l % 4 holding chunk
    // (l % 4) ^ tswz(row) of the row's 64 bytes; binary: waves 0..3, rows 32 w .. + 31, lane l row 32 w + l / 2,
    // slot l % 2 holding group (l % 2) ^ bswz(row) of the row's 32 bytes, waves 4..7 into the scratch area); waves
    // 8..15 the tokens' scales of (group, part) w - 8
    if (w < 8 && BIN) {
      const int row = 32 * (w & 3) + (lane >> 1), j = (lane & 1) ^ bswz(row);
      ob = (uint32_t)(row * groups * 16 + j * 16);
    } else if (w < 8) {
      const int row = 16 * w + (lane >> 2), j = (lane & 3) ^ tswz(row);
      ob = (uint32_t)(row * groups * 32 + (j >> 1) * 32 + (j & 1) * 16);
    } else {
      ob = (uint32_t)(lane * J.sframe + (w - 8) * 4);
    }
    // load c: waves 0..7 the sums of (group, part) w; waves 8..11 the float16 scales (group (w - 8) / 2, rows
    // 64 ((w - 8) % 2) + l)
    if (w < 8) {
      oc = (uint32_t)(lane * J.sframe + nsc + w * 4);
    } else {
      const int i = w - 8;
      oc = (uint32_t)(((64 * (i & 1) + lane) * groups + (i >> 1)) * 2);
    }
  }

  HQ_DEV void load(StageT &S, int s) {
    const int w = wave;
    dma16(rx, S.x + w * 1024, oa, s * TG * 128);
    if (w < 8 && (!BIN || w < 4)) dma16(rw, S.w + w * 1024, ob, s * TG * (BIN ? 16 : 32));
    else if (w < 8) dma16(rxs, junk, 0, 0);
    else dma4(rxs, &S.xs[w - 8][0], ob, s * TG * 16);
    if (w < 8) dma4(rxs, &S.sums[w][0], oc, s * TG * 16);
    else if (w < 12) dma2(rws, &S.d[(w - 8) >> 1][64 * ((w - 8) & 1)], oc, s * TG * 2);
    else dma4(rxs, junk, 0, 0);
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

// 8 bytes at byte o (a multiple of 8) of a token's 256 stage bytes
HQ_DEV uint2 t_acts8(const StageT &S, int tok, int o) {
  return *(const uint2 *)(S.x + tok * 256 + (((o >> 4) ^ (tok & 15)) << 4) + (o & 8));
}

// binary's planes 2 kh, 2 kh + 1 of block h (bits 4 h + 2 kh and + 1 of every byte, doubled: kernels/binary.ts:19-22)
HQ_DEV v4i bit_pair(uint32_t w0, uint32_t w1, int b) {
  v4i r;
  r[0] = (int32_t)(((w0 >> b) & 0x01010101u) << 1);
  r[1] = (int32_t)(((w1 >> b) & 0x01010101u) << 1);
  r[2] = (int32_t)(((w0 >> (b + 1)) & 0x01010101u) << 1);
  r[3] = (int32_t)(((w1 >> (b + 1)) & 0x01010101u) << 1);
  return r;
}

// part k of group gi of the stage for the lane's slice, both token halves: f(f(whole * xs) * d) into the part's
// chain (relaxed/signs.ts:31)
template <bool BIN>
HQ_DEV void t_group(float acc0[16], float acc1[16], const StageT &S, int gi, int k, int slice, int lane) {
  const int h = k >> 1, s = k & 1, kh = lane >> 5, row = 32 * slice + (lane & 31);
  // B: the row's codes of planes 2 kh, 2 kh + 1, bytes c = 8 s .. + 7 of block h (ternary: chunk 2 gi + h, half s;
  // binary: group gi's 16 bytes, half s, bits 4 h + 2 kh ..)
  v4i B;
  if (BIN) {
    const uint2 wv = *(const uint2 *)(S.w + row * 32 + ((gi ^ bswz(row)) << 4) + 8 * s);
    B = bit_pair(wv.x, wv.y, 4 * h + 2 * kh);
  } else {
    const int j = 2 * gi + h;
    const uint2 wv = *(const uint2 *)(S.w + row * 64 + ((j ^ tswz(row)) << 4) + 8 * s);
    B = kh == 0 ? plane_pair<0>(wv.x, wv.y) : plane_pair<2>(wv.x, wv.y);
  }
  const float d = half_to_float(S.d[gi][row]);
  const int o = 128 * gi + 64 * h + 8 * s + 32 * kh;
#pragma unroll
  for (int half = 0; half < 2; half++) {
    const int tok = 32 * half + (lane & 31);
    const uint2 a0 = t_acts8(S, tok, o), a1 = t_acts8(S, tok, o + 16);
    v4i A;
    A[0] = (int32_t)a0.x; A[1] = (int32_t)a0.y; A[2] = (int32_t)a1.x; A[3] = (int32_t)a1.y;
    const int tbase = 32 * half + 4 * kh;
    v16i C;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int4 c4 = *(const int4 *)&S.sums[4 * gi + k][tbase + 8 * q];
      C[4 * q] = c4.x; C[4 * q + 1] = c4.y; C[4 * q + 2] = c4.z; C[4 * q + 3] = c4.w;
    }
    C = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, C, 0, 0, 0);
    float *acc = half ? acc1 : acc0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const float4 x4 = *(const float4 *)&S.xs[4 * gi + k][tbase + 8 * q];
      const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
      for (int e = 0; e < 4; e++) acc[4 * q + e] = fadd(acc[4 * q + e], fmul(fmul((float)C[4 * q + e], xv[e]), d));
    }
  }
}

template <bool BIN>
HQ_DEV void t_step(Ternary<BIN> &L, const StageT &cur, StageT &next, int s, int stages, int groups, float acc0[16],
                   float acc1[16], int slice, int part, int lane) {
  if (s >= stages) return;
  wait_for<TLOADS>(s, stages);
  if (s + AHEAD < stages) L.load(next, s + AHEAD);
  // part `part` of groups 2 s and 2 s + 1 (relaxed/signs.ts:28-31)
  t_group<BIN>(acc0, acc1, cur, 0, part, slice, lane);
  if (TG * s + 1 < groups) t_group<BIN>(acc0, acc1, cur, 1, part, slice, lane);
}

template <bool BIN>
__global__ __launch_bounds__(NT) void gemm_ternary(Job J) {
  __shared__ StageT b0, b1, b2, b3;
  __shared__ __attribute__((aligned(16))) char junk[1024];
  const int M = J.count;
  const int groups = J.n >> 7;
  int rb, tb;
  tile_of(blockIdx.x, gridDim.x, (J.r1 - J.r0 + BR - 1) / BR, rb, tb);
  const int row0 = J.r0 + rb * BR, tok0 = tb * BT;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int slice = wave >> 2, part = wave & 3;

  float acc0[16], acc1[16];
#pragma unroll
  for (int r = 0; r < 16; r++) acc0[r] = acc1[r] = 0.0f;

  Ternary<BIN> L(J, row0, tok0, M, wave, junk);
  const int stages = (groups + TG - 1) / TG;
  if (stages > 0) L.load(b0, 0);
  if (stages > 1) L.load(b1, 1);
  if (stages > 2) L.load(b2, 2);
  for (int s = 0; s < stages; s += RING) {
    t_step<BIN>(L, b0, b3, s, stages, groups, acc0, acc1, slice, part, lane);
    t_step<BIN>(L, b1, b0, s + 1, stages, groups, acc0, acc1, slice, part, lane);
    t_step<BIN>(L, b2, b1, s + 2, stages, groups, acc0, acc1, slice, part, lane);
    t_step<BIN>(L, b3, b2, s + 3, stages, groups, acc0, acc1, slice, part, lane);
  }
  stage_ready<0>();
  add_chains(acc0, acc1, (float *)&b0, (float *)&b1, slice, part, lane);
  if (part == 3) {
    const int rw = row0 + 32 * slice + (lane & 31);
    if (rw < J.r1) {
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int tbase = tok0 + 32 * h + 4 * (lane >> 5);
        const float *acc = h ? acc1 : acc0;
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
}

}  // namespace

bool gemm_supported(Kind kind) { return kind == Q8R || kind == Q6R || signs_kind(kind); }

hipError_t launch_gemm(Kind kind, const Job &job, hipStream_t s) {
  const int rows = job.r1 - job.r0;
  if (rows <= 0 || job.count <= 0) return hipSuccess;
  const int token_tiles = (job.count + BT - 1) / BT;
  dim3 grid(((rows + BR - 1) / BR) * token_tiles), block(NT);
  const bool wc = job.wc != nullptr;
  // int8 / int6: 64-row tiles where 128-row ones would leave fewer than two blocks a compute unit
  const bool narrow = (int64_t)((rows + BR - 1) / BR) * token_tiles < 2 * (int64_t)cu_count();
  const dim3 grid64(((rows + 63) / 64) * token_tiles), block64(q_threads<64>()), block128(q_threads<128>());
  switch (kind) {
  case Q8R:
    if (narrow) {
      if (wc) hipLaunchKernelGGL((gemm_relaxed<8, true, 64>), grid64, block64, 0, s, job);
      else hipLaunchKernelGGL((gemm_relaxed<8, false, 64>), grid64, block64, 0, s, job);
    } else {
      if (wc) hipLaunchKernelGGL((gemm_relaxed<8, true, 128>), grid, block128, 0, s, job);
      else hipLaunchKernelGGL((gemm_relaxed<8, false, 128>), grid, block128, 0, s, job);
    }
    break;
  case Q6R:
    if (narrow) {
      if (wc) hipLaunchKernelGGL((gemm_relaxed<6, true, 64>), grid64, block64, 0, s, job);
      else hipLaunchKernelGGL((gemm_relaxed<6, false, 64>), grid64, block64, 0, s, job);
    } else {
      if (wc) hipLaunchKernelGGL((gemm_relaxed<6, true, 128>), grid, block128, 0, s, job);
      else hipLaunchKernelGGL((gemm_relaxed<6, false, 128>), grid, block128, 0, s, job);
    }
    break;
  case T2R:
  case T2: hipLaunchKernelGGL(gemm_ternary<false>, grid, block, 0, s, job); break;
  case B1R:
  case B1: hipLaunchKernelGGL(gemm_ternary<true>, grid, block, 0, s, job); break;
  default: return hipErrorNotSupported;
  }
  return hipGetLastError();
}

}  // namespace hq
