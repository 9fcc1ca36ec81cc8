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
// (relaxed/int8.ts:40-47).  Here a wave IS a lane k of the reference: the 4 waves of one slice of the tile take
// chain k = 0..3 each, adding their groups / parts in order into registers, and at the end add their sums through LDS
// in that order.  Each term is f(f(C) * f(ws * xs)) (int8, int6) or f(f(f(C) * xs) * d) (ternary), rounded as the
// reference rounds it (-ffp-contract=off).
//
// The scales' product of int8 / int6, f(ws * xs) for every (row, token), is an outer product on the matrix core: one
// v_mfma_f32_32x32x1_2b_f32 (two 32 x 32 blocks, K = 1) gives a 32-row slice's products with both 32-token halves,
// each rounded once as v_mul_f32 rounds it (subnormals, zeros, infinities and NaN included), in the same lane layout
// as the integer MFMA's result.
//
// Roofline.  The dense int8 MFMA peak is 5.0 POPS (32 cycles a v_mfma_i32_32x32x32_i8, 32768 MACs, a SIMD), but the
// bit-exact epilogue is 3 VALU operations per (row, token, group): convert, multiply, add (ternary 4), which this
// build issues unpacked (packed float32 instructions are off).  Measured on MI355X: two or more waves a SIMD issue a
// wave's VALU instruction every ~2.2 cycles (one wave alone every ~4.4), and a SIMD whose VALU is busy that way does
// not run MFMAs beside it, so a 32 x 32 sub-tile's group costs ~48 x 2.2 cycles of VALU plus 32 (integer MFMA) + 32
// (half a 32x32x1_2b) + 16 (half a correction MFMA) of the matrix core: ~185 cycles for 65536 operations, about a
// third of the int8 peak (0.83 POPS at 2.3 GHz) — the bound this kernel is measured against.
//
// Tiles.  int8 / int6: a block (4 waves, two blocks a CU) computes a 64-row x 64-token tile; wave w is chain w, four
// 32 x 32 sub-tiles (two row slices x two token halves: the weights' operand read once for two MFMAs, the tokens' for
// two slices).  Launches whose 64-row tiles would leave block slots idle take 32-row tiles (one slice, ~150 VGPRs,
// a ring of 3 stage buffers: three blocks a CU).  Ternary: a block of 16 waves computes a 128-row x 64-token tile
// (12 waves and 96 rows for launches whose 128-row tiles would end in a part-empty round); wave w takes rows
// 32 (w / 4) .. + 31 and chain w % 4, both 32-token halves.
//
// Pipeline (int8 / int6).  A wave issues each sub-tile's MFMAs one sub-tile ahead of its epilogue, so the matrix core
// works on the next sub-tile while the VALU folds this one.  The operands go from HBM / L2 straight into LDS with
// buffer-to-LDS loads into a ring of 4 stage buffers (3 for 32-row tiles; a stage: 4 groups of int8 / int6, 2 groups
// of 128 of ternary): at the barrier for stage s, which says that stage s's loads have landed and that every wave has
// read stage s - 1's operands, a wave reads its operands of stage s and issues its loads of stage s + 3 (s + 2) into
// stage s - 1's buffer.  A
// wave issues the same loads every stage, so one s_waitcnt vmcnt count says "my loads of stage s have landed".  A load
// past the tile's last row or token, or past the last group, reads zeros (buffer bounds; such results are never
// stored).  The 16-byte chunks of a row are stored XOR-swizzled so that the MFMA operand reads (32 rows or tokens, one
// chunk each) spread over the LDS banks, and tiles are ordered so that the blocks one XCD runs at a time share rows
// and tokens in that XCD's L2.
#include "common.hpp"
#include "launch.hpp"
#include "stage.hpp"

namespace hq {

namespace {

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int BT = 64;           // a tile's tokens
constexpr int RING = 4;           // stage buffers
constexpr int AHEAD = RING - 1;   // stages loaded beyond the one computed
// the int8 / int6 tiles' rings: 4 buffers for 64-row tiles (76 KB, two blocks a CU), 3 for 32-row tiles (45 KB,
// three blocks a CU: more waves a SIMD against one stage less in flight, measured 2-4 % faster than 4 buffers and two
// blocks)
template <int R> constexpr int ring_of() { return R == 32 ? 3 : 4; }

HQ_DEV v16i zero16i() {
  v16i z;
#pragma unroll
  for (int r = 0; r < 16; r++) z[r] = 0;
  return z;
}
HQ_DEV v32f zero32f() {
  v32f z;
#pragma unroll
  for (int r = 0; r < 32; r++) z[r] = 0.0f;
  return z;
}

// the 4 chains of a slice added in LDS, ((a0 + a1) + a2) + a3, for both token halves: wave k adds its sums to what
// waves 0..k-1 left (the 16 values of a lane are the same (row, token)s in the four waves of a slice); the sums end
// in chain 3's waves.  p0, p1: 4 x 16 x 64 floats each that nothing else uses meanwhile, value r of a lane at
// [r][lane] (consecutive lanes, consecutive banks)
HQ_DEV void add_chains(float acc0[16], float acc1[16], float *p0, float *p1, int slice, int chain, int lane) {
  float *q0 = p0 + slice * 16 * 64 + lane, *q1 = p1 + slice * 16 * 64 + lane;
  for (int k = 0; k < 4; k++) {
    __syncthreads();
    if (chain == k) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        if (k > 0) {
          acc0[r] = fadd(q0[r * 64], acc0[r]);
          acc1[r] = fadd(q1[r * 64], acc1[r]);
        }
        if (k < 3) {
          q0[r * 64] = acc0[r];
          q1[r * 64] = acc1[r];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// int8 / int6 weights, relaxed activations (matmul_q8r_tile, matmul_q6r)
// MFMA A = activations (m = token), B = weights (n = row): lane l holds row l % 32 of its slice and tokens
// 8 (r / 4) + 4 (l / 32) + r % 4 of its half (register r = 0..15); K half l / 32 is bytes 16 (l / 32) .. + 15 of the
// group.  The scales' outer product takes A = the scale of token l of the tile and B = the scale of row l % 32 of the
// slice: its register r (r + 16) is the same (token, row) of the first (second) token half.
// ---------------------------------------------------------------------------------------------------------------
constexpr int QG = 4;   // groups a stage
constexpr int QT = 256; // threads a block: 4 waves, one chain each

// A stage of a tile of R rows (64: two row slices x two token halves a wave; 32: one slice x two halves, for launches
// of few tiles).  The rows' scales have room for 64 rows whatever R is: a wide scale load fills 64.
template <int R>
struct alignas(16) StageQ {
  char w[R * 128];     // int8: R rows x 4 groups x 32 bytes, chunks swizzled; int6: R rows x 4 x 24 bytes
  char x[BT * 128];    // 64 tokens x 4 groups x 32 bytes, chunks swizzled
  float ws[64][QG];    // the rows' scales of the stage's groups
  int32_t wc[64][QG];  // the rows' corrections (with the caller's wc)
  float xs[BT][QG];    // the tokens' scales
};

// A stage's scales are 16 contiguous bytes of a row (or token).  Where every such run is 16-byte aligned (WIDE: the
// group count a multiple of 4 and the bases and token stride 16-byte aligned) one lane loads a row's 16 bytes, 64
// rows a load; otherwise four lanes load a row's four scales, 16 rows a load, group g of row r stored at
// g ^ gswz(r) so that 32 rows 16 bytes apart reading one group hit 32 different banks.  Loads into LDS cost about
// the same whatever their width, so the wide form's fewer loads are what count.
HQ_DEV int gswz(int r) { return (r >> 3) & 3; }
template <bool WIDE> HQ_DEV int sslot(int r, int g) { return WIDE ? g : g ^ gswz(r); }

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

// A block's loads of a stage, as 1 KB pieces (256 B for the narrow scale loads) dealt to the four waves in turn:
// the weights' pieces (8 of int8, 6 of int6 a 64-row tile; half as many for 32 rows), the activations' (8), then the
// scales' (wide: the rows', the corrections' with wc, the tokens'; narrow: R / 16 of the rows' kinds, 4 of the
// tokens').  Wave W issues pieces W, W + 4, ..., so its loads a stage
// are count(W); no load is issued that is not needed.  W is a template argument (the kernel runs one copy of its
// main loop a wave), so a wave's loads are straight-line code: chosen at run time, every stage took a tree of
// scalar branches per piece (measured 4-6 % of the launch).
template <int PACK, bool WC, bool WIDE, int W, int R>
struct Relaxed {
  static constexpr int GB = PACK == 8 ? 32 : 24;           // bytes of a group of weights
  static constexpr int NWP = (PACK == 8 ? 8 : 6) * R / 64;  // the weights' pieces
  static constexpr int NRK = WC ? 2 : 1;                   // kinds of the rows' scale pieces: ws, (wc)
  static constexpr int SPR = WIDE ? 1 : R / 16;            // pieces of each
  static constexpr int SPT = WIDE ? 1 : 4;                 // pieces of the tokens' scales
  static constexpr int P = NWP + 8 + NRK * SPR + SPT;      // pieces a stage
  static constexpr int PW = (P + 3) / 4;            // the most pieces of a wave
  static constexpr int count = P / 4 + (W < P % 4 ? 1 : 0);  // this wave's
  static constexpr int wave = W;
  __amdgpu_buffer_rsrc_t rw, rx, rws, rwc, rxs;
  uint32_t off[PW];

  HQ_DEV Relaxed(const Job &J, int row0, int tok0, int M) {
    constexpr int w = W;
    const int lane = threadIdx.x & 63, ng = J.n >> 5;
    const int64_t rb = (int64_t)ng * GB;
    rw = resource(J.wq + row0 * rb, (J.r1 - row0) * rb);
    rws = resource(J.ws + (int64_t)row0 * ng * 4, (int64_t)(J.r1 - row0) * ng * 4);
    rwc = resource(J.wc + (int64_t)row0 * ng * 4, WC ? (int64_t)(J.r1 - row0) * ng * 4 : 0);
    rx = resource(J.xq + tok0 * J.frame, (M - 1 - tok0) * J.frame + J.n);
    rxs = resource(J.xs + tok0 * J.sframe, (M - 1 - tok0) * J.sframe + 4 * ng);
#pragma unroll
    for (int k = 0; k < PW; k++) {
      const int p = w + 4 * k;
      uint32_t o = 0;
      if (p < NWP) {
        // int8: rows 8 p .. + 7, lane l row 8 p + l / 8, slot l % 8 holding chunk (l % 8) ^ swz(row); int6: 16-byte
        // piece 64 p + l of 64 rows x 96 bytes
        if (PACK == 8) {
          const int row = 8 * p + (lane >> 3), ch = (lane & 7) ^ swz(row);
          o = (uint32_t)(row * rb + (ch >> 1) * 32 + (ch & 1) * 16);
        } else {
          const int q = 64 * p + lane;
          o = (uint32_t)((q / 6) * rb + (q % 6) * 16);
        }
      } else if (p < NWP + 8) {
        // the activations of tokens 8 c .. + 7, as the weights
        const int c = p - NWP, tok = 8 * c + (lane >> 3), ch = (lane & 7) ^ swz(tok);
        o = (uint32_t)(tok * J.frame + (ch >> 1) * 32 + (ch & 1) * 16);
      } else if (p < P) {
        const int q = p - NWP - 8;  // ws pieces, then wc's, then xs's
        const bool tokens = q >= NRK * SPR;
        const int i = tokens ? q - NRK * SPR : q % SPR;
        if (WIDE) {  // lane l: row (or token) l, its 16 bytes
          o = tokens ? (uint32_t)(lane * J.sframe) : (uint32_t)(lane * ng * 4);
        } else {     // lane l: row 16 i + l / 4, group (l % 4) ^ gswz(row)
          const int r = 16 * i + (lane >> 2), g = (lane & 3) ^ gswz(r);
          o = tokens ? (uint32_t)(r * J.sframe + g * 4) : (uint32_t)((r * ng + g) * 4);
        }
      }
      off[k] = o;
    }
  }

  // wave w's loads of stage s (groups 4 s .. 4 s + 3) into S
  HQ_DEV void load(StageQ<R> &S, int s) {
#pragma unroll
    for (int k = 0; k < PW; k++) {
      const int p = wave + 4 * k;
      if (p < NWP) {
        dma16(rw, S.w + p * 1024, off[k], s * QG * GB);
      } else if (p < NWP + 8) {
        dma16(rx, S.x + (p - NWP) * 1024, off[k], s * QG * 32);
      } else if (p < P) {
        const int q = p - NWP - 8;
        const bool tokens = q >= NRK * SPR;
        const int i = tokens ? q - NRK * SPR : q % SPR;
        // a branch for each resource: a resource chosen by a select is a per-lane value to the compiler, which then
        // loops over its lanes (v_readfirstlane) around every load (measured 28 % of the launch with wc)
        if (tokens) {
          if (WIDE) dma16(rxs, &S.xs[16 * i][0], off[k], s * QG * 4);
          else dma4(rxs, &S.xs[16 * i][0], off[k], s * QG * 4);
        } else if (q < SPR) {
          if (WIDE) dma16(rws, &S.ws[16 * i][0], off[k], s * QG * 4);
          else dma4(rws, &S.ws[16 * i][0], off[k], s * QG * 4);
        } else {
          if (WIDE) dma16(rwc, &S.wc[16 * i][0], off[k], s * QG * 4);
          else dma4(rwc, &S.wc[16 * i][0], off[k], s * QG * 4);
        }
      }
    }
  }
};

// stage s's loads have landed everywhere: this wave's own, with those of the stages after it still in flight (two
// with a ring of 4 buffers, one with 3), then the block's barrier
template <int PACK, bool WC, bool WIDE, int W, int R>
HQ_DEV void q_ready() {
  stage_ready<(ring_of<R>() - 2) * Relaxed<PACK, WC, WIDE, W, R>::count>();
}

// a wave's operands of one group gi of a stage: the activations of both token halves, the weights of both row slices
// (int6 widened to int8), the scale of token `lane` and of the slices' rows, the slices' corrections (with wc)
struct OpsQ {
  v4i X[2], W[2];
  float xs, ws[2];
  int32_t wc[2];
};

// The main loop's reads of a stage's operands are one block of ds_read instructions and one wait for them.  Read as
// C++ loads, the compiler would also wait for every buffer-to-LDS load still in flight before them (it cannot tell
// that those write other stage buffers once more than a few are in flight), which would leave the loads no time to
// land ahead of their stage; here the stage barrier alone says when a buffer is ready.
template <int PACK, bool WC>
HQ_DEV void ds_ops(OpsQ &o, uint2 six[2][3], const uint32_t ax[2], const uint32_t aw[2], uint32_t axs,
                   const uint32_t aws[2], const uint32_t awc[2]) {
  if (PACK == 8 && WC) {
    asm volatile(
        "ds_read_b128 %0, %9\n\tds_read_b128 %1, %10\n\tds_read_b128 %2, %11\n\tds_read_b128 %3, %12\n\t"
        "ds_read_b32 %4, %13\n\tds_read_b32 %5, %14\n\tds_read_b32 %6, %15\n\tds_read_b32 %7, %16\n\t"
        "ds_read_b32 %8, %17\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(o.X[0]), "=&v"(o.X[1]), "=&v"(o.W[0]), "=&v"(o.W[1]), "=&v"(o.xs), "=&v"(o.ws[0]), "=&v"(o.ws[1]),
          "=&v"(o.wc[0]), "=&v"(o.wc[1])
        : "v"(ax[0]), "v"(ax[1]), "v"(aw[0]), "v"(aw[1]), "v"(axs), "v"(aws[0]), "v"(aws[1]), "v"(awc[0]),
          "v"(awc[1])
        : "memory");
  } else if (PACK == 8) {
    asm volatile(
        "ds_read_b128 %0, %7\n\tds_read_b128 %1, %8\n\tds_read_b128 %2, %9\n\tds_read_b128 %3, %10\n\t"
        "ds_read_b32 %4, %11\n\tds_read_b32 %5, %12\n\tds_read_b32 %6, %13\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(o.X[0]), "=&v"(o.X[1]), "=&v"(o.W[0]), "=&v"(o.W[1]), "=&v"(o.xs), "=&v"(o.ws[0]), "=&v"(o.ws[1])
        : "v"(ax[0]), "v"(ax[1]), "v"(aw[0]), "v"(aw[1]), "v"(axs), "v"(aws[0]), "v"(aws[1])
        : "memory");
    o.wc[0] = o.wc[1] = 0;
  } else {
    // int6: a slice's group is three 8-byte pieces (the low nibbles, then the top bits) at aw, + 8, + 16
    asm volatile(
        "ds_read_b128 %0, %11\n\tds_read_b128 %1, %12\n\t"
        "ds_read_b64 %2, %13\n\tds_read_b64 %3, %13 offset:8\n\tds_read_b64 %4, %13 offset:16\n\t"
        "ds_read_b64 %5, %14\n\tds_read_b64 %6, %14 offset:8\n\tds_read_b64 %7, %14 offset:16\n\t"
        "ds_read_b32 %8, %15\n\tds_read_b32 %9, %16\n\tds_read_b32 %10, %17\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(o.X[0]), "=&v"(o.X[1]), "=&v"(six[0][0]), "=&v"(six[0][1]), "=&v"(six[0][2]), "=&v"(six[1][0]),
          "=&v"(six[1][1]), "=&v"(six[1][2]), "=&v"(o.xs), "=&v"(o.ws[0]), "=&v"(o.ws[1])
        : "v"(ax[0]), "v"(ax[1]), "v"(aw[0]), "v"(aw[1]), "v"(axs), "v"(aws[0]), "v"(aws[1])
        : "memory");
    if (WC) {
      asm volatile("ds_read_b32 %0, %2\n\tds_read_b32 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                   : "=&v"(o.wc[0]), "=&v"(o.wc[1]) : "v"(awc[0]), "v"(awc[1]) : "memory");
    } else {
      o.wc[0] = o.wc[1] = 0;
    }
  }
}

// K half kh of an int6 group from its three 8-byte pieces (six_half's arithmetic on registers)
HQ_DEV v4i six_regs(const uint2 p[3], int kh) {
  const uint32_t lo[4] = {p[0].x, p[0].y, p[1].x, p[1].y};
  const uint32_t top[2] = {p[2].x, p[2].y};
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

// a wave's operands of group gi of stage S (ds_ops' reads; a 32-row tile's second slice reads the first's again)
template <int PACK, bool WC, bool WIDE, int R>
HQ_DEV OpsQ read_ops(const StageQ<R> &S, int gi, int lane) {
  OpsQ o;
  uint2 six[2][3];
  const int kh = lane >> 5, l32 = lane & 31;
  uint32_t ax[2], aw[2], aws[2], awc[2];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int t = l32 + 32 * h;
    ax[h] = lds_addr(S.x + t * 128 + ((2 * gi + kh) ^ swz(t)) * 16);
  }
#pragma unroll
  for (int sp = 0; sp < 2; sp++) {
    const int row = (R == 64 ? 32 * sp : 0) + l32;
    aw[sp] = PACK == 8 ? lds_addr(S.w + row * 128 + ((2 * gi + kh) ^ swz(row)) * 16) : lds_addr(S.w + row * 96 + gi * 24);
    aws[sp] = lds_addr(&S.ws[row][sslot<WIDE>(row, gi)]);
    awc[sp] = lds_addr(&S.wc[row][sslot<WIDE>(row, gi)]);
  }
  ds_ops<PACK, WC>(o, six, ax, aw, lds_addr(&S.xs[lane][sslot<WIDE>(lane, gi)]), aws, awc);
  if (PACK == 6) {
    o.W[0] = six_regs(six[0], kh);
    if (R == 64) o.W[1] = six_regs(six[1], kh);
  }
  return o;
}

// the same from C++ loads (outside the main loop, where no load into LDS is in flight)
template <int PACK, bool WC, bool WIDE, int R>
HQ_DEV OpsQ read_ops_plain(const StageQ<R> &S, int gi, int lane) {
  OpsQ o;
  const int kh = lane >> 5, l32 = lane & 31;
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int t = l32 + 32 * h;
    o.X[h] = *(const v4i *)(S.x + t * 128 + ((2 * gi + kh) ^ swz(t)) * 16);
  }
#pragma unroll
  for (int sp = 0; sp < R / 32; sp++) {
    const int row = 32 * sp + l32;
    if (PACK == 8) o.W[sp] = *(const v4i *)(S.w + row * 128 + ((2 * gi + kh) ^ swz(row)) * 16);
    else o.W[sp] = six_half(S.w + row * 96 + gi * 24, kh);
    o.ws[sp] = S.ws[row][sslot<WIDE>(row, gi)];
    o.wc[sp] = WC ? S.wc[row][sslot<WIDE>(row, gi)] : 0;
  }
  o.xs = S.xs[lane][sslot<WIDE>(lane, gi)];
  return o;
}

// the accumulator input of slice sp's integer MFMAs: the caller's correction of the lane's row (the same for every
// token), or -64 sum(w) of the row (32 bytes of -64 against the weights)
template <bool WC>
HQ_DEV v16i corrections(const OpsQ &o, int sp) {
  if (WC) {
    v16i c;
#pragma unroll
    for (int r = 0; r < 16; r++) c[r] = o.wc[sp];
    return c;
  }
  const v4i m64 = {(int32_t)0xc0c0c0c0, (int32_t)0xc0c0c0c0, (int32_t)0xc0c0c0c0, (int32_t)0xc0c0c0c0};
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(m64, o.W[sp], zero16i(), 0, 0, 0);
}
HQ_DEV v16i integers(const OpsQ &o, int sp, int h, const v16i &cin) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(o.X[h], o.W[sp], cin, 0, 0, 0);
}
// f(xs * ws) of slice sp with both token halves (registers 0..15: the first half, 16..31: the second)
HQ_DEV v32f scales(const OpsQ &o, int sp) { return __builtin_amdgcn_mfma_f32_32x32x1f32(o.xs, o.ws[sp], zero32f(), 0, 0, 0); }

// the chain's term of one sub-tile, f(f(C) * f(ws * xs)) added in order (relaxed/int8.ts:26-39)
HQ_DEV void fold(float a[16], const v16i &c, const v32f &sc, int h) {
#pragma unroll
  for (int r = 0; r < 16; r++) a[r] = fadd(a[r], fmul((float)c[r], sc[16 * h + r]));
}

// Stage s of wave W's chain (group 4 s + W): the stage's loads landed everywhere (the block's barrier), the
// wave's operands read from `cur`, its loads of stage s + 3 (s + 2 with 3 buffers) issued into `dma` (the buffer
// stage s - 1's operands came from, which every wave has read by this barrier), then the four sub-tiles (slice, half)
// = (0, 0), (0, 1), (1, 0), (1, 1) (a 32-row tile: the first two), each sub-tile's MFMAs issued before the previous
// one's fold so that the matrix core and the VALU take turns without waiting for each other.  Every wave has issued
// its loads of stages up to s + 2 (s + 1) at the barrier (a stage past the job's last group loads zeros, and its
// buffer is never read), so "stage s landed" is always "at most two stages (one) of this wave's loads in flight".
template <int PACK, bool WC, bool WIDE, int W, int R>
HQ_DEV void q_stage(Relaxed<PACK, WC, WIDE, W, R> &L, const StageQ<R> &cur, StageQ<R> &dma, int s, float acc[4][16],
                    int lane) {
  q_ready<PACK, WC, WIDE, W, R>();
  const OpsQ op = read_ops<PACK, WC, WIDE, R>(cur, W, lane);
  L.load(dma, s + ring_of<R>() - 1);
  const v16i cin0 = corrections<WC>(op, 0);
  const v32f S0 = scales(op, 0);
  const v16i C0 = integers(op, 0, 0, cin0);
  const v16i C1 = integers(op, 0, 1, cin0);
  if (R == 32) {
    fold(acc[0], C0, S0, 0);
    fold(acc[1], C1, S0, 1);
    return;
  }
  const v16i cin1 = corrections<WC>(op, 1);
  fold(acc[0], C0, S0, 0);
  const v32f S1 = scales(op, 1);
  const v16i C2 = integers(op, 1, 0, cin1);
  fold(acc[1], C1, S0, 1);
  const v16i C3 = integers(op, 1, 1, cin1);
  fold(acc[2], C2, S1, 0);
  fold(acc[3], C3, S1, 1);
}

// the 4 chains of the tile added in LDS, ((a0 + a1) + a2) + a3, for its four sub-tiles: wave k adds its sums to
// what waves 0..k-1 left (the values of a lane are the same (row, token)s in the four waves); the sums end in chain
// 3's wave.  p0 (sub-tiles 0, 1) and p1 (2, 3): 32 x 64 floats each that nothing else uses, value v of a lane at
// [v][lane] (consecutive lanes, consecutive banks).  NS: the sub-tiles, 4 (64-row tiles) or 2 (32 rows)
template <int NS>
HQ_DEV void add_chains4(float acc[4][16], float *p0, float *p1, int chain, int lane) {
  float *q[2] = {p0 + lane, p1 + lane};
  for (int k = 0; k < 4; k++) {
    __syncthreads();
    if (chain == k) {
#pragma unroll
      for (int i = 0; i < NS; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          float *m = q[i >> 1] + (16 * (i & 1) + r) * 64;
          if (k > 0) acc[i][r] = fadd(*m, acc[i][r]);
          if (k < 3) *m = acc[i][r];
        }
    }
  }
}

// A 64-row tile's end: the chains' sums ((a0 + a1) + a2) + a3 made by the four waves at once, each storing a quarter
// of the tile.  In two halves (sub-tiles 0, 1, then 2, 3) every wave writes the half's 32 values of a lane as 8
// float4s ([quad][lane], wave w's at p[w / 2] + 8 KB (w % 2)), and after the barrier wave q adds the quads 2 q and
// 2 q + 1 of the four waves in chain order, then the terms of the groups past the fours one at a time (from the tail
// stage T: each wave makes them for its own sub-tile of the half, the integer and scale MFMAs of its slice and token
// half), and stores them.  (Measured against a chain-at-a-time add through four barriers with one wave storing the
// tile: 1-3 % of a launch.)
template <int PACK, bool WC, bool WIDE>
HQ_DEV void finish_tile(const float acc[4][16], float *p0, float *p1, const StageQ<64> &T, int tail, int chain,
                        int lane, const Job &J, int row0, int tok0) {
  float *const part[4] = {p0, p0 + 2048, p1, p1 + 2048};
  const int th = chain >> 1, r0 = 8 * (chain & 1);  // this wave's sub-tile of a half (its token half), its values
#pragma unroll
  for (int half = 0; half < 2; half++) {
    __syncthreads();
#pragma unroll
    for (int vq = 0; vq < 8; vq++) {
      const float *a = acc[2 * half + (vq >> 2)] + 4 * (vq & 3);
      *(float4 *)(part[chain] + (vq * 64 + lane) * 4) = make_float4(a[0], a[1], a[2], a[3]);
    }
    __syncthreads();
    // the groups past the fours: f(f(C) * f(ws * xs)) of values r0 .. r0 + 7 of sub-tile (slice half, token half th)
    float tt[QG - 1][8];
#pragma unroll
    for (int gi = 0; gi < QG - 1; gi++) {
      if (gi >= tail) break;
      const OpsQ o = read_ops_plain<PACK, WC, WIDE, 64>(T, gi, lane);
      const v16i C = integers(o, half, th, corrections<WC>(o, half));
      const v32f sc = scales(o, half);
#pragma unroll
      for (int m = 0; m < 8; m++) tt[gi][m] = fmul((float)C[r0 + m], sc[16 * th + r0 + m]);
    }
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const int vq = 2 * chain + k;
      float4 c[4];
#pragma unroll
      for (int w = 0; w < 4; w++) c[w] = *(const float4 *)(part[w] + (vq * 64 + lane) * 4);
      float v[4] = {fadd(fadd(fadd(c[0].x, c[1].x), c[2].x), c[3].x), fadd(fadd(fadd(c[0].y, c[1].y), c[2].y), c[3].y),
                    fadd(fadd(fadd(c[0].z, c[1].z), c[2].z), c[3].z), fadd(fadd(fadd(c[0].w, c[1].w), c[2].w), c[3].w)};
#pragma unroll
      for (int gi = 0; gi < QG - 1; gi++) {
        if (gi >= tail) break;
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] = fadd(v[e], tt[gi][4 * k + e]);
      }
      // value r = r0 + 4 k + e of sub-tile 2 half + th: row 32 half + lane % 32, token 32 th + 8 (r / 4) + 4 (lane / 32)
      // + e
      const int row = row0 + 32 * half + (lane & 31);
      if (row < J.r1) {
        const int tbase = tok0 + 32 * th + 2 * r0 + 8 * k + 4 * (lane >> 5);
#pragma unroll
        for (int e = 0; e < 4; e++)
          if (tbase + e < J.count) ((float *)(J.out + (tbase + e) * J.os))[row] = v[e];
      }
    }
  }
}

// the tile's end in wave `chain` (every load landed, the chains added, the groups past the fours, the stores); in the
// wave's own copy of the main loop's function, so that its accumulators pass to it where they are
template <int PACK, bool WC, bool WIDE, int R>
HQ_DEV void q_end(const Job &J, int row0, int tok0, int M, int stages, StageQ<R> &b0, StageQ<R> &b1, StageQ<R> &b2,
                  StageQ<R> &b3, float acc[4][16], int chain, int lane) {
  const int ng = J.n >> 5, ng4 = ng & ~3;
  stage_ready<0>();  // every load has landed (the tail's too) and every wave is done with the stages
  auto ring = [&](int i) -> StageQ<R> & { return i == 0 ? b0 : i == 1 ? b1 : i == 2 ? b2 : b3; };
  constexpr int RING = ring_of<R>();
  if constexpr (R == 64) {
    finish_tile<PACK, WC, WIDE>(acc, (float *)&ring((stages + 1) % RING), (float *)&ring((stages + 2) % RING),
                                ring(stages % RING), ng - ng4, chain, lane, J, row0, tok0);
    return;
  }
  // a 32-row tile: the chains added one after the other through LDS, chain 3 storing the tile
  add_chains4<R / 16>(acc, (float *)&ring((stages + 1) % RING), (float *)&ring((stages + 2) % RING), chain, lane);
  if (chain == 3) {
    // the groups past the fours, one at a time, after the four chains' sum (relaxed/int8.ts:40-47)
    const StageQ<R> &T = ring(stages % RING);
#pragma unroll
    for (int gi = 0; gi < QG - 1; gi++) {
      if (gi >= ng - ng4) break;
      const OpsQ o = read_ops_plain<PACK, WC, WIDE, R>(T, gi, lane);
#pragma unroll
      for (int sp = 0; sp < R / 32; sp++) {
        const v16i cin = corrections<WC>(o, sp);
        const v32f sc = scales(o, sp);
#pragma unroll
        for (int h = 0; h < 2; h++) fold(acc[2 * sp + h], integers(o, sp, h, cin), sc, h);
      }
    }
#pragma unroll
    for (int i = 0; i < R / 16; i++) {
      const int row = row0 + 32 * (i >> 1) + (lane & 31);
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

// wave W's stages of the tile (chain W): its loads, every stage in order, then the tile's end
template <int PACK, bool WC, bool WIDE, int W, int R>
HQ_DEV void q_chain(const Job &J, int row0, int tok0, int M, int stages, StageQ<R> &b0, StageQ<R> &b1,
                    StageQ<R> &b2, StageQ<R> &b3, float acc[4][16], int lane) {
  Relaxed<PACK, WC, WIDE, W, R> L(J, row0, tok0, M);
  // stages 0..2 first (0..1 with 3 buffers; whatever the job has: a stage past its groups loads zeros); stage s's
  // operands come from buffer s % 4 (s % 3) and its loads of stage s + 3 (s + 2) go into buffer s - 1's
  L.load(b0, 0);
  L.load(b1, 1);
  if constexpr (ring_of<R>() == 3) {
    for (int s = 0; s < stages; s += 3) {
      q_stage<PACK, WC, WIDE, W, R>(L, b0, b2, s, acc, lane);
      if (s + 1 >= stages) break;
      q_stage<PACK, WC, WIDE, W, R>(L, b1, b0, s + 1, acc, lane);
      if (s + 2 >= stages) break;
      q_stage<PACK, WC, WIDE, W, R>(L, b2, b1, s + 2, acc, lane);
    }
    q_end<PACK, WC, WIDE, R>(J, row0, tok0, M, stages, b0, b1, b2, b2, acc, W, lane);
    return;
  }
  L.load(b2, 2);
  for (int s = 0; s < stages; s += RING) {
    q_stage<PACK, WC, WIDE, W, R>(L, b0, b3, s, acc, lane);
    if (s + 1 >= stages) break;
    q_stage<PACK, WC, WIDE, W, R>(L, b1, b0, s + 1, acc, lane);
    if (s + 2 >= stages) break;
    q_stage<PACK, WC, WIDE, W, R>(L, b2, b1, s + 2, acc, lane);
    if (s + 3 >= stages) break;
    q_stage<PACK, WC, WIDE, W, R>(L, b3, b2, s + 3, acc, lane);
  }
  q_end<PACK, WC, WIDE, R>(J, row0, tok0, M, stages, b0, b1, b2, b3, acc, W, lane);
}

template <int PACK, bool WC, bool WIDE, int R>
__global__ __launch_bounds__(QT, ring_of<R>() == 3 ? 3 : 2) void gemm_relaxed(Job J) {
  __shared__ StageQ<R> b0, b1, b2;
  __shared__ StageQ<R> b3x[1];  // not allocated for a ring of 3 (never used then)
  StageQ<R> &b3 = ring_of<R>() == 3 ? b2 : b3x[0];
  const int M = J.count;
  int rb, tb;
  tile_of(blockIdx.x, gridDim.x, (J.r1 - J.r0 + R - 1) / R, rb, tb);
  const int row0 = J.r0 + rb * R, tok0 = tb * BT;
  const int lane = threadIdx.x & 63;
  const int chain = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  float acc[4][16];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[i][r] = 0.0f;

  const int stages = (J.n >> 5) / QG;  // whole stages of the four chains; the groups past them are one more stage
  switch (chain) {
  case 0: q_chain<PACK, WC, WIDE, 0, R>(J, row0, tok0, M, stages, b0, b1, b2, b3, acc, lane); break;
  case 1: q_chain<PACK, WC, WIDE, 1, R>(J, row0, tok0, M, stages, b0, b1, b2, b3, acc, lane); break;
  case 2: q_chain<PACK, WC, WIDE, 2, R>(J, row0, tok0, M, stages, b0, b1, b2, b3, acc, lane); break;
  default: q_chain<PACK, WC, WIDE, 3, R>(J, row0, tok0, M, stages, b0, b1, b2, b3, acc, lane); break;
  }
}

// ---------------------------------------------------------------------------------------------------------------
// ternary (matmul_t2r_tile)
// MFMA A = activations (m = token), B = codes (n = row): lane l holds row l % 32 of its slice and tokens
// 8 (r / 4) + 4 (l / 32) + r % 4 of its half.  Part k of a group of 128 (block h = k / 2, bytes c = 8 (k % 2) .. + 7
// of it) as 32 K values in the order plane-major: K half kh of a lane is planes 2 kh, 2 kh + 1, eight c's each, for
// the codes and for interleave()'s activation bytes 64 h + 16 p + 8 (k % 2) .. + 7 alike.
// A tile is R rows (128, or 96 for launches whose 128-row tiles would end in a part-empty round) x 64 tokens, a block
// of R / 32 slices x 4 parts = 4 R / 32 waves, one block a CU.
// ---------------------------------------------------------------------------------------------------------------
constexpr int TG = 2;  // groups of 128 a stage

template <int R>
struct alignas(16) StageT {
  char w[R * 64];            // R rows x 2 groups x 32 code bytes; 16-byte chunk j of row r at j ^ tswz(r) (binary: R
                             // rows x 2 x 16, group j of row r at j ^ bswz(r))
  char x[BT * 256];          // 64 tokens x 2 groups x 128 activation bytes; chunk c of token t at c ^ (t & 15)
  float xs[TG * 4][BT];      // the tokens' scales of each (group, part)
  int32_t sums[TG * 4][BT];  // and their sums
  uint32_t d[TG][128];       // the rows' float16 group scales, one a word (96-row tiles: rows 96..127 loaded, unread)
};

HQ_DEV int tswz(int r) { return (r >> 2) & 3; }
// binary: a row's two 16-byte groups of a stage, swapped on every other 8 rows
HQ_DEV int bswz(int r) { return (r >> 3) & 1; }

// A block's loads of a stage, as pieces dealt to the waves in turn (wave w takes pieces w, w + NW, ...): 16 pieces of
// the activations (tokens 4 p .. + 3, 1 KB each), the codes (16 rows a piece; binary 32), the tokens' scales and sums
// of each (group, part) (256 bytes each), the rows' scales (64 rows a piece, 2 bytes a row).  Every wave issues PW
// loads a stage (a load past the pieces reads 1 KB into a junk area), so one wait count serves every wave.
template <bool BIN, int R>
struct Ternary {
  static constexpr int NW = 4 * (R / 32);                   // waves
  static constexpr int NC = BIN ? R / 32 : R / 16;          // code pieces
  static constexpr int ND = (R + 63) / 64;                  // row-scale pieces a group
  static constexpr int P = 16 + NC + 16 + TG * ND;          // pieces a stage
  static constexpr int PW = (P + NW - 1) / NW;              // loads a wave a stage
  __amdgpu_buffer_rsrc_t rw, rx, rxs, rws;
  uint32_t off[PW];
  int wave;
  char *junk;

  HQ_DEV Ternary(const Job &J, int row0, int tok0, int M, int w, char *junk_area) : wave(w), junk(junk_area) {
    const int lane = threadIdx.x & 63, groups = J.n >> 7;
    const int nsc = 4 * (J.n >> 5);
    constexpr int GB = BIN ? 16 : 32;
    rw = resource(J.wq + (int64_t)row0 * groups * GB, (int64_t)(J.r1 - row0) * groups * GB);
    rws = resource(J.ws + (int64_t)row0 * groups * 2, (int64_t)(J.r1 - row0) * groups * 2);
    rx = resource(J.xq + tok0 * J.frame, (M - 1 - tok0) * J.frame + J.n);
    rxs = resource(J.xs + tok0 * J.sframe, (M - 1 - tok0) * J.sframe + 2 * nsc);
#pragma unroll
    for (int k = 0; k < PW; k++) {
      const int p = w + NW * k;
      uint32_t o = 0;
      if (p < 16) {
        const int tok = 4 * p + (lane >> 4), c = (lane & 15) ^ (tok & 15);
        o = (uint32_t)(tok * J.frame + c * 16);
      } else if (p < 16 + NC) {
        const int q = p - 16;
        if (BIN) {
          const int row = 32 * q + (lane >> 1), j = (lane & 1) ^ bswz(row);
          o = (uint32_t)(row * groups * 16 + j * 16);
        } else {
          const int row = 16 * q + (lane >> 2), j = (lane & 3) ^ tswz(row);
          o = (uint32_t)(row * groups * 32 + (j >> 1) * 32 + (j & 1) * 16);
        }
      } else if (p < 24 + NC) {
        o = (uint32_t)(lane * J.sframe + (p - 16 - NC) * 4);
      } else if (p < 32 + NC) {
        o = (uint32_t)(lane * J.sframe + nsc + (p - 24 - NC) * 4);
      } else if (p < P) {
        const int q = p - 32 - NC, g = q / ND, i = q % ND;
        o = (uint32_t)(((64 * i + lane) * groups + g) * 2);
      }
      off[k] = o;
    }
  }

  // (the stage buffer's address made opaque, so that the compiler forms each load's LDS destination here instead of
  // holding every buffer's destinations in scalar registers across the main loop)
  HQ_DEV void load(StageT<R> &S, int s) {
    uint32_t base = lds_addr(&S);
    asm volatile("" : "+s"(base));
    const auto at = [&](size_t o) { return (void *)(uintptr_t)(base + (uint32_t)o); };
#pragma unroll
    for (int k = 0; k < PW; k++) {
      const int p = wave + NW * k;
      if (p < 16) dma16(rx, at(offsetof(StageT<R>, x) + p * 1024), off[k], s * TG * 128);
      else if (p < 16 + NC) dma16(rw, at(offsetof(StageT<R>, w) + (p - 16) * 1024), off[k], s * TG * (BIN ? 16 : 32));
      else if (p < 24 + NC) dma4(rxs, at(offsetof(StageT<R>, xs) + (p - 16 - NC) * 4 * BT), off[k], s * TG * 16);
      else if (p < 32 + NC) dma4(rxs, at(offsetof(StageT<R>, sums) + (p - 24 - NC) * 4 * BT), off[k], s * TG * 16);
      else if (p < P) {
        const int q = p - 32 - NC;
        dma2(rws, at(offsetof(StageT<R>, d) + ((q / ND) * 128 + 64 * (q % ND)) * 4), off[k], s * TG * 2);
      } else dma16(rxs, junk, 0, 0);
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
// chain (relaxed/signs.ts:31).  The stage's operands are read by blocks of ds_reads with one wait each: read as C++
// loads, each would first wait for every buffer-to-LDS load in flight, the next stages' included (the compiler cannot
// tell that those write other stage buffers), and no stage's loads would overlap the stages before it.  The codes'
// address and the others are byte offsets added to the stage buffer's address, made opaque to the compiler so that it
// adds them here rather than keeping every stage buffer's addresses in registers.
template <bool BIN, int R>
HQ_DEV void t_group(float acc0[16], float acc1[16], const StageT<R> &S, int gi, int k, int slice, int lane) {
  const int h = k >> 1, s = k & 1, kh = lane >> 5, row = 32 * slice + (lane & 31);
  const int o = 128 * gi + 64 * h + 8 * s + 32 * kh;
  uint32_t base = lds_addr(&S);
  asm volatile("" : "+s"(base));
  const uint32_t aw = base + (BIN ? (uint32_t)(offsetof(StageT<R>, w) + row * 32 + ((gi ^ bswz(row)) << 4) + 8 * s)
                                  : (uint32_t)(offsetof(StageT<R>, w) + row * 64 + (((2 * gi + h) ^ tswz(row)) << 4) + 8 * s));
  const uint32_t ad = base + (uint32_t)(offsetof(StageT<R>, d) + (gi * 128 + row) * 4);
  uint32_t aa[2][2];
#pragma unroll
  for (int half = 0; half < 2; half++) {
    const int tok = 32 * half + (lane & 31);
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int oi = o + 16 * i;
      aa[half][i] = base + (uint32_t)(offsetof(StageT<R>, x) + tok * 256 + (((oi >> 4) ^ (tok & 15)) << 4) + (oi & 8));
    }
  }
  const uint32_t asum = base + (uint32_t)(offsetof(StageT<R>, sums) + ((4 * gi + k) * BT + 4 * kh) * 4);
  const uint32_t axs = base + (uint32_t)(offsetof(StageT<R>, xs) + ((4 * gi + k) * BT + 4 * kh) * 4);
  uint2 wv, a0, a1;
  uint32_t dh;
  v4i c[4];
  asm volatile(
      "ds_read_b64 %0, %8\n\tds_read_b32 %1, %9\n\tds_read_b64 %2, %10\n\tds_read_b64 %3, %11\n\t"
      "ds_read_b128 %4, %12\n\tds_read_b128 %5, %12 offset:32\n\tds_read_b128 %6, %12 offset:64\n\t"
      "ds_read_b128 %7, %12 offset:96\n\ts_waitcnt lgkmcnt(0)"
      : "=&v"(wv), "=&v"(dh), "=&v"(a0), "=&v"(a1), "=&v"(c[0]), "=&v"(c[1]), "=&v"(c[2]), "=&v"(c[3])
      : "v"(aw), "v"(ad), "v"(aa[0][0]), "v"(aa[0][1]), "v"(asum)
      : "memory");
  v4i B;
  if (BIN) B = bit_pair(wv.x, wv.y, 4 * h + 2 * kh);
  else B = kh == 0 ? plane_pair<0>(wv.x, wv.y) : plane_pair<2>(wv.x, wv.y);
  const float d = half_to_float(dh);
  const auto product = [&](const uint2 &p0, const uint2 &p1, const v4i cq[4]) {
    v4i A;
    A[0] = (int32_t)p0.x; A[1] = (int32_t)p0.y; A[2] = (int32_t)p1.x; A[3] = (int32_t)p1.y;
    v16i cin;
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
      for (int e = 0; e < 4; e++) cin[4 * q + e] = cq[q][e];
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, cin, 0, 0, 0);
  };
  const v16i C0 = product(a0, a1, c);
  v4f x[4];
  asm volatile(
      "ds_read_b64 %0, %10\n\tds_read_b64 %1, %11\n\t"
      "ds_read_b128 %2, %12 offset:128\n\tds_read_b128 %3, %12 offset:160\n\tds_read_b128 %4, %12 offset:192\n\t"
      "ds_read_b128 %5, %12 offset:224\n\tds_read_b128 %6, %13\n\tds_read_b128 %7, %13 offset:32\n\t"
      "ds_read_b128 %8, %13 offset:64\n\tds_read_b128 %9, %13 offset:96\n\ts_waitcnt lgkmcnt(0)"
      : "=&v"(a0), "=&v"(a1), "=&v"(c[0]), "=&v"(c[1]), "=&v"(c[2]), "=&v"(c[3]), "=&v"(x[0]), "=&v"(x[1]),
        "=&v"(x[2]), "=&v"(x[3])
      : "v"(aa[1][0]), "v"(aa[1][1]), "v"(asum), "v"(axs)
      : "memory");
  const v16i C1 = product(a0, a1, c);
#pragma unroll
  for (int q = 0; q < 4; q++)
#pragma unroll
    for (int e = 0; e < 4; e++) acc0[4 * q + e] = fadd(acc0[4 * q + e], fmul(fmul((float)C0[4 * q + e], x[q][e]), d));
  asm volatile(
      "ds_read_b128 %0, %4 offset:128\n\tds_read_b128 %1, %4 offset:160\n\tds_read_b128 %2, %4 offset:192\n\t"
      "ds_read_b128 %3, %4 offset:224\n\ts_waitcnt lgkmcnt(0)"
      : "=&v"(x[0]), "=&v"(x[1]), "=&v"(x[2]), "=&v"(x[3])
      : "v"(axs)
      : "memory");
#pragma unroll
  for (int q = 0; q < 4; q++)
#pragma unroll
    for (int e = 0; e < 4; e++) acc1[4 * q + e] = fadd(acc1[4 * q + e], fmul(fmul((float)C1[4 * q + e], x[q][e]), d));
}

// stage s of the tile: its loads landed everywhere (two stages after it still in flight), the loads of stage s + 3
// issued into the buffer stage s - 1 was read from, then part `part` of groups 2 s and 2 s + 1 (relaxed/signs.ts:28-31)
template <bool BIN, int R>
HQ_DEV void t_step(Ternary<BIN, R> &L, const StageT<R> &cur, StageT<R> &next, int s, int stages, int groups,
                    float acc0[16], float acc1[16], int slice, int part, int lane) {
  if (s >= stages) return;
  wait_for<Ternary<BIN, R>::PW>(s, stages, AHEAD - 1);
  if (s + AHEAD < stages) L.load(next, s + AHEAD);
  t_group<BIN, R>(acc0, acc1, cur, 0, part, slice, lane);
  if (TG * s + 1 < groups) t_group<BIN, R>(acc0, acc1, cur, 1, part, slice, lane);
}

// the tile's stages, the four parts' chains added in order ((p0 + p1) + p2) + p3 (math.ts:7-9), part 3's waves storing
template <bool BIN, int R>
__global__ __launch_bounds__(64 * 4 * (R / 32)) void gemm_ternary(Job J) {
  __shared__ StageT<R> b0, b1, b2, b3;
  __shared__ __attribute__((aligned(16))) char junk[1024];
  const int M = J.count;
  const int groups = J.n >> 7;
  int rb, tb;
  tile_of(blockIdx.x, gridDim.x, (J.r1 - J.r0 + R - 1) / R, rb, tb);
  const int row0 = J.r0 + rb * R, tok0 = tb * BT;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int slice = wave >> 2, part = wave & 3;
  float acc0[16], acc1[16];
#pragma unroll
  for (int r = 0; r < 16; r++) acc0[r] = acc1[r] = 0.0f;
  Ternary<BIN, R> L(J, row0, tok0, M, wave, junk);
  const int stages = (groups + TG - 1) / TG;
  if (stages > 0) L.load(b0, 0);
  if (stages > 1) L.load(b1, 1);
  if (stages > 2) L.load(b2, 2);
  for (int s = 0; s < stages; s += RING) {
    t_step<BIN, R>(L, b0, b3, s, stages, groups, acc0, acc1, slice, part, lane);
    t_step<BIN, R>(L, b1, b0, s + 1, stages, groups, acc0, acc1, slice, part, lane);
    t_step<BIN, R>(L, b2, b1, s + 2, stages, groups, acc0, acc1, slice, part, lane);
    t_step<BIN, R>(L, b3, b2, s + 3, stages, groups, acc0, acc1, slice, part, lane);
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

// The ternary tile's rows for a launch: 96 where that costs less, a launch costing its rounds of tiles over the CUs
// (one block a CU) times the tile's rows times its cost a row (a 96-row tile of 12 waves does 1.155 times the 128-row
// tile's time a row, measured over launches of many rounds: 348 against 402 TOPS).  27B at M = 256: gate/up 544
// tiles of 128 rows (3 rounds, the last an eighth full) against 728 of 96 (3 rounds), 276 -> 331 TOPS; down 160 of
// 128 (96 CUs idle) against 216 of 96, 276 -> 329; at M = 1024 both keep 128 rows.
int ternary_rows(int rows, int token_tiles) {
  const int64_t cus = cu_count();
  const int64_t r128 = ((int64_t)((rows + 127) / 128) * token_tiles + cus - 1) / cus;
  const int64_t r96 = ((int64_t)((rows + 95) / 96) * token_tiles + cus - 1) / cus;
  return 96.0 * 1.155 * (double)r96 < 128.0 * (double)r128 ? 96 : 128;
}

// int8 / int6: the wide scale loads where a stage's four scales of every row and token are 16-byte aligned runs
bool wide_scales(const Job &j) {
  const auto a16 = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
  return (j.n >> 5) % 4 == 0 && a16(j.ws) && (j.wc == nullptr || a16(j.wc)) && a16(j.xs) &&
         (j.count <= 1 || j.sframe % 16 == 0);
}

template <bool BIN, int R>
void launch_ternary(const Job &job, int token_tiles, hipStream_t s) {
  const dim3 grid(((job.r1 - job.r0 + R - 1) / R) * token_tiles);
  hipLaunchKernelGGL((gemm_ternary<BIN, R>), grid, dim3(8 * R), 0, s, job);
}

template <int PACK, int R>
void launch_relaxed(const Job &job, int token_tiles, hipStream_t s) {
  const dim3 grid(((job.r1 - job.r0 + R - 1) / R) * token_tiles);
  const bool wc = job.wc != nullptr, wide = wide_scales(job);
  if (wc && wide) hipLaunchKernelGGL((gemm_relaxed<PACK, true, true, R>), grid, dim3(QT), 0, s, job);
  else if (wc) hipLaunchKernelGGL((gemm_relaxed<PACK, true, false, R>), grid, dim3(QT), 0, s, job);
  else if (wide) hipLaunchKernelGGL((gemm_relaxed<PACK, false, true, R>), grid, dim3(QT), 0, s, job);
  else hipLaunchKernelGGL((gemm_relaxed<PACK, false, false, R>), grid, dim3(QT), 0, s, job);
}

// 32-row tiles (three blocks a CU) where they cost less than 64-row tiles (two a CU): a launch costs its tiles over
// the CUs' block slots in rounds (at least one, however few its tiles), a round of 32-row tiles kTile32 of one of
// 64-row tiles (measured over launches of many rounds: 426 against 508 TOPS at 14336 x 2 x 4096, M = 2048, so a
// round of 3 x 32-row tiles a CU costs 0.89 of one of 2 x 64-row tiles).  Against nine prompt shapes measured both
// ways (the 8B layer at M = 2048, Llama-3.2-1B at 512, the 27B projections at 256) it picks the faster height each
// time: 64 for the 8B shapes, the 1B gate/up and the 27B gate/up, 32 for the other 1B shapes and the 27B down.
constexpr double kTile32 = 0.89;
bool short_tiles(int rows, int token_tiles) {
  const double cus = (double)cu_count();
  const double t64 = (double)((rows + 63) / 64) * token_tiles, t32 = (double)((rows + 31) / 32) * token_tiles;
  return kTile32 * fmax(1.0, t32 / (3 * cus)) < fmax(1.0, t64 / (2 * cus));
}

}  // namespace

bool gemm_supported(Kind kind) { return kind == Q8R || kind == Q6R || signs_kind(kind); }

hipError_t launch_gemm(Kind kind, const Job &job, hipStream_t s) {
  const int rows = job.r1 - job.r0;
  if (rows <= 0 || job.count <= 0) return hipSuccess;
  const int token_tiles = (job.count + BT - 1) / BT;
  switch (kind) {
  case Q8R:
    if (short_tiles(rows, token_tiles)) launch_relaxed<8, 32>(job, token_tiles, s);
    else launch_relaxed<8, 64>(job, token_tiles, s);
    break;
  case Q6R:
    if (short_tiles(rows, token_tiles)) launch_relaxed<6, 32>(job, token_tiles, s);
    else launch_relaxed<6, 64>(job, token_tiles, s);
    break;
  case T2R:
  case T2:
    if (ternary_rows(rows, token_tiles) == 96) launch_ternary<false, 96>(job, token_tiles, s);
    else launch_ternary<false, 128>(job, token_tiles, s);
    break;
  case B1R:
  case B1:
    if (ternary_rows(rows, token_tiles) == 96) launch_ternary<true, 96>(job, token_tiles, s);
    else launch_ternary<true, 128>(job, token_tiles, s);
    break;
  default: return hipErrorNotSupported;
  }
  return hipGetLastError();
}

}  // namespace hq
