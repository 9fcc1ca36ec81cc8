// gemm_tol.hip — the prompt tile of relaxed int8 weights (matmul_q8r_tile's products, kernels/relaxed/int8.ts:52-166)
// to the north star's float32 tolerance instead of to the bit: every group's integer exact, the groups added in
// another float32 order.
//
// What it computes: y[t][r] = sum over groups g, in order, of f(ws[r][g] xs[t][g]) * d_g[r][t], each term one fused
// multiply-add into a float32 accumulator, with d_g = sum_k w[r][k] (q[t][k] - 64) the reference's exact group
// integer with int8_sums' corrections (relaxed/int8.ts:26-37, kernel/matmul.ts:50-58; relaxed activation bytes are
// taken as signed int8, as the bit-exact kernels take them).  Against the reference's order (lane k of groups 4j + k,
// then ((l0 + l1) + l2) + l3 and the groups past the fours) only float32 rounding differs: the tests hold every
// matrix to |err| <= 1e-5 max|y| (the reference's LINE, tests/tile-bench.ts:34-41), and where every term and every
// partial sum is exact (scales powers of two, small sums) to the reference's number, bit for bit.
//
// Why a second form: the bit-exact tile (gemm.hip) spends three float32 VALU operations on every (row, token, group)
// — convert, multiply, add in the reference's order — and on gfx950 those, not the matrix cores, bound it.  Here:
//  * the group's integer leaves the matrix core as a float32 already: two v_mfma_f32_32x32x16_f16 on the int8 values
//    widened to float16 (exact: |w| <= 128, |q - 64| <= 192, so every product and every partial sum of a group is an
//    integer below 2^24 and the float32 accumulation is exact);
//  * the scales' products are an outer product on the matrix core (v_mfma_f32_32x32x1_2b_f32), in the fold's layout,
//    each rounded once as v_mul_f32 rounds it;
//  * the fold is one v_fma_f32 an output.
// The activations are widened once, before the tiles, by tol_prepare (q - 64 as float16; their scales group-major);
// the weights are widened in registers, by each wave once a group for its 128 tokens (a byte ^ 0x80 put under a
// float16 exponent byte 0x64 is 1152 + the byte; one packed float16 add takes 1152 away, exactly).
//
// Tiles: a block of 4 waves computes 128 rows x 128 tokens; wave w rows 32 w .. + 31 and all 128 tokens (4 halves of
// 32): every wave owns its outputs over all the groups, so nothing is added across waves.  A stage is two groups —
// the tokens' float16 activations (16 KB), the rows' bytes (8 KB) and the two scales of each row and token — loaded
// by the buffer-to-LDS path into a ring of 3 stage buffers, two stages in flight; two blocks a CU.
#include "common.hpp"
#include "launch.hpp"
#include "stage.hpp"

namespace hq {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

constexpr int TR = 128, TT = 128;  // a tile's rows and tokens
constexpr int TG = 2;              // groups a stage
constexpr int TRING = 3;           // stage buffers
constexpr int TW = 256;            // threads a block
constexpr int XPLANE = TT * 64;    // a stage's float16 activations of one group: 128 tokens x 64 bytes
constexpr int WPLANE = TR * 32;    // a stage's weights of one group: 128 rows x 32 bytes

// A stage: its two groups' activations and weights as planes (group 2 s + gl in plane gl), so that a group's
// operands are at the same lane addresses in every plane (the plane an immediate offset, the buffer a base)
struct alignas(16) StageF {
  char x[TG][XPLANE];  // token t of plane gl: 32 float16 (64 bytes), 16-byte chunk c at c ^ xswz(t)
  char w[TG][WPLANE];  // row r of plane gl: 32 bytes, chunk c at c ^ wswz(r)
  float ws[TR][TG];    // the rows' scales of the stage's groups
  float xs[TG][TT];    // the tokens' scales, group-major
};
constexpr int SB = 26624;  // sizeof(StageF): buffer b of the ring at b SB
static_assert(sizeof(StageF) == SB, "stage size");

// 16 lanes (64 banks) or 8 (32 banks) reading one chunk of consecutive rows 64 (or 32) bytes apart hit distinct banks
HQ_DEV int xswz(int t) { return ((t >> 1) ^ (t >> 3)) & 3; }
HQ_DEV int wswz(int r) { return ((r >> 2) ^ (r >> 3)) & 1; }

// the float16 of 8 int8 (two dwords) plus a bias: byte ^ 0x80 under the exponent byte 0x64 is the half 1152 + byte,
// and one packed add of `minus` = -(1152 - bias) leaves byte + bias (every value exact: |.| <= 2048)
HQ_DEV h8 widen8(uint32_t d0, uint32_t d1, _Float16 minus) {
  const h2 m = {minus, minus};
  h8 v;
  const uint32_t d[2] = {d0 ^ 0x80808080u, d1 ^ 0x80808080u};
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const h2 lo = __builtin_bit_cast(h2, perm(0x64646464u, d[i], 0x05010400u)) + m;  // bytes 0, 1
    const h2 hi = __builtin_bit_cast(h2, perm(0x64646464u, d[i], 0x07030602u)) + m;  // bytes 2, 3
    v[4 * i] = lo[0];
    v[4 * i + 1] = lo[1];
    v[4 * i + 2] = hi[0];
    v[4 * i + 3] = hi[1];
  }
  return v;
}

struct TolJob {
  char *out;
  const char *xh, *xst, *wq, *ws;
  int32_t n, r0, r1, count, cp;
  int64_t os;
};

// A block's loads of a stage as 32 pieces dealt to the waves in turn (wave W takes W, W + 4, ...): 16 of the
// activations (plane p / 8, 16 tokens x 64 bytes each), 8 of the weights (plane q / 4, 32 rows x 32 bytes), 4 of the
// rows' scales (32 rows x 2, four bytes a lane), and the tokens' scales (2 groups x 128, 16 bytes a lane), loaded by
// the last four pieces alike (the same bytes to the same place), so that every wave issues 8 loads a stage.
template <int W>
struct TolLoads {
  static constexpr int PW = 8;
  __amdgpu_buffer_rsrc_t rx, rw, rws, rxs;
  uint32_t off[PW];

  HQ_DEV TolLoads(const TolJob &J, int row0, int tok0) {
    const int lane = threadIdx.x & 63, ng = J.n >> 5;
    const int64_t tb = 2 * (int64_t)J.n;  // a token's float16 row
    rx = resource(J.xh + tok0 * tb, (J.count - tok0) * tb);
    rw = resource(J.wq + (int64_t)row0 * J.n, (int64_t)(J.r1 - row0) * J.n);
    rws = resource(J.ws + (int64_t)row0 * ng * 4, (int64_t)(J.r1 - row0) * ng * 4);
    rxs = resource(J.xst + (int64_t)tok0 * 4, ((int64_t)ng * J.cp - tok0) * 4);
#pragma unroll
    for (int k = 0; k < PW; k++) {
      const int p = W + 4 * k;
      uint32_t o;
      if (p < 16) {
        const int tok = 16 * (p & 7) + (lane >> 2), ch = (lane & 3) ^ xswz(tok);
        o = (uint32_t)(tok * tb + (p >> 3) * 64 + ch * 16);
      } else if (p < 24) {
        const int q = p - 16, row = 32 * (q & 3) + (lane >> 1), ch = (lane & 1) ^ wswz(row);
        o = (uint32_t)(row * J.n + (q >> 2) * 32 + ch * 16);
      } else if (p < 28) {
        const int row = 32 * (p - 24) + (lane >> 1);
        o = (uint32_t)((row * ng + (lane & 1)) * 4);
      } else {
        o = (uint32_t)(((lane >> 5) * J.cp + 4 * (lane & 31)) * 4);
      }
      off[k] = o;
    }
  }

  // this wave's loads of stage s (groups 2 s, 2 s + 1) into S (s and cp are the same in every lane: said so, or the
  // compiler would loop over the lanes around each load)
  HQ_DEV void load(StageF &S, int s, int cp) {
    s = __builtin_amdgcn_readfirstlane(s);
    cp = __builtin_amdgcn_readfirstlane(cp);
#pragma unroll
    for (int k = 0; k < PW; k++) {
      const int p = W + 4 * k;
      if (p < 16) dma16(rx, S.x[p >> 3] + (p & 7) * 1024, off[k], s * TG * 64);
      else if (p < 24) dma16(rw, S.w[(p - 16) >> 2] + ((p - 16) & 3) * 1024, off[k], s * TG * 32);
      else if (p < 28) dma4(rws, &S.ws[32 * (p - 24)][0], off[k], s * TG * 4);
      else dma16(rxs, &S.xs[0][0], off[k], s * TG * cp * 4);
    }
  }
};

// ---- operand reads: LDS reads whose results are waited for later (wait), each at a lane address plus an immediate
// (the plane).  The wait names the registers it completes ("+v"), so that nothing reads them before it.
template <int OFF>
HQ_DEV h8 ld128(uint32_t a) {
  h8 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=&v"(v) : "v"(a), "i"(OFF));
  return v;
}
template <int OFF>
HQ_DEV v4i ld128i(uint32_t a) {
  v4i v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=&v"(v) : "v"(a), "i"(OFF));
  return v;
}
template <int OFF>
HQ_DEV float ld32(uint32_t a) {
  float v;
  asm volatile("ds_read_b32 %0, %1 offset:%2" : "=&v"(v) : "v"(a), "i"(OFF));
  return v;
}

struct Half {  // a token half's activations of one group: K runs 0 and 1
  h8 k0, k1;
};
struct Head {  // a group's weights (16 bytes a lane), its rows' scale, and the scales of tokens lane and 64 + lane
  v4i w;
  float ws, xs0, xs1;
};
HQ_DEV void wait(Half &a) { asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a.k0), "+v"(a.k1)); }
HQ_DEV void wait(Half &a, Head &h) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a.k0), "+v"(a.k1), "+v"(h.w), "+v"(h.ws), "+v"(h.xs0), "+v"(h.xs1));
}

// a lane's addresses into a stage buffer's plane 0: its token l % 32's two K runs (token half h's are 2048 h bytes
// on: xswz(32 h + t) is xswz(t)), its row's weights and scales, the scale of token lane
struct Addr {
  uint32_t x[2], w, ws, xs;
};
HQ_DEV Addr addresses(const StageF &S, int slice, int lane) {
  Addr a;
  const int kh = lane >> 5, l32 = lane & 31, row = 32 * slice + l32;
#pragma unroll
  for (int j = 0; j < 2; j++) a.x[j] = lds_addr(S.x[0] + l32 * 64 + (((2 * kh + j) ^ xswz(l32)) << 4));
  a.w = lds_addr(S.w[0] + row * 32 + ((kh ^ wswz(row)) << 4));
  a.ws = lds_addr(&S.ws[row][0]);
  a.xs = lds_addr(&S.xs[0][lane]);
  return a;
}
// group g + 1's addresses from group g's: the next plane of the buffer (g even), or plane 0 of the next stage's buffer
// (g odd: buffer (g / 2 + 1) % 3); each array's plane is its own size
HQ_DEV Addr after(const Addr &a, int g) {
  const int b = (g >> 1) % TRING, up = (b == TRING - 1 ? 1 - TRING : 1) * SB;
  const bool odd = g & 1;
  Addr m;
#pragma unroll
  for (int j = 0; j < 2; j++) m.x[j] = a.x[j] + (uint32_t)(odd ? up - XPLANE : XPLANE);
  m.w = a.w + (uint32_t)(odd ? up - WPLANE : WPLANE);
  m.ws = a.ws + (uint32_t)(odd ? up - 4 : 4);
  m.xs = a.xs + (uint32_t)(odd ? up - 4 * TT : 4 * TT);
  return m;
}

HQ_DEV Half read_half(const Addr &ad, int h) {
  Half a;
  switch (h) {  // (a constant at every call)
  case 0: a.k0 = ld128<0>(ad.x[0]); a.k1 = ld128<0>(ad.x[1]); break;
  case 1: a.k0 = ld128<2048>(ad.x[0]); a.k1 = ld128<2048>(ad.x[1]); break;
  case 2: a.k0 = ld128<4096>(ad.x[0]); a.k1 = ld128<4096>(ad.x[1]); break;
  default: a.k0 = ld128<6144>(ad.x[0]); a.k1 = ld128<6144>(ad.x[1]); break;
  }
  return a;
}
HQ_DEV Head read_head(const Addr &ad) {
  Head h;
  h.w = ld128i<0>(ad.w);
  h.ws = ld32<0>(ad.ws);
  h.xs0 = ld32<0>(ad.xs);
  h.xs1 = ld32<256>(ad.xs);
  return h;
}

// What a wave carries from unit to unit: the previous unit's product (folded in the next unit), the scale products in
// use (halves 0, 1 of the group, then halves 2, 3), the group's weights as float16, its head, the current unit's
// activations
struct Carry {
  v16f fp;
  v32f s;
  h8 wf0, wf1;
  Head hd;
  Half a;
};

HQ_DEV v32f outer(float xs, float ws) {
  const v32f z = {};
  return __builtin_amdgcn_mfma_f32_32x32x1f32(xs, ws, z, 0, 0, 0);
}
template <int LO>
HQ_DEV void fold8(float acc[16], const v16f &f, const v32f &s, int so) {
#pragma unroll
  for (int r = LO; r < LO + 8; r++) acc[r] = __builtin_fmaf(f[r], s[so + r], acc[r]);
}
HQ_DEV void widen_weights(Carry &c) {
  const _Float16 minus = (_Float16)0.0f - (_Float16)1152.0f;
  c.wf0 = widen8((uint32_t)c.hd.w[0], (uint32_t)c.hd.w[1], minus);
  c.wf1 = widen8((uint32_t)c.hd.w[2], (uint32_t)c.hd.w[3], minus);
}

// One unit (a group's token half): its two float16 MFMAs with the fold of the previous unit's product between them
// (acc[PH] += fp * s, s's values 16 (PH % 2) ..), so that the matrix core and the VALU work on independent things in
// one wave; the next unit's reads `next` issued after the first MFMA.  Returns this unit's product.
template <int PH, typename Next>
HQ_DEV v16f unit(Carry &c, const Half &a, float acc[4][16], Next next) {
  const v16f z = {};
  v16f f = __builtin_amdgcn_mfma_f32_32x32x16_f16(a.k0, c.wf0, z, 0, 0, 0);
  __builtin_amdgcn_sched_barrier(0);
  next();
  fold8<0>(acc[PH], c.fp, c.s, 16 * (PH & 1));
  __builtin_amdgcn_sched_barrier(0);
  f = __builtin_amdgcn_mfma_f32_32x32x16_f16(a.k1, c.wf1, f, 0, 0, 0);
  __builtin_amdgcn_sched_barrier(0);
  fold8<8>(acc[PH], c.fp, c.s, 16 * (PH & 1));
  return f;
}

// Group g (its operands' addresses `ad`, the next group's `an`) in four units; at its start the group's head is in c
// (weights widened) and its first half's activations are read and waited for.  A group's scale products are made
// when the ones before them are used (halves 0, 1 after the previous group's halves 2, 3 are folded; halves 2, 3
// after halves 0, 1): one of them live.  At the last group of a stage the next stage's buffer is made ready (every
// wave past its reads of this one, the next stage landed) and the stage three ahead is loaded into this buffer.
template <int W>
HQ_DEV void group(Carry &c, float acc[4][16], const Addr &ad, const Addr &an, TolLoads<W> &L, StageF *ring, int g,
                  int ng, int stages, int cp) {
  const bool more = g + 1 < ng;
  Half n;
  // unit 0: the previous group's half 3 folded here
  v16f f = unit<3>(c, c.a, acc, [&] { n = read_half(ad, 1); });
  c.fp = f;
  c.s = outer(c.hd.xs0, c.hd.ws);
  wait(n);
  f = unit<0>(c, n, acc, [&] { c.a = read_half(ad, 2); });
  c.fp = f;
  wait(c.a);
  f = unit<1>(c, c.a, acc, [&] { n = read_half(ad, 3); });
  c.fp = f;
  c.s = outer(c.hd.xs1, c.hd.ws);
  // the next group's head and first activations are read whether or not there is one (the addresses are in the
  // ring either way, and a past-the-end group's values are never used): register state that changed only on one
  // path would keep this group's values live to the join
  if (more && (g & 1)) {
    // every read of this buffer is done (this wave's last, issued above, waited for), the next stage has landed (the
    // one after it may still be in flight): then the barrier, and the stage three ahead into this buffer
    wait(n);
    const int s = g >> 1;
    if (s + 2 < stages) stage_ready<TolLoads<W>::PW>();
    else stage_ready<0>();
    if (s + 3 < stages) L.load(ring[s % TRING], s + 3, cp);
  }
  Head hn = read_head(an);
  wait(n, hn);
  f = unit<2>(c, n, acc, [&] { c.a = read_half(an, 0); });
  c.fp = f;
  c.hd = hn;
  widen_weights(c);
  wait(c.a);
}

template <int W>
HQ_DEV void tol_wave(const TolJob &J, int row0, int tok0, StageF *ring, float acc[4][16], int lane) {
  TolLoads<W> L(J, row0, tok0);
  const int ng = J.n >> 5, stages = (ng + TG - 1) / TG;
  const Addr ad = addresses(ring[0], W, lane);  // group 0's (buffer 0, plane 0)
  L.load(ring[0], 0, J.cp);
  if (stages > 1) L.load(ring[1], 1, J.cp);
  if (stages > 1) stage_ready<TolLoads<W>::PW>();
  else stage_ready<0>();
  if (stages > 2) L.load(ring[2], 2, J.cp);
  Carry c;
  // the first group's first unit folds a product of zeros with zero scales: fma(0, 0, acc) is acc exactly
#pragma unroll
  for (int r = 0; r < 16; r++) c.fp[r] = 0.0f;
#pragma unroll
  for (int r = 0; r < 32; r++) c.s[r] = 0.0f;
  c.hd = read_head(ad);
  c.a = read_half(ad, 0);
  wait(c.a, c.hd);
  widen_weights(c);
  Addr cur = ad;
  for (int g = 0; g < ng; g++) {
    const Addr next = after(cur, g);
    group<W>(c, acc, cur, next, L, ring, g, ng, stages, J.cp);
    cur = next;
  }
  fold8<0>(acc[3], c.fp, c.s, 16);  // the last unit's product
  fold8<8>(acc[3], c.fp, c.s, 16);
}

__global__ __launch_bounds__(TW, 2) void gemm_tol(TolJob J) {
  __shared__ StageF ring[TRING];
  int rb, tb;
  tile_of(blockIdx.x, gridDim.x, (J.r1 - J.r0 + TR - 1) / TR, rb, tb);
  const int row0 = J.r0 + rb * TR, tok0 = tb * TT;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float acc[4][16];
#pragma unroll
  for (int h = 0; h < 4; h++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[h][r] = 0.0f;
  switch (wave) {
  case 0: tol_wave<0>(J, row0, tok0, ring, acc, lane); break;
  case 1: tol_wave<1>(J, row0, tok0, ring, acc, lane); break;
  case 2: tol_wave<2>(J, row0, tok0, ring, acc, lane); break;
  default: tol_wave<3>(J, row0, tok0, ring, acc, lane); break;
  }
  // lane l: row l % 32 of the wave's rows; value r of half h: token 32 h + 8 (r / 4) + 4 (l / 32) + r % 4
  const int row = row0 + 32 * wave + (lane & 31);
  if (row < J.r1) {
#pragma unroll
    for (int h = 0; h < 4; h++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int t = tok0 + 32 * h + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (t < J.count) ((float *)(J.out + t * J.os))[row] = acc[h][r];
      }
  }
}

// the activations as the tiles take them, in one launch: the first `xblocks` blocks widen token t's bytes (xq + t
// frame) to float16 q - 64 at xh + 2 n t, sixteen a thread; the others copy its scales (xs + t sframe) group-major
// to xst + 4 (g cp + t), zeros past the last token
__global__ __launch_bounds__(256) void tol_prepare(const char *xq, const char *xs, int64_t frame, int64_t sframe,
                                                   int32_t n, int32_t count, int32_t cp, int64_t xblocks,
                                                   _Float16 *xh, float *xst) {
  if ((int64_t)blockIdx.x < xblocks) {
    const int64_t per = n >> 4;  // sixteen bytes a thread
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= per * count) return;
    const int64_t t = i / per, c = i - t * per;
    const uint4 q = *(const uint4 *)(xq + t * frame + 16 * c);
    const _Float16 minus = (_Float16)0.0f - (_Float16)1216.0f;  // 1152 + byte - 1216 = byte - 64
    h8 *dst = (h8 *)(xh + t * (int64_t)n + 16 * c);
    dst[0] = widen8(q.x, q.y, minus);
    dst[1] = widen8(q.z, q.w, minus);
    return;
  }
  const int ng = n >> 5;
  const int64_t i = ((int64_t)blockIdx.x - xblocks) * 256 + threadIdx.x;
  if (i >= (int64_t)ng * cp) return;
  const int64_t g = i / cp, t = i - g * cp;
  xst[i] = t < count ? *(const float *)(xs + t * sframe + 4 * g) : 0.0f;
}

}  // namespace

int64_t tol_work_bytes(int32_t n, int32_t count) {
  const int64_t cp = ((int64_t)count + 3) & ~(int64_t)3;
  return ((2 * (int64_t)n * count + 255) & ~(int64_t)255) + 4 * (int64_t)(n >> 5) * cp;
}

int64_t tol_tiles(int32_t rows, int32_t count) {
  return ((int64_t)rows + TR - 1) / TR * (((int64_t)count + TT - 1) / TT);
}

hipError_t launch_gemm_tol(const Job &job, char *work, hipStream_t s) {
  const int rows = job.r1 - job.r0;
  if (rows <= 0 || job.count <= 0) return hipSuccess;
  const int n = job.n, ng = n >> 5, count = job.count;
  const int cp = (count + 3) & ~3;
  _Float16 *xh = (_Float16 *)work;
  float *xst = (float *)(work + (((2 * (int64_t)n * count) + 255) & ~(int64_t)255));
  const int64_t xblocks = ((int64_t)(n >> 4) * count + 255) / 256, sblocks = ((int64_t)ng * cp + 255) / 256;
  hipLaunchKernelGGL(tol_prepare, dim3((uint32_t)(xblocks + sblocks)), dim3(256), 0, s, job.xq, job.xs, job.frame,
                     job.sframe, n, count, cp, xblocks, xh, xst);
  TolJob J{job.out, (const char *)xh, (const char *)xst, job.wq, job.ws, n, job.r0, job.r1, count, cp, job.os};
  const dim3 grid((uint32_t)tol_tiles(rows, count));
  hipLaunchKernelGGL(gemm_tol, grid, dim3(TW), 0, s, J);
  return hipGetLastError();
}

}  // namespace hq
