/* fast.c — TEST INFRASTRUCTURE ONLY: the CPU baseline bench.py times beside the GPU.
 *
 * A vectorised restatement (x86-64 AVX2) of the reference's relaxed int8 products, matmul_q8r
 * (kernels/relaxed/int8.ts:17-50) and its prompt tile matmul_q8r_tile (int8.ts:52-166), as the reference's own CPU
 * path runs them with wasm SIMD (relaxed_dot of unsigned 7-bit activations by int8 weights, four float32 lanes):
 *   - a group's integer: vpmaddubsw of the 32 activations (0..127) by the 32 weights (pairs of products sum to at most
 *     2 x 127 x 128 < 2^15: no saturation), vpmaddwd by ones, the eight int32 lanes added; plus its correction wc;
 *   - the four float32 chains are the four lanes of an SSE register: lane k += f(d_k) x f(ws_k x xs_k) for the groups
 *     4j + k, then ((l0 + l1) + l2) + l3 and the groups past the fours one at a time.
 * Every output is the oracle's (oracle.c's o_matmul_q8r) to the bit: the integers are exact and the float32
 * operations are the same ones in the same order.  tests/test_oracle.py checks that.
 *
 * The tile takes 4 rows x 4 tokens at a time (each group's 4 weight vectors and 4 activation vectors loaded once
 * for 16 integer dots), as the reference's tile does (int8.ts:68-146).  Threads take chunks of rows in turn as the
 * reference's phase() cuts them (src/runtime/forward/threads.ts:45: 4 chunks a thread; quads of rows for a tile). */
#include <immintrin.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdint.h>
#include <time.h>

#define GS 32

static inline __m256i group_dots(const int8_t *w, const uint8_t *x) {
  const __m256i p = _mm256_maddubs_epi16(_mm256_loadu_si256((const __m256i *)x), _mm256_loadu_si256((const __m256i *)w));
  return _mm256_madd_epi16(p, _mm256_set1_epi16(1));
}

/* the four int32 sums of four vectors of eight lanes, as one SSE register (a, b, c, d) */
static inline __m128i sum4(__m256i a, __m256i b, __m256i c, __m256i d) {
  const __m256i ab = _mm256_hadd_epi32(a, b), cd = _mm256_hadd_epi32(c, d);
  const __m256i abcd = _mm256_hadd_epi32(ab, cd); /* a01+a23 b.. c.. d.. | a45+a67 ... */
  return _mm_add_epi32(_mm256_castsi256_si128(abcd), _mm256_extracti128_si256(abcd, 1));
}

static inline int32_t sum1(__m256i a) {
  const __m128i s = _mm_add_epi32(_mm256_castsi256_si128(a), _mm256_extracti128_si256(a, 1));
  const __m128i t = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
  return _mm_cvtsi128_si32(_mm_add_epi32(t, _mm_shuffle_epi32(t, 0xB1)));
}

/* one row of matmul_q8r: its lanes, then the hsum and the tail groups */
static float q8r_row(const int8_t *w, const uint8_t *xq, const float *xs, const float *srow, const int32_t *crow,
                     int32_t ng) {
  const int32_t ng4 = ng & ~3;
  __m128 lane = _mm_setzero_ps();
  for (int32_t g = 0; g < ng4; g += 4) {
    const __m128i d = _mm_add_epi32(sum4(group_dots(w + g * GS, xq + g * GS), group_dots(w + (g + 1) * GS, xq + (g + 1) * GS),
                                         group_dots(w + (g + 2) * GS, xq + (g + 2) * GS),
                                         group_dots(w + (g + 3) * GS, xq + (g + 3) * GS)),
                                    _mm_loadu_si128((const __m128i *)(crow + g)));
    const __m128 s = _mm_mul_ps(_mm_loadu_ps(srow + g), _mm_loadu_ps(xs + g));
    lane = _mm_add_ps(lane, _mm_mul_ps(_mm_cvtepi32_ps(d), s));
  }
  float l[4];
  _mm_storeu_ps(l, lane);
  float sum = ((l[0] + l[1]) + l[2]) + l[3];
  for (int32_t g = ng4; g < ng; g++) {
    const int32_t d = sum1(group_dots(w + g * GS, xq + g * GS)) + crow[g];
    const float s = srow[g] * xs[g];
    sum = sum + (float)d * s;
  }
  return sum;
}

void f_matmul_q8r(float *xout, const uint8_t *xq, const float *xs, const int8_t *wq, const float *ws,
                  const int32_t *wc, int32_t n, int32_t r0, int32_t r1) {
  const int32_t ng = n / GS;
  for (int32_t i = r0; i < r1; i++)
    xout[i] = q8r_row(wq + (int64_t)i * n, xq, xs, ws + (int64_t)i * ng, wc + (int64_t)i * ng, ng);
}

/* rows r0..r0+3 by tokens t0..t0+3 of the tile (every (row, token) matmul_q8r's number) */
static void q8r_quad(char *xout, const char *xq, const char *xs, const int8_t *wq, const float *ws, const int32_t *wc,
                     int32_t n, int32_t r0, int32_t t0, int32_t os, int32_t frame) {
  const int32_t ng = n / GS, ng4 = ng & ~3;
  const int8_t *w[4];
  const float *sr[4];
  const int32_t *cr[4];
  const uint8_t *x[4];
  const float *xsc[4];
  for (int k = 0; k < 4; k++) {
    w[k] = wq + (int64_t)(r0 + k) * n;
    sr[k] = ws + (int64_t)(r0 + k) * ng;
    cr[k] = wc + (int64_t)(r0 + k) * ng;
    x[k] = (const uint8_t *)(xq + (int64_t)(t0 + k) * frame);
    xsc[k] = (const float *)(xs + (int64_t)(t0 + k) * frame);
  }
  __m128 lane[4][4];
  for (int r = 0; r < 4; r++)
    for (int t = 0; t < 4; t++) lane[r][t] = _mm_setzero_ps();
  for (int32_t g = 0; g < ng4; g += 4) {
    for (int r = 0; r < 4; r++) {
      const __m128i c = _mm_loadu_si128((const __m128i *)(cr[r] + g));
      const __m128 wsr = _mm_loadu_ps(sr[r] + g);
      for (int t = 0; t < 4; t++) {
        const __m128i d = _mm_add_epi32(sum4(group_dots(w[r] + g * GS, x[t] + g * GS),
                                             group_dots(w[r] + (g + 1) * GS, x[t] + (g + 1) * GS),
                                             group_dots(w[r] + (g + 2) * GS, x[t] + (g + 2) * GS),
                                             group_dots(w[r] + (g + 3) * GS, x[t] + (g + 3) * GS)),
                                        c);
        const __m128 s = _mm_mul_ps(wsr, _mm_loadu_ps(xsc[t] + g));
        lane[r][t] = _mm_add_ps(lane[r][t], _mm_mul_ps(_mm_cvtepi32_ps(d), s));
      }
    }
  }
  for (int r = 0; r < 4; r++)
    for (int t = 0; t < 4; t++) {
      float l[4];
      _mm_storeu_ps(l, lane[r][t]);
      float sum = ((l[0] + l[1]) + l[2]) + l[3];
      for (int32_t g = ng4; g < ng; g++) {
        const int32_t d = sum1(group_dots(w[r] + g * GS, x[t] + g * GS)) + cr[r][g];
        const float s = sr[r][g] * xsc[t][g];
        sum = sum + (float)d * s;
      }
      ((float *)(xout + (int64_t)(t0 + t) * os))[r0 + r] = sum;
    }
}

void f_matmul_q8r_tile(void *xout, const void *xq, const void *xs, const int8_t *wq, const float *ws,
                       const int32_t *wc, int32_t n, int32_t r0, int32_t r1, int32_t count, int32_t os,
                       int32_t frame) {
  const int32_t rq = r0 + ((r1 - r0) & ~3), tq = count & ~3;
  for (int32_t r = r0; r < rq; r += 4)
    for (int32_t t = 0; t < tq; t += 4) q8r_quad((char *)xout, (const char *)xq, (const char *)xs, wq, ws, wc, n, r, t, os, frame);
  /* the rows past the quads for every token, and the tokens past the quads for the quads' rows */
  for (int32_t t = 0; t < count; t++) {
    float *o = (float *)((char *)xout + (int64_t)t * os);
    const uint8_t *x = (const uint8_t *)((const char *)xq + (int64_t)t * frame);
    const float *s = (const float *)((const char *)xs + (int64_t)t * frame);
    if (t >= tq) f_matmul_q8r(o, x, s, wq, ws, wc, n, r0, rq);
    f_matmul_q8r(o, x, s, wq, ws, wc, n, rq, r1);
  }
}

/* ---- timing: rows in chunks taken in turn by `threads` threads ----------------------------------------------- */
typedef struct {
  float *xout;
  const void *xq, *xs;
  const int8_t *wq;
  const float *ws;
  const int32_t *wc;
  int32_t n, rows, count, os, frame, chunk, chunks;
  atomic_int next;
} fast_job;

static void *fast_worker(void *arg) {
  fast_job *j = (fast_job *)arg;
  for (;;) {
    const int32_t c = atomic_fetch_add(&j->next, 1);
    if (c >= j->chunks) break;
    const int32_t r0 = c * j->chunk, r1 = r0 + j->chunk < j->rows ? r0 + j->chunk : j->rows;
    if (j->count == 0) f_matmul_q8r(j->xout, j->xq, j->xs, j->wq, j->ws, j->wc, j->n, r0, r1);
    else f_matmul_q8r_tile(j->xout, j->xq, j->xs, j->wq, j->ws, j->wc, j->n, r0, r1, j->count, j->os, j->frame);
  }
  return NULL;
}

/* seconds one call takes: matmul_q8r (count 0) or matmul_q8r_tile of `count` tokens over rows 0..rows, on
 * `threads` threads (the calling one among them) */
double f_time_q8r(float *xout, const void *xq, const void *xs, const int8_t *wq, const float *ws, const int32_t *wc,
                  int32_t n, int32_t rows, int32_t count, int32_t os, int32_t frame, int32_t threads) {
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  pthread_t tid[256];
  fast_job j = {xout, xq, xs, wq, ws, wc, n, rows, count, os, frame, 0, 0, 0};
  if (count == 0) {
    j.chunk = (rows + 4 * threads - 1) / (4 * threads);
  } else { /* threads.ts:109-110: quads of rows */
    j.chunk = threads == 1 ? rows : 4 * ((rows + 16 * threads - 1) / (16 * threads));
  }
  if (j.chunk < 1) j.chunk = 1;
  j.chunks = (rows + j.chunk - 1) / j.chunk;
  atomic_init(&j.next, 0);
  struct timespec a, b;
  clock_gettime(CLOCK_MONOTONIC, &a);
  for (int32_t t = 1; t < threads; t++) pthread_create(&tid[t], NULL, fast_worker, &j);
  fast_worker(&j);
  for (int32_t t = 1; t < threads; t++) pthread_join(tid[t], NULL);
  clock_gettime(CLOCK_MONOTONIC, &b);
  return (double)(b.tv_sec - a.tv_sec) + 1e-9 * (double)(b.tv_nsec - a.tv_nsec);
}
