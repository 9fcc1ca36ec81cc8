/* oracle.h — TEST INFRASTRUCTURE ONLY.
 *
 * A scalar C restatement of the reference's quantized-matmul arithmetic (takano32/pyodide-llm, kernels/ .ts files),
 * in the reference's own float32 order, used as the parity checker for the HIP library and as the timed CPU
 * baseline ("port").  Nothing on the product path may link, load or call it: only tests/, the smoke check of
 * __graft_entry__.py and bench.py's cpu_baseline leg do.
 *
 * Each function names the reference lines it follows.  Pointers are host pointers; byte strides (os, frame) are
 * bytes, as in the reference.  Every function is reentrant and touches only the rows / tokens it is given.
 */
#ifndef HQ_ORACLE_H
#define HQ_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* kernels/kernel/quantize.ts:124-151 */
void o_quantize_x(void *xq, float *xs, const float *x, int32_t n, int32_t bias);
/* kernels/kernel/matmul.ts:50-58 */
void o_int8_sums(int32_t *out, const int8_t *w, int32_t groups);
/* kernels/kernel/matmul.ts:38-46 (six.ts:16-31 widening) */
void o_six_sums(int32_t *out, const uint8_t *w, int32_t groups);
/* kernels/six.ts:16-31: one 24-byte group -> its 32 int8 values */
void o_six_unpack(int8_t *out32, const uint8_t *group24);
/* kernels/kernel/matmul.ts:134-146 */
void o_interleave(int8_t *xq, float *xs, int32_t n);
/* kernels/kernel/halves.ts:21-23 (half) */
float o_half(uint16_t h);

/* kernels/relaxed/int8.ts:17-50 */
void o_matmul_q8r(float *xout, const uint8_t *xq, const float *xs, const int8_t *wq, const float *ws,
                  const int32_t *wc, int32_t n, int32_t r0, int32_t r1);
/* kernels/kernel/matmul.ts:77-104 */
void o_matmul_q8(float *xout, const int8_t *xq, const float *xs, const int8_t *wq, const float *ws, int32_t n,
                 int32_t r0, int32_t r1);
/* kernels/relaxed/int8.ts:147-166 (every (row, token) is matmul_q8r's number, int8.ts:60-65) */
void o_matmul_q8r_tile(void *xout, const void *xq, const void *xs, const int8_t *wq, const float *ws,
                       const int32_t *wc, int32_t n, int32_t r0, int32_t r1, int32_t count, int32_t os,
                       int32_t frame);
/* kernels/relaxed/six.ts:16-39 */
void o_matmul_q6r(float *xout, const uint8_t *xq, const float *xs, const uint8_t *wq, const float *ws,
                  const int32_t *wc, int32_t n, int32_t r0, int32_t r1);
/* kernels/kernel/matmul.ts:227-244 */
void o_matmul_q6(float *xout, const int8_t *xq, const float *xs, const uint8_t *wq, const float *ws, int32_t n,
                 int32_t r0, int32_t r1);
/* kernels/relaxed/signs.ts:28-55, 117-119 (matmul_t2r) and kernels/kernel/matmul.ts:196-220 (matmul_t2): the
 * same numbers to the bit (tests/ternary-check.ts:7-10) */
void o_matmul_t2r(float *xout, const int8_t *xq, const float *xs, const uint8_t *wq, const uint16_t *ws,
                  int32_t n, int32_t r0, int32_t r1, int32_t three);
/* kernels/relaxed/signs.ts:77-114, 120-122 */
void o_matmul_t2r_tile(void *xout, const void *xq, const void *xs, const uint8_t *wq, const uint16_t *ws,
                       int32_t n, int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame,
                       int32_t three);
/* kernels/relaxed/signs.ts:123-125 (matmul_b1r) and kernels/kernel/matmul.ts:222-224 (matmul_b1): binary weights
 * (kernels/binary.ts: 16 bytes a group of 128, weight 64h + 4c + p at bit 4h + p of byte c), ternary's kernels with
 * bitCodes for the codes (signs.ts:33-37); ternary's numbers for the same signs (tests/ternary-check.ts:286-341) */
void o_matmul_b1r(float *xout, const int8_t *xq, const float *xs, const uint8_t *wq, const uint16_t *ws,
                  int32_t n, int32_t r0, int32_t r1, int32_t two);
/* kernels/relaxed/signs.ts:77-114, 126-128 */
void o_matmul_b1r_tile(void *xout, const void *xq, const void *xs, const uint8_t *wq, const uint16_t *ws,
                       int32_t n, int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame,
                       int32_t two);
/* kernels/kernel/quantize.ts:184-247: n float32 (groups of 128) -> 16 bytes a group (bit 4h + p of byte c set
 * where value 64h + 4c + p is not below 0) and the largest |value| of every group; 1 where a value is not plus or
 * minus its group's largest, else 0 */
int32_t o_binary_x(uint8_t *out, float *xs, const float *x, int32_t n);
/* kernels/kernel/quantize.ts:161-182 (quantize6_x): groups of 32 -> 24 bytes and a scale / 4 each */
void o_quantize6_x(uint8_t *out, float *xs, const float *x, int32_t n);
/* kernels/kernel/quantize.ts:197-225 (ternary_x): groups of 128 -> 32 bytes of codes and the largest |value|; 1 where
 * a value is not ternary */
int32_t o_ternary_x(uint8_t *out, float *xs, const float *x, int32_t n);

/* llama.cpp's blocks of 256 weights (kernels/blocks/types.ts: Q2_K 10, Q4_K 12, IQ2_XXS 16, IQ2_XS 17, IQ3_XXS 18,
 * IQ1_S 19, IQ3_S 21, IQ2_S 22, IQ4_XS 23, IQ1_M 29): the bytes of a block of `type` (types.ts:103-106), 0 for
 * another */
int32_t o_sb_bytes(int32_t type);
/* kernels/blocks/types.ts:323-348: the 34992 bytes of tables from the codebooks row (33808 bytes) */
int32_t o_sb_tables(uint8_t *area, const uint8_t *codebooks);
/* kernels/blocks/token.ts:149-165: after quantize_x(.., 0)'s n/32 scales at xs, the int16 sums of each 16 and 8 */
void o_sums_x(void *xs, const int8_t *xq, int32_t n);
/* kernels/blocks/token.ts:111-147 (matmul_sbr; matmul_sb the same numbers): rows r0..r1 of w (n weights a row in
 * blocks of `type`), tab: o_sb_tables's area, xq / xs: quantize_x(.., 0) + sums_x */
void o_matmul_sbr(float *xout, const int8_t *xq, const void *xs, const uint8_t *w, const uint8_t *tab, int32_t n,
                  int32_t r0, int32_t r1, int32_t type);
/* kernels/blocks/tile.ts (matmul_sbr_tile, matmul_sbw_tile): every (row, token) matmul_sbr's number */
void o_matmul_sbr_tile(void *xout, const void *xq, const void *xs, const uint8_t *w, const uint8_t *tab, int32_t n,
                       int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame, int32_t type);
/* kernels/blocks/row.ts:7-72 (sb_row): a row's n weights as float32 */
void o_sb_row(float *out, const uint8_t *w, const uint8_t *tab, int32_t n, int32_t type);

/* kernels/kernel/matmul.ts:246-266 (add_columns): y[j] += a[c] rows[c][j] for c = 0 .. count-1 in order, each
 * product and each sum a float32 (the four-wide loop and the scalar tail add in this one order) */
void o_add_columns(float *y, const float *rows, const float *a, int32_t count, int32_t n);

/* CPU baseline: the GEMV above over rows [0, rows) on `threads` host threads, rows handed out in chunks as the
 * reference's phase() does (src/runtime/forward/threads.ts:45, 90-137: 4 chunks a thread, a shared counter).
 * kind: 0 matmul_q8r, 1 matmul_q8, 2 matmul_q6r, 3 matmul_q6, 4 matmul_t2r.  Runs `reps` times, returns seconds
 * of the fastest run. */
double o_time_gemv(int32_t kind, float *xout, const void *xq, const void *xs, const void *wq, const void *ws,
                   const void *wc, int32_t n, int32_t rows, int32_t threads, int32_t reps);

#ifdef __cplusplus
}
#endif
#endif
