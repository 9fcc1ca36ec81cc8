/* hq.h — the C-ABI of libhq.so: pyodide-llm's quantized-matmul kernels on one AMD Instinct MI355X (gfx950).
 *
 * The first block exports the reference kernels under their own names, arguments and order
 * (takano32/pyodide-llm src/runtime/jobs.ts:101-140, the `Arguments` type; src/python/engine/kernels.py:42-51 for
 * the ctypes form of the same table: usize -> pointer, i32 -> int32_t, f32 -> float).  A host that binds the
 * WebAssembly exports by name (bun:ffi, N-API, ctypes) binds these instead.  What differs from the WebAssembly
 * module:
 *   - every pointer is a DEVICE address (hipMalloc'd, managed, or mapped pinned host memory), passed as a 64-bit
 *     integer where the host language has no pointer type (bun:ffi `u64` / `ptr`);
 *   - every call is stream-ordered: it is enqueued on the library's current stream (hq_set_stream; the null stream
 *     until one is set) and returns before the GPU has finished.  The results are visible to later work on that
 *     stream, and to the host after hq_synchronize() or a synchronous copy;
 *   - a call whose arguments break a precondition launches nothing and records an error code and message for
 *     hq_last_error() / hq_last_error_message() (per host thread), where the WebAssembly kernels (compiled
 *     --noAssert) would write wrong memory.  Preconditions: n > 0, n % 32 == 0 (int8, int6) or n % 128 == 0
 *     (ternary), 0 <= r0 <= r1, count >= 0, three == 3; device pointers of the weights (int8, ternary) and of the
 *     activations 16-byte aligned, int6 weights 8-byte aligned, scales / corrections / outputs 4-byte aligned;
 *     frame a multiple of 16 and os a multiple of 4 where count > 1.
 *   - the relaxed int8 / int6 kernels' activation bytes are the 7-bit second factor of the reference's
 *     relaxed_dot_i8x16_i7x16 (kernels/ceilings_relaxed.ts:6-8): 0..127, as quantize_x(bias 64) writes them.  For
 *     other bytes the reference's sums depend on the machine; libhq takes every byte as a signed int8 (in the token
 *     kernels and the prompt tiles alike).
 *   - matmul_q8r / matmul_q6r / matmul_q8r_tile accept wc == NULL (no counterpart in the reference): the group's
 *     integer is then dot(w, q - 64) computed directly, which is what the reference's integer is whenever wc is
 *     int8_sums' / six_sums' (relaxed/int8.ts:6-11), without reading wc (12.5 % fewer bytes for int8).
 * Every (row, token) output is the reference kernel's float32 number to the bit: the integer of each group is exact
 * and the float32 operations run in the reference's order (see each declaration's citation).
 *
 * The second block (hq_*) is the library's own: stream and error handling, the status-returning `_ex` forms of the
 * kernels (an explicit stream; a failure is also kept for hq_last_error()), the batched activation preparation of a
 * prompt, and
 * hq_phase(), which runs a whole phase of jobs written in the reference's job-table form in as few launches as the
 * jobs allow (src/runtime/jobs.ts:36-46 for the table, 456-477 for what runner() does with each job).
 */
#ifndef HQ_H
#define HQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- the reference's kernels, drop-in (device pointers, stream-ordered, errors via hq_last_error) ------------ */

/* kernels/kernel/quantize.ts:124-151: x (n float32) -> xq (n int8, with the bias added: 0 -> -127..127, 64 ->
 * 1..127) and xs (n/32 float32 scales) */
void quantize_x(void *xq, void *xs, const void *x, int32_t n, int32_t bias);
/* kernels/kernel/matmul.ts:50-58: out[g] = -64 * sum of the 32 int8 of group g (the corrections of matmul_q8r) */
void int8_sums(void *out, const void *w, int32_t groups);
/* kernels/kernel/matmul.ts:38-46: the same of int6 groups (24 bytes each, kernels/six.ts) */
void six_sums(void *out, const void *w, int32_t groups);
/* kernels/kernel/matmul.ts:134-146: the activations of quantize_x(bias 0) laid out in planes for the ternary
 * products, in place, and after the n/32 scales at xs one int32 a group: minus the group's sum */
void interleave(void *xq, void *xs, int32_t n);

/* kernels/relaxed/int8.ts:17-50: rows [r0, r1) of int8 weights (wq: rows of n, ws: n/32 float32 a row, wc: n/32
 * int32 a row) times the activations of quantize_x(bias 64) -> xout[r0..r1) */
void matmul_q8r(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, const void *wc,
                int32_t n, int32_t r0, int32_t r1);
/* kernels/kernel/matmul.ts:77-104: the same with the activations of quantize_x(bias 0) and no corrections */
void matmul_q8(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n, int32_t r0,
               int32_t r1);
/* kernels/relaxed/int8.ts:147-166: matmul_q8r for `count` tokens: token t's activations and scales at xq + t frame
 * and xs + t frame (bytes), its outputs at xout + t os (bytes); every (row, token) is matmul_q8r's number */
void matmul_q8r_tile(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, const void *wc,
                     int32_t n, int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame);
/* kernels/relaxed/six.ts:16-39: int6 weights (24 bytes a group of 32, kernels/six.ts), as matmul_q8r */
void matmul_q6r(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, const void *wc,
                int32_t n, int32_t r0, int32_t r1);
/* kernels/kernel/matmul.ts:227-244: int6 weights, as matmul_q8 */
void matmul_q6(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n, int32_t r0,
               int32_t r1);
/* kernels/relaxed/signs.ts:117-119: ternary weights (32 bytes a group of 128, kernels/ternary.ts; ws: float16
 * scales, one a group) times the activations interleave() left (xs: scales, then the sums) */
void matmul_t2r(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n, int32_t r0,
                int32_t r1, int32_t three);
/* kernels/kernel/matmul.ts:218-220: the same numbers (tests/ternary-check.ts:7-10) */
void matmul_t2(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n, int32_t r0,
               int32_t r1, int32_t three);
/* kernels/relaxed/signs.ts:120-122: matmul_t2r for `count` tokens, strides as matmul_q8r_tile's */
void matmul_t2r_tile(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n,
                     int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame, int32_t three);
/* kernels/relaxed/signs.ts:123-125: binary weights (16 bytes a group of 128, kernels/binary.ts: weight 64h + 4c + p
 * at bit 4h + p of byte c, set for +1; ws: float16 scales, one a group) times the activations interleave() left;
 * every number is matmul_t2r's for the same signs (tests/ternary-check.ts:286-341).  two must be 2 (jobs.ts:52) */
void matmul_b1r(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n, int32_t r0,
                int32_t r1, int32_t two);
/* kernels/kernel/matmul.ts:222-224: the same numbers */
void matmul_b1(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n, int32_t r0,
               int32_t r1, int32_t two);
/* kernels/relaxed/signs.ts:126-128: matmul_b1r for `count` tokens, strides as matmul_q8r_tile's */
void matmul_b1r_tile(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n,
                     int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame, int32_t two);
/* kernels/kernel/quantize.ts:232-247: n float32 values at x (device; groups of 128) -> out (n/8 bytes: bit 4h + p of
 * byte c of a group set where value 64h + 4c + p is not below 0) and xs (the largest |value| of every group, float32);
 * returns 1 where a value is not plus or minus its group's largest (or the call failed: hq_last_error), else 0.
 * It waits for the library's stream to know. */
int32_t binary_x(void *out, void *xs, const void *x, int32_t n);
/* kernels/kernel/quantize.ts:161-182: n float32 values at x (device; groups of 32) -> out (24 bytes a group: the six
 * bits v of each value, v = round(value / scale) in -32..31 with scale = the group's largest |value| / 31, packed as
 * kernels/six.ts reads them) and xs (scale / 4, float32, a group) */
void quantize6_x(void *out, void *xs, const void *x, int32_t n);
/* kernels/kernel/quantize.ts:197-225: n float32 values at x (device; groups of 128) -> out (n/4 bytes: the code
 * sign + 1 of value j at bits 2 (j & 3) of byte j >> 2) and xs (the largest |value| of every group, float32);
 * returns 1 where a value is neither 0 nor plus or minus its group's largest (or the call failed: hq_last_error),
 * else 0.  It waits for the library's stream to know. */
int32_t ternary_x(void *out, void *xs, const void *x, int32_t n);

/* llama.cpp's blocks of 256 weights (kernels/blocks/: Q2_K 10, Q4_K 12, IQ2_XXS 16, IQ2_XS 17, IQ3_XXS 18, IQ1_S 19,
 * IQ3_S 21, IQ2_S 22, IQ4_XS 23, IQ1_M 29; a row is whole blocks, n a multiple of 256; w 2-byte aligned).
 * kernels/blocks/types.ts:323-348: the 34992 bytes of tables at area (16-byte aligned) from the checkpoint's row of
 * codebooks (33808 bytes: the six grids a value a byte, then IQ4_XS's 16 values); returns 34992 */
int32_t sb_tables(void *area, const void *codebooks);
/* kernels/blocks/token.ts:149-165: after quantize_x(xq, xs, x, n, 0)'s n/32 scales at xs, the int16 sums of each
 * 16 of the n activations (n/16), then of each 8 (n/8) */
void sums_x(void *xs, const void *xq, int32_t n);
/* kernels/blocks/token.ts:140-142 (matmul_sbr): rows r0..r1 of w (blocks of `type`) times the activations of
 * quantize_x(.., 0) + sums_x (xq, xs 16-byte aligned); tab: sb_tables's area */
void matmul_sbr(void *xout, const void *xq, const void *xs, const void *w, const void *tab, int32_t n, int32_t r0,
                int32_t r1, int32_t type);
/* kernels/blocks/token.ts:137-139 (matmul_sb): the same numbers */
void matmul_sb(void *xout, const void *xq, const void *xs, const void *w, const void *tab, int32_t n, int32_t r0,
               int32_t r1, int32_t type);
/* kernels/blocks/tile.ts:144-147: matmul_sbr for `count` tokens, strides as matmul_q8r_tile's (multiples of 16) */
void matmul_sbr_tile(void *xout, const void *xq, const void *xs, const void *w, const void *tab, int32_t n, int32_t r0,
                     int32_t r1, int32_t count, int32_t os, int32_t frame, int32_t type);
/* kernels/blocks/tile.ts:231-253: the same numbers (the reference's form for engines whose dot product multiplies
 * signed by signed, with a scratch area of the caller's; this library needs none and does not touch it) */
void matmul_sbw_tile(void *xout, const void *xq, const void *xs, const void *w, const void *tab, int32_t n, int32_t r0,
                     int32_t r1, int32_t count, int32_t os, int32_t frame, int32_t type, void *scratch);
/* kernels/blocks/tile.ts:158-162: out[k] (int32) = the sum of the 4 products a[4k + j] b[4k + j] of the 16 signed
 * bytes at a and b (device): on this device every product is exact, signed by signed */
void signed_dots(void *out, const void *a, const void *b);
/* kernels/blocks/row.ts: the n weights of the row at w as float32 (out 16-byte aligned), each as the converter's
 * reader (src/python/convert/superblocks.py) gives it */
void sb_row(void *out, const void *w, const void *tab, int32_t n, int32_t type);

/* kernels/kernel/matmul.ts:246-266 (add_columns, jobs.ts:108): y[j] += the sum over c < count of a[c] rows[c][j],
 * for j < n, added to y[j] one product at a time in the order of c (each product a float32); rows is (count, n)
 * row-major; y, rows, a 4-byte aligned (device) */
void add_columns(void *y, const void *rows, const void *a, int32_t count, int32_t n);

/* ---- the library's own ----------------------------------------------------------------------------------------- */

enum {
  HQ_OK = 0,
  HQ_ERR_ARGUMENT = 1,  /* a size, range, count or constant the kernel does not take */
  HQ_ERR_ALIGNMENT = 2, /* a pointer or stride not aligned as the kernel reads it */
  HQ_ERR_NULL = 3,      /* a required pointer is NULL */
  HQ_ERR_HIP = 4,       /* the HIP runtime refused the launch or reported an earlier asynchronous error */
  HQ_ERR_KIND = 5,      /* hq_phase: a job kind this library does not run */
  HQ_ERR_DEVICE = 6     /* no gfx950 device */
};

/* the version string, e.g. "hq 1.0 gfx950" */
const char *hq_version(void);
/* sets up the current HIP device (checks it is gfx950); optional, the first call does it; HQ_* status */
int32_t hq_init(void);
/* the stream the drop-in calls enqueue on, process-wide (a hipStream_t; NULL: the null stream) */
int32_t hq_set_stream(void *stream);
void *hq_get_stream(void);
/* waits for the current stream; HQ_OK or HQ_ERR_HIP */
int32_t hq_synchronize(void);
/* the status of the last failed call of this host thread (HQ_OK when none), its message, and a reset */
int32_t hq_last_error(void);
const char *hq_last_error_message(void);
void hq_clear_error(void);

/* status-returning forms of the drop-in kernels, on an explicit stream (NULL: the null stream) */
int32_t hq_quantize_x_ex(void *xq, void *xs, const void *x, int32_t n, int32_t bias, void *stream);
int32_t hq_int8_sums_ex(void *out, const void *w, int32_t groups, void *stream);
int32_t hq_six_sums_ex(void *out, const void *w, int32_t groups, void *stream);
int32_t hq_interleave_ex(void *xq, void *xs, int32_t n, void *stream);
int32_t hq_matmul_q8r_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, const void *wc,
                         int32_t n, int32_t r0, int32_t r1, void *stream);
int32_t hq_matmul_q8_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n,
                        int32_t r0, int32_t r1, void *stream);
int32_t hq_matmul_q8r_tile_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws,
                              const void *wc, int32_t n, int32_t r0, int32_t r1, int32_t count, int32_t os,
                              int32_t frame, void *stream);
int32_t hq_matmul_q6r_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, const void *wc,
                         int32_t n, int32_t r0, int32_t r1, void *stream);
int32_t hq_matmul_q6_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n,
                        int32_t r0, int32_t r1, void *stream);
int32_t hq_matmul_t2r_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n,
                         int32_t r0, int32_t r1, int32_t three, void *stream);
int32_t hq_matmul_t2r_tile_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n,
                              int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame, int32_t three,
                              void *stream);
int32_t hq_matmul_b1r_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n,
                         int32_t r0, int32_t r1, int32_t two, void *stream);
int32_t hq_matmul_b1r_tile_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n,
                              int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame, int32_t two,
                              void *stream);
/* binary_x on a stream, without waiting: `bad` (device, 4-byte aligned; may be NULL) is set to 1 where a value is
 * refused and left as it was otherwise, so the caller clears it first */
int32_t hq_binary_x_ex(void *out, void *xs, const void *x, int32_t n, void *bad, void *stream);
/* quantize6_x on a stream; ternary_x on a stream, without waiting (`bad` as hq_binary_x_ex's) */
int32_t hq_quantize6_x_ex(void *out, void *xs, const void *x, int32_t n, void *stream);
int32_t hq_ternary_x_ex(void *out, void *xs, const void *x, int32_t n, void *bad, void *stream);
int32_t hq_sb_tables_ex(void *area, const void *codebooks, void *stream);
int32_t hq_matmul_sbr_ex(void *xout, const void *xq, const void *xs, const void *w, const void *tab, int32_t n,
                         int32_t r0, int32_t r1, int32_t type, void *stream);
int32_t hq_matmul_sbr_tile_ex(void *xout, const void *xq, const void *xs, const void *w, const void *tab, int32_t n,
                              int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame, int32_t type,
                              void *stream);
int32_t hq_sb_row_ex(void *out, const void *w, const void *tab, int32_t n, int32_t type, void *stream);

/* The classifier's outlier channels (src/runtime/forward/tensors.ts:170-187, engine.ts:459-466): the columns of the
 * packed classifier for these channels (a host array of count <= 64 channel numbers below dim), widened to float32
 * as columns[i][w] = value(w dim + c_i) x its group's scale, for the vocab words w; values and scales as the loader
 * keeps them (packing: HQ_PACK_INT8, whose group is the largest power of two up to 32 that divides dim, float32
 * scales; HQ_PACK_INT6, groups of 32, float32 scales; HQ_PACK_TERNARY / HQ_PACK_BINARY, groups of 128, float16
 * scales). columns 4-byte aligned. */
enum { HQ_PACK_INT8 = 0, HQ_PACK_INT6 = 1, HQ_PACK_TERNARY = 2, HQ_PACK_BINARY = 3 };
int32_t hq_outlier_columns_ex(void *columns, const void *values, const void *scales, int32_t packing,
                              const int32_t *channels, int32_t count, int32_t vocab, int32_t dim, void *stream);
/* engine.ts:461-464: picked[i] = x[c_i], then x[c_i] = 0, channel by channel (x the classifier's input before
 * quantize_x; channels a host array as above); add_columns then adds their products to the logits */
int32_t hq_take_channels_ex(void *picked, void *x, const int32_t *channels, int32_t count, void *stream);
int32_t hq_add_columns_ex(void *y, const void *rows, const void *a, int32_t count, int32_t n, void *stream);

/* The activations of `count` tokens prepared in one launch (src/runtime/forward/engine.ts:405 calls ready() once a
 * token): token t's float32 values at x + t x_stride (bytes) -> xq + t frame and xs + t frame, as quantize_x; and,
 * for the ternary packing, interleave() of each (src/runtime/jobs.ts:421-424). */
int32_t hq_quantize_x_batch(void *xq, void *xs, const void *x, int32_t n, int32_t bias, int32_t count, int32_t frame,
                            int32_t x_stride, void *stream);
int32_t hq_interleave_batch(void *xq, void *xs, int32_t n, int32_t count, int32_t frame, void *stream);
/* sums_x of `count` tokens (token t's xq and xs at + t frame) */
int32_t hq_sums_x_batch(void *xs, const void *xq, int32_t n, int32_t count, int32_t frame, void *stream);

/* One phase of jobs (src/runtime/forward/threads.ts:90-137, src/runtime/jobs.ts:36-46): `jobs` holds `count` jobs
 * of `stride` float64 each (the reference's table has JOB = 16: the first 14 are used), each
 *   [kind, out, a, b, a4, a5, a6, a7, a8, rows, count, os, as, bs]
 * with kind the place of its line in jobs.ts's WORK (0 matmul_q8r, 1 matmul_q8, 5 matmul_q6r, 6 matmul_q6,
 * 8 matmul_t2r, 9 matmul_t2, 10 matmul_sbr, 11 matmul_sb, 12 matmul_sbw, 13 matmul_b1r, 14 matmul_b1), the eight arguments as WORK's `one` reads them, and every row [0, rows) of every one
 * of `count` tokens run (a job's out / a / b advance by os / as / bs bytes a token).  The addresses are device
 * addresses held exactly in the doubles (below 2^53).  Jobs of one kind and token count share a launch. */
int32_t hq_phase(const double *jobs, int32_t count, int32_t stride, void *stream);

/* src/runtime/forward/engine.ts:381-407 (matmulsAlike): the phase of jobs of one input, from its float32
 * activations: every job takes the same n and token count, token t's n values at x + t x_stride (bytes; x and
 * x_stride 16-byte aligned).  A kind at a time, the input is readied into its jobs' a / b as that kind takes it
 * (quantize_x at its bias, and interleave for ternary and binary, sums_x for llama.cpp's blocks; jobs.ts:376-379,
 * 385-395, 421-424: a pair of a / b several jobs share is readied once) and then those jobs run as hq_phase runs
 * them; a job's a and b advance by one frame a token (as = bs).  Every output is the number quantize_x + the kernel
 * give, and a / b hold the readied activations after the call. */
int32_t hq_matmuls(const void *x, int32_t x_stride, const double *jobs, int32_t count, int32_t stride, void *stream);

/* hq_matmuls without the caller's staging, for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc); it has no counterpart in the reference.  The same jobs
 * and outputs, but the jobs' a, b, as and bs are not read: the input is readied into a staging area the library
 * holds on each device (a static device array of 4 MiB, looked up by hq_init or by the first call on a device), a
 * token's activations round_up(n, 256) + round_up(n / 2, 256) bytes apart.  Refused (HQ_ERR_ARGUMENT) when the
 * tokens do not fit: count x that frame must be at most 4 MiB (n = 4096: 682 tokens).  No device memory is
 * allocated or freed.  Every call on one device shares that device's staging: calls that overlap on one device
 * (other streams, other threads) race; calls in one stream follow each other. */
int32_t hq_matmuls_static(const void *x, int32_t x_stride, const double *jobs, int32_t count, int32_t stride,
                          void *stream);

/* matmul_q8r_tile's products (src/runtime/forward/engine.ts's prompt blocks; kernels/relaxed/int8.ts:52-166) to the
 * north star's float32 tolerance instead of to the bit, for prompts on the matrix cores: xout + t os row i (i in
 * [r0, r1), t < count) = sum over the groups g of f(ws[i][g] xs_t[g]) * d_g, with d_g = sum_k w[i][k] (q_t[k] - 64)
 * exact (the corrections int8_sums gives, made from the weights: there is no wc argument) and the groups added in an
 * order of this library's, each term one fused multiply-add.  Every output is within 1e-5 max|y| of the reference's
 * (max over the matrix's outputs; tests/tile-bench.ts:34-41's LINE), and equal to it where every term and sum is
 * exact.  Arguments as hq_matmul_q8r_tile_ex's (xq and xs of token t at + t frame; xq, wq 16-byte aligned), plus a
 * device workspace of at least hq_tol_work_bytes(n, count) bytes, 256-byte aligned, that the call writes (the
 * activations widened to float16 and the scales regrouped) before its tiles read it: calls that share a workspace
 * on one stream follow each other, on two streams they race.  Its counterpart in the reference: none (its prompt
 * tile is the bit-exact matmul_q8r_tile). */
int64_t hq_tol_work_bytes(int32_t n, int32_t count);
int32_t hq_matmul_q8r_tile_tol_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws,
                                  int32_t n, int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame,
                                  void *work, int64_t work_bytes, void *stream);
/* The launches hq_matmul_q8r_tile_tol_ex gives its tolerance tile (128 rows x 128 tokens): those of at least `tiles`
 * tiles; a smaller one takes the bit-exact kernels instead (hq_matmul_q8r_tile_ex's, corrections derived: the
 * reference's numbers, inside any tolerance), whose smaller tiles fill the GPU where 128 x 128 would leave it idle.
 * -1 (the default): one round of two blocks a compute unit; 0: every launch takes the tile.  Returns the previous
 * setting; below -1: HQ_ERR_ARGUMENT, nothing changed.  One setting for the process.  Its counterpart in the
 * reference: none. */
int32_t hq_tol_min_tiles(int32_t tiles);

/* Which kernels take a job of `kind` (hq_phase's numbers), row length n and `count` tokens whose activations are
 * frame bytes apart and their scales sframe: 1 the matrix-core tile (16 tokens or more, and every offset within a
 * tile of 64 tokens, 128 for llama.cpp's blocks, and of 128 rows below 4 GiB), 0 the token kernel (4 tokens a
 * launch: the same numbers), -1 a kind not run here.  Host-only: no device is touched. */
int32_t hq_job_path(int32_t kind, int32_t n, int32_t count, int64_t frame, int64_t sframe);

/* The ceilings the kernels are measured against (no counterpart on this path: the reference's CPU ceiling loops,
 * kernels/ceilings.ts:12-25 and ceilings_relaxed.ts:34-52, are its model).  hq_ceiling_read reads every byte of
 * [p, p + bytes) once (bytes a multiple of 16): time it for the achievable HBM read bandwidth of a buffer past the
 * caches.  hq_ceiling_mfma runs `iterations` x 8 v_mfma_i32_32x32x32_i8 (32768 MACs each) in every wave of `blocks`
 * blocks of 4 waves, on registers: the achievable dense int8 rate.  sink: 256 int32 of scratch, almost never
 * written. */
int32_t hq_ceiling_read(const void *p, int64_t bytes, void *sink, void *stream);
int32_t hq_ceiling_mfma(int32_t blocks, int32_t iterations, void *sink, void *stream);
/* The prompt tiles' register work alone (no loads, no LDS), two waves a SIMD: form 0 the bit-exact tile's epilogue
 * (a correction MFMA, the scales' f32 outer product, the int8 MFMAs, and convert, multiply, add an output), form 1
 * the tolerance tile's (the weights' float16 widening, the float16 MFMAs, the outer product, a fused multiply-add an
 * output); `iterations` groups of a wave's four 32 x 32 sub-tiles (262 144 operations) a wave of `blocks` blocks of
 * 4 waves.
 * The most a tile of that epilogue can give; no counterpart in the reference. */
int32_t hq_ceiling_epilogue(int32_t form, int32_t blocks, int32_t iterations, void *sink, void *stream);

#ifdef __cplusplus
}
#endif
#endif
