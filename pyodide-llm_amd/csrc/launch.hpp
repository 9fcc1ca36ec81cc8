// launch.hpp — the host-side launchers of libhq.so's kernels (defined in quantize.hip, gemv.hip, gemm.hip) and
// the job descriptors they take.  abi.cpp validates the C-ABI's arguments and calls these; they only launch.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hq {

// one matrix-times-activations job: rows [r0, r1) of the weights at wq (scales ws, corrections wc or NULL) for
// `count` tokens (activations at xq + t frame, their scales at xs + t sframe; outputs at out + t os, row i at + 4 i)
struct Job {
  char *out;
  const char *xq, *xs, *wq, *ws, *wc;
  int32_t n, r0, r1, count;
  int64_t os, frame, sframe;
};

// a kind's number is its place in the reference's WORK (src/runtime/jobs.ts:207-336)
enum Kind : int32_t { Q8R = 0, Q8 = 1, Q6R = 5, Q6 = 6, T2R = 8, T2 = 9, B1R = 13, B1 = 14 };
// the kinds whose weights are signs and a float16 scale a group of 128 (ternary, binary): interleave()'s activations
constexpr bool signs_kind(Kind k) { return k == T2R || k == T2 || k == B1R || k == B1; }
constexpr bool binary_kind(Kind k) { return k == B1R || k == B1; }

// activations: count tokens of n values (x + t x_stride) -> xq + t frame, xs + t frame
hipError_t launch_quantize_x(char *xq, char *xs, const char *x, int32_t n, int32_t bias, int32_t count,
                             int64_t frame, int64_t x_stride, hipStream_t s);
hipError_t launch_interleave(char *xq, char *xs, int32_t n, int32_t count, int64_t frame, hipStream_t s);
hipError_t launch_int8_sums(int32_t *out, const char *w, int32_t groups, hipStream_t s);
hipError_t launch_six_sums(int32_t *out, const char *w, int32_t groups, hipStream_t s);
// binary weights from float32: groups of 128 -> 16 bytes and the largest |value| each; *bad = 1 (bad: NULL or a word
// the caller cleared) where a value is not plus or minus its group's largest
hipError_t launch_binary_x(uint8_t *out, float *xs, const float *x, int32_t groups, int32_t *bad, hipStream_t s);

// GEMV-shaped products (every job of one kind and one token count, 1..4; up to kMaxJobs jobs a launch)
constexpr int kMaxJobs = 8;
hipError_t launch_gemv(Kind kind, const Job *jobs, int32_t njobs, hipStream_t s);
// the relaxed kinds with quantize_x fused: each block quantizes token t's n float32 activations at x + t x_stride
// (bias 64) into LDS itself; the jobs' xq / xs are not read
hipError_t launch_gemv_fused(Kind kind, const Job *jobs, int32_t njobs, const char *x, int64_t x_stride,
                             hipStream_t s);

// MFMA GEMM-shaped products (one job a launch; count > 4 tokens): the tiles of matmul_q8r_tile, matmul_q6r and
// matmul_t2r_tile over a prompt.  Returns hipErrorNotSupported for a kind that has none.
hipError_t launch_gemm(Kind kind, const Job &job, hipStream_t s);

// the ceilings (ceilings.hip): every byte of [p, p + bytes) read once; `iterations` x 8 MFMAs a wave of `blocks`
// blocks of 4 waves.  sink: 256 words that are almost never written
hipError_t launch_ceiling_read(const char *p, int64_t bytes, uint32_t *sink, hipStream_t s);
hipError_t launch_ceiling_mfma(int32_t blocks, int32_t iterations, int32_t *sink, hipStream_t s);

// which path a job of `count` tokens takes
constexpr int kGemvMaxTokens = 4;
bool gemm_supported(Kind kind);

}  // namespace hq
