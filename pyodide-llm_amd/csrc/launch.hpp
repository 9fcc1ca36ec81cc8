// launch.hpp — the host-side launchers of libhq.so's kernels (defined in quantize.hip, gemv.hip, gemm.hip) and
// the job descriptors they take.  abi.cpp validates the C-ABI's arguments and calls these; they only launch.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hq {

// one matrix-times-activations job: rows [r0, r1) of the weights at wq (scales ws, corrections wc or NULL) for
// `count` tokens (activations at xq + t frame, their scales at xs + t sframe; outputs at out + t os, row i at + 4 i)
// llama.cpp's blocks (the sb kinds): ws is the tables (sb_tables's area) and type the block type
struct Job {
  char *out;
  const char *xq, *xs, *wq, *ws, *wc;
  int32_t n, r0, r1, count;
  int64_t os, frame, sframe;
  int32_t type;
};

// a kind's number is its place in the reference's WORK (src/runtime/jobs.ts:207-336)
enum Kind : int32_t { Q8R = 0, Q8 = 1, Q6R = 5, Q6 = 6, T2R = 8, T2 = 9, SBR = 10, SB = 11, SBW = 12, B1R = 13, B1 = 14 };
// the kinds whose weights are signs and a float16 scale a group of 128 (ternary, binary): interleave()'s activations
constexpr bool signs_kind(Kind k) { return k == T2R || k == T2 || k == B1R || k == B1; }
constexpr bool binary_kind(Kind k) { return k == B1R || k == B1; }
// llama.cpp's blocks of 256 weights (kernels/blocks/): matmul_sbr, matmul_sb (and matmul_sbw's numbers, the same)
constexpr bool blocks_kind(Kind k) { return k == SBR || k == SB || k == SBW; }
// the bytes of a block of a GGUF type (Q2_K 10, Q4_K 12, IQ2_XXS 16, IQ2_XS 17, IQ3_XXS 18, IQ1_S 19, IQ3_S 21,
// IQ2_S 22, IQ4_XS 23, IQ1_M 29), 0 for another (kernels/blocks/types.ts:103-106)
constexpr int32_t sb_block_bytes(int32_t type) {
  return type == 16 ? 66 : type == 21 ? 110 : type == 17 ? 74 : type == 22 ? 82 : type == 18 ? 98 : type == 29 ? 56
       : type == 19 ? 50 : type == 10 ? 84 : type == 23 ? 136 : type == 12 ? 144 : 0;
}
constexpr int32_t kSbTables = 34992;  // the bytes of sb_tables's area
constexpr int32_t kSbCodebooks = 33808;  // the bytes of the codebooks row it is made of

// activations: count tokens of n values (x + t x_stride) -> xq + t frame, xs + t frame
hipError_t launch_quantize_x(char *xq, char *xs, const char *x, int32_t n, int32_t bias, int32_t count,
                             int64_t frame, int64_t x_stride, hipStream_t s);
hipError_t launch_interleave(char *xq, char *xs, int32_t n, int32_t count, int64_t frame, hipStream_t s);
hipError_t launch_int8_sums(int32_t *out, const char *w, int32_t groups, hipStream_t s);
hipError_t launch_six_sums(int32_t *out, const char *w, int32_t groups, hipStream_t s);
// binary weights from float32: groups of 128 -> 16 bytes and the largest |value| each; *bad = 1 (bad: NULL or a word
// the caller cleared) where a value is not plus or minus its group's largest
hipError_t launch_binary_x(uint8_t *out, float *xs, const float *x, int32_t groups, int32_t *bad, hipStream_t s);
// int6 weights from float32: groups of 32 -> 24 bytes and the scale / 4 each; ternary weights: groups of 128 -> 32
// bytes of codes and the largest |value|, *bad = 1 (bad: NULL or a word the caller cleared) where one is not ternary
hipError_t launch_quantize6_x(uint8_t *out, float *xs, const float *x, int32_t groups, hipStream_t s);
hipError_t launch_ternary_x(uint8_t *out, float *xs, const float *x, int32_t groups, int32_t *bad, hipStream_t s);

// the current device's compute units (256 on an MI355X; 256 when the query fails), for grids of blocks that take
// work in turn
inline int cu_count() {
  static int cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int cus = 0;
    cache[dev] = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0
                     ? cus : 256;
  }
  return cache[dev];
}

// GEMV-shaped products (every job of one kind and one token count, 1..4; up to kMaxJobs jobs a launch)
constexpr int kMaxJobs = 8;
hipError_t launch_gemv(Kind kind, const Job *jobs, int32_t njobs, hipStream_t s);

// llama.cpp's blocks: the tables from the codebooks row; a token's sums of 16 and 8 after its scales (count tokens,
// frame apart); a row as float32; the products (jobs of the sb kinds, 1..4 tokens, up to kMaxJobs a launch); the
// four lanes of the signed dot product of 16 bytes by 16
hipError_t launch_sb_tables(uint8_t *area, const uint8_t *codebooks, hipStream_t s);
hipError_t launch_sums_x(char *xs, const char *xq, int32_t n, int32_t count, int64_t frame, hipStream_t s);
hipError_t launch_sb_row(float *out, const char *w, const uint8_t *tab, int32_t n, int32_t type, hipStream_t s);
hipError_t launch_sb(const Job *jobs, int32_t njobs, hipStream_t s);
// a prompt of kSbTileMin tokens or more of one job (the sb kinds), on the matrix cores: every (row, token)
// launch_sb's number
constexpr int kSbTileMin = 16;
constexpr int64_t kSbTileFrameMax = (int64_t)1 << 24;  // frame and sframe of a job the tile takes: 128 tokens' offsets fit in int32
hipError_t launch_sb_tile(const Job &job, hipStream_t s);
hipError_t launch_signed_dots(int32_t *out, const int8_t *a, const int8_t *b, hipStream_t s);

// the classifier's outlier channels: add_columns (y += the columns' products, in order); the columns of a packed
// classifier widened to float32 (packing: kPack*; group: the weights a scale is of); the channels taken apart
constexpr int kPackInt8 = 0, kPackInt6 = 1, kPackTernary = 2, kPackBinary = 3;
constexpr int kMaxChannels = 64;
struct Channels {
  int32_t c[kMaxChannels];
  int32_t count;
};
hipError_t launch_add_columns(float *y, const float *rows, const float *a, int32_t count, int32_t n, hipStream_t s);
hipError_t launch_outlier_columns(float *columns, const uint8_t *values, const uint8_t *scales, int32_t packing,
                                  const Channels &ch, int32_t vocab, int32_t dim, int32_t group, hipStream_t s);
hipError_t launch_take_channels(float *picked, float *x, const Channels &ch, hipStream_t s);

// MFMA GEMM-shaped products (one job a launch; count > 4 tokens): the tiles of matmul_q8r_tile, matmul_q6r and
// matmul_t2r_tile over a prompt.  Returns hipErrorNotSupported for a kind that has none.
hipError_t launch_gemm(Kind kind, const Job &job, hipStream_t s);

// the relaxed int8 prompt tile to float32 tolerance (gemm_tol.hip): the job's activations widened into `work`
// (tol_work_bytes(n, count) bytes, 256-byte aligned), then the tiles; job.wc is not read (corrections derived)
int64_t tol_work_bytes(int32_t n, int32_t count);
hipError_t launch_gemm_tol(const Job &job, char *work, hipStream_t s);
// the tiles launch_gemm_tol gives `rows` rows of `count` tokens
int64_t tol_tiles(int32_t rows, int32_t count);

// the ceilings (ceilings.hip): every byte of [p, p + bytes) read once; `iterations` x 8 MFMAs a wave of `blocks`
// blocks of 4 waves.  sink: 256 words that are almost never written
hipError_t launch_ceiling_read(const char *p, int64_t bytes, uint32_t *sink, hipStream_t s);
hipError_t launch_ceiling_mfma(int32_t blocks, int32_t iterations, int32_t *sink, hipStream_t s);
// the prompt tiles' register work (form 0 the bit-exact tile's, 1 the tolerance tile's): `iterations` groups of a
// wave's four 32 x 32 sub-tiles a wave of `blocks` blocks of 4 waves
hipError_t launch_ceiling_epilogue(int32_t form, int32_t blocks, int32_t iterations, int32_t *sink, hipStream_t s);

// which path a job of `count` tokens takes
constexpr int kGemvMaxTokens = 4;
bool gemm_supported(Kind kind);

}  // namespace hq
