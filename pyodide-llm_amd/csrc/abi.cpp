// abi.cpp — libhq.so's C-ABI (include/hq.h): argument checks, the error state, the stream, and which kernel each
// call takes.  No kernel is here; the launchers are in quantize.hip, gemv.hip and gemm.hip.
#include "hq.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "launch.hpp"

namespace {

thread_local int32_t g_error = HQ_OK;
thread_local char g_message[512] = "";
std::atomic<void *> g_stream{nullptr};
// hq_tol_min_tiles's setting: -1, one round of two blocks a compute unit
std::atomic<int32_t> g_tol_min_tiles{-1};

// more tokens than this take the matrix cores (fewer: the token kernel, the weights read once a 4 tokens)
constexpr int32_t kGemmMinTokens = 16;

// Which kernels take a job: 1 the matrix-core tile, 0 the token kernel (4 tokens a launch).  The tiles keep a lane's
// offsets within a tile in 32 bits: 64 tokens of activations (frame and sframe bytes apart: 128 for the blocks' tile)
// and 128 rows of weights, so a job whose tile would reach 4 GiB from its first byte takes the token kernel, whose
// addresses are 64-bit.
int32_t path_of(hq::Kind kind, const hq::Job &j) {
  if (hq::blocks_kind(kind)) {
    return j.count >= hq::kSbTileMin && j.frame > 0 && j.sframe > 0 && j.frame < hq::kSbTileFrameMax &&
           j.sframe < hq::kSbTileFrameMax;
  }
  if (j.count < kGemmMinTokens || !hq::gemm_supported(kind)) return 0;
  constexpr int64_t kLimit = (int64_t)1 << 32;
  const int64_t row_bytes = hq::signs_kind(kind) ? (int64_t)(j.n >> 7) * 32 : (int64_t)(j.n >> 5) * 32;
  const int64_t scales = hq::signs_kind(kind) ? 8 * (int64_t)(j.n >> 5) : 4 * (int64_t)(j.n >> 5);
  return 64 * j.frame + j.n < kLimit && 64 * j.sframe + scales < kLimit && 128 * row_bytes < kLimit;
}

int32_t fail(int32_t code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_message, sizeof g_message, fmt, ap);
  va_end(ap);
  g_error = code;
  return code;
}

int32_t hip_status(hipError_t e, const char *what) {
  if (e == hipSuccess) return HQ_OK;
  return fail(HQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// the device check, once a device
std::mutex g_init_mutex;
int8_t g_device_ok[64];  // 0 unknown, 1 gfx950, -1 not

int32_t ensure_device() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(HQ_ERR_DEVICE, "no HIP device: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= 64) return fail(HQ_ERR_DEVICE, "device %d out of range", dev);
  if (g_device_ok[dev] == 1) return HQ_OK;
  std::lock_guard<std::mutex> lock(g_init_mutex);
  if (g_device_ok[dev] == 0) {
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return fail(HQ_ERR_DEVICE, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    g_device_ok[dev] = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : -1;
    if (g_device_ok[dev] != 1) {
      return fail(HQ_ERR_DEVICE, "device %d is %s: libhq.so holds gfx950 code only", dev, prop.gcnArchName);
    }
  }
  return g_device_ok[dev] == 1 ? HQ_OK : fail(HQ_ERR_DEVICE, "device %d is not gfx950", dev);
}

bool aligned(const void *p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// hq_matmuls_static's staging of the readied activations: a device array of the library's own, one copy on each
// device (the runtime makes it when it loads the library's code there; it lives until the process ends).  In host
// code `scratch` names a host-side stand-in: its device address is looked up once a device (hipGetSymbolAddress,
// with that device current) and only that address reaches a kernel.
constexpr int64_t kStagingBytes = (int64_t)4 << 20;
static __device__ __align__(256) char scratch[kStagingBytes];
std::atomic<char *> g_scratch[64];

int32_t scratch_of(char **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(HQ_ERR_DEVICE, "no HIP device: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= 64) return fail(HQ_ERR_DEVICE, "device %d out of range", dev);
  char *p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_init_mutex);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      void *at = nullptr;
      e = hipGetSymbolAddress(&at, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !at) return fail(HQ_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
      p = (char *)at;
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return HQ_OK;
}

hipStream_t stream_of(void *s) { return (hipStream_t)s; }

constexpr int kKinds = 15;  // kinds are numbered by their place in WORK: the last one run here is matmul_b1 (14)

const char *kind_name(hq::Kind k) {
  switch (k) {
  case hq::Q8R: return "matmul_q8r";
  case hq::Q8: return "matmul_q8";
  case hq::Q6R: return "matmul_q6r";
  case hq::Q6: return "matmul_q6";
  case hq::T2R: return "matmul_t2r";
  case hq::T2: return "matmul_t2";
  case hq::B1R: return "matmul_b1r";
  case hq::B1: return "matmul_b1";
  case hq::SBR: return "matmul_sbr";
  case hq::SB: return "matmul_sb";
  case hq::SBW: return "matmul_sbw";
  }
  return "?";
}

// ternary and binary: whole groups of 128, interleave()'s activations, float16 scales
bool ternary(hq::Kind k) { return hq::signs_kind(k); }
bool relaxed(hq::Kind k) { return k == hq::Q8R || k == hq::Q6R; }
bool six(hq::Kind k) { return k == hq::Q6R || k == hq::Q6; }

// the preconditions of a job of llama.cpp's blocks
int32_t check_blocks_job(hq::Kind kind, const hq::Job &j) {
  const char *name = kind_name(kind);
  if (!hq::sb_block_bytes(j.type)) return fail(HQ_ERR_ARGUMENT, "%s: type %d is not one of the ten block types", name, j.type);
  if (j.n <= 0 || j.n % 256) return fail(HQ_ERR_ARGUMENT, "%s: n = %d is not a positive multiple of 256", name, j.n);
  if (j.r0 < 0 || j.r1 < j.r0) return fail(HQ_ERR_ARGUMENT, "%s: rows %d..%d", name, j.r0, j.r1);
  if (j.count < 0) return fail(HQ_ERR_ARGUMENT, "%s: count = %d", name, j.count);
  if (j.r1 == j.r0 || j.count == 0) return HQ_OK;
  if (!j.out || !j.xq || !j.xs || !j.wq || !j.ws) return fail(HQ_ERR_NULL, "%s: a NULL pointer", name);
  if (!aligned(j.wq, 2)) return fail(HQ_ERR_ALIGNMENT, "%s: w not 2-byte aligned", name);
  if ((int64_t)j.r1 * (j.n >> 8) * hq::sb_block_bytes(j.type) > 0xFFFFFFF0LL)
    return fail(HQ_ERR_ARGUMENT, "%s: rows 0..%d of w take 4 GiB or more", name, j.r1);
  if (!aligned(j.ws, 16)) return fail(HQ_ERR_ALIGNMENT, "%s: the tables not 16-byte aligned", name);
  if (!aligned(j.xq, 16) || !aligned(j.xs, 16)) return fail(HQ_ERR_ALIGNMENT, "%s: xq or xs not 16-byte aligned", name);
  if (!aligned(j.out, 4)) return fail(HQ_ERR_ALIGNMENT, "%s: xout not 4-byte aligned", name);
  if (j.count > 1) {
    if (j.os < 0 || j.os % 4) return fail(HQ_ERR_ALIGNMENT, "%s: os = %lld is not a multiple of 4", name, (long long)j.os);
    if (j.frame < 0 || j.frame % 16 || j.sframe < 0 || j.sframe % 16)
      return fail(HQ_ERR_ALIGNMENT, "%s: a token stride is not a multiple of 16", name);
  }
  return HQ_OK;
}

// the preconditions of a matrix job (include/hq.h's list)
int32_t check_job(hq::Kind kind, const hq::Job &j, int32_t three) {
  if (hq::blocks_kind(kind)) return check_blocks_job(kind, j);
  const char *name = kind_name(kind);
  const int32_t unit = ternary(kind) ? 128 : 32;
  if (j.n <= 0 || j.n % unit) return fail(HQ_ERR_ARGUMENT, "%s: n = %d is not a positive multiple of %d", name, j.n, unit);
  if (j.r0 < 0 || j.r1 < j.r0) return fail(HQ_ERR_ARGUMENT, "%s: rows %d..%d", name, j.r0, j.r1);
  if (j.count < 0) return fail(HQ_ERR_ARGUMENT, "%s: count = %d", name, j.count);
  if (ternary(kind) && three != (hq::binary_kind(kind) ? 2 : 3))
    return fail(HQ_ERR_ARGUMENT, "%s: %s = %d, not %d", name, hq::binary_kind(kind) ? "two" : "three", three,
                hq::binary_kind(kind) ? 2 : 3);
  if (j.r1 == j.r0 || j.count == 0) return HQ_OK;
  if (!j.out || !j.xq || !j.xs || !j.wq || !j.ws) return fail(HQ_ERR_NULL, "%s: a NULL pointer", name);
  const uintptr_t wa = six(kind) ? 8 : 16;
  if (!aligned(j.wq, wa)) return fail(HQ_ERR_ALIGNMENT, "%s: wq not %d-byte aligned", name, (int)wa);
  if (!aligned(j.xq, 16)) return fail(HQ_ERR_ALIGNMENT, "%s: xq not 16-byte aligned", name);
  if (!aligned(j.xs, ternary(kind) ? 16 : 4)) return fail(HQ_ERR_ALIGNMENT, "%s: xs misaligned", name);
  if (!aligned(j.ws, ternary(kind) ? 2 : 4)) return fail(HQ_ERR_ALIGNMENT, "%s: ws misaligned", name);
  if (j.wc && !aligned(j.wc, 4)) return fail(HQ_ERR_ALIGNMENT, "%s: wc not 4-byte aligned", name);
  if (!aligned(j.out, 4)) return fail(HQ_ERR_ALIGNMENT, "%s: xout not 4-byte aligned", name);
  if (j.count > 1) {
    if (j.os < 0 || j.os % 4) return fail(HQ_ERR_ALIGNMENT, "%s: os = %lld is not a multiple of 4", name, (long long)j.os);
    if (j.frame < 0 || j.frame % 16) return fail(HQ_ERR_ALIGNMENT, "%s: frame = %lld is not a multiple of 16", name, (long long)j.frame);
    if (j.sframe < 0 || j.sframe % (ternary(kind) ? 16 : 4))
      return fail(HQ_ERR_ALIGNMENT, "%s: the scales' stride %lld is misaligned", name, (long long)j.sframe);
  }
  return HQ_OK;
}

// runs jobs of one kind: GEMV jobs (up to 4 tokens; more in slices of 4) batched in launches of up to kMaxJobs,
// GEMM jobs one a launch
int32_t run_blocks(hq::Kind kind, const std::vector<hq::Job> &jobs, hipStream_t s) {
  // up to 4 tokens a launch (a prompt in slices of 4: every (row, token) the token kernel's number), jobs of one
  // block type, one token count and one tables' area together
  std::vector<hq::Job> parts;
  for (const hq::Job &j : jobs) {
    if (j.r1 == j.r0 || j.count == 0) continue;
    // a prompt: the matrix-core tile (its offsets within a tile of tokens are 32-bit: frames under 16 MB)
    if (path_of(kind, j)) {
      const int32_t st = hip_status(hq::launch_sb_tile(j, s), kind_name(kind));
      if (st) return st;
      continue;
    }
    for (int32_t t0 = 0; t0 < j.count; t0 += hq::kGemvMaxTokens) {
      hq::Job part = j;
      part.count = j.count - t0 < hq::kGemvMaxTokens ? j.count - t0 : hq::kGemvMaxTokens;
      part.out = j.out + t0 * j.os;
      part.xq = j.xq + t0 * j.frame;
      part.xs = j.xs + t0 * j.sframe;
      parts.push_back(part);
    }
  }
  std::vector<bool> done(parts.size(), false);
  for (size_t i = 0; i < parts.size(); i++) {
    if (done[i]) continue;
    std::vector<hq::Job> same;
    for (size_t k = i; k < parts.size() && same.size() < (size_t)hq::kMaxJobs; k++)
      if (!done[k] && parts[k].type == parts[i].type && parts[k].count == parts[i].count && parts[k].ws == parts[i].ws) {
        same.push_back(parts[k]);
        done[k] = true;
      }
    const int32_t st = hip_status(hq::launch_sb(same.data(), (int32_t)same.size(), s), kind_name(kind));
    if (st) return st;
  }
  return HQ_OK;
}

int32_t run_jobs(hq::Kind kind, const std::vector<hq::Job> &jobs, hipStream_t s) {
  if (hq::blocks_kind(kind)) return run_blocks(kind, jobs, s);
  std::vector<hq::Job> gemv[hq::kGemvMaxTokens + 1][2];  // by token count, by wc-ness
  for (const hq::Job &j : jobs) {
    if (j.r1 == j.r0 || j.count == 0) continue;
    if (path_of(kind, j)) {
      const int32_t st = hip_status(hq::launch_gemm(kind, j, s), kind_name(kind));
      if (st) return st;
      continue;
    }
    for (int32_t t0 = 0; t0 < j.count; t0 += hq::kGemvMaxTokens) {
      hq::Job part = j;
      part.count = j.count - t0 < hq::kGemvMaxTokens ? j.count - t0 : hq::kGemvMaxTokens;
      part.out = j.out + t0 * j.os;
      part.xq = j.xq + t0 * j.frame;
      part.xs = j.xs + t0 * j.sframe;
      gemv[part.count][part.wc != nullptr].push_back(part);
    }
  }
  for (int c = 1; c <= hq::kGemvMaxTokens; c++)
    for (int w = 0; w < 2; w++) {
      const auto &list = gemv[c][w];
      for (size_t i = 0; i < list.size(); i += hq::kMaxJobs) {
        const int32_t m = (int32_t)(list.size() - i < (size_t)hq::kMaxJobs ? list.size() - i : hq::kMaxJobs);
        const int32_t st = hip_status(hq::launch_gemv(kind, &list[i], m, s), kind_name(kind));
        if (st) return st;
      }
    }
  return HQ_OK;
}

int32_t matmul(hq::Kind kind, void *xout, const void *xq, const void *xs, const void *wq, const void *ws,
               const void *wc, int32_t n, int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame,
               int32_t three, void *stream) {
  g_error = HQ_OK;
  hq::Job j{(char *)xout, (const char *)xq, (const char *)xs, (const char *)wq, (const char *)ws,
            relaxed(kind) ? (const char *)wc : nullptr, n, r0, r1, count, os, frame, frame};
  if (int32_t st = check_job(kind, j, three)) return st;
  if (j.r1 == j.r0 || j.count == 0) return HQ_OK;
  if (int32_t st = ensure_device()) return st;
  return run_jobs(kind, {j}, stream_of(stream));
}

int32_t matmul_blocks(hq::Kind kind, void *xout, const void *xq, const void *xs, const void *w, const void *tab,
                      int32_t n, int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame, int32_t type,
                      void *stream) {
  g_error = HQ_OK;
  hq::Job j{(char *)xout, (const char *)xq, (const char *)xs, (const char *)w, (const char *)tab, nullptr, n, r0, r1,
            count, os, frame, frame, type};
  if (int32_t st = check_job(kind, j, 0)) return st;
  if (j.r1 == j.r0 || j.count == 0) return HQ_OK;
  if (int32_t st = ensure_device()) return st;
  return run_jobs(kind, {j}, stream_of(stream));
}

// a host list of channel numbers (each below dim) as the kernels take it
int32_t channels_of(const char *who, const int32_t *channels, int32_t count, int32_t dim, hq::Channels &ch) {
  if (count < 0 || count > hq::kMaxChannels)
    return fail(HQ_ERR_ARGUMENT, "%s: %d channels (at most %d)", who, count, hq::kMaxChannels);
  if (count && !channels) return fail(HQ_ERR_NULL, "%s: channels NULL", who);
  ch.count = count;
  for (int32_t i = 0; i < count; i++) {
    if (channels[i] < 0 || channels[i] >= dim)
      return fail(HQ_ERR_ARGUMENT, "%s: channel %d is not below %d", who, channels[i], dim);
    ch.c[i] = channels[i];
  }
  return HQ_OK;
}
// the weights a scale is of (dtypes.py: int8's group32, int6's 32, ternary's and binary's 128)
int32_t group_of(int32_t packing, int32_t dim) {
  if (packing == hq::kPackTernary || packing == hq::kPackBinary) return 128;
  if (packing == hq::kPackInt6) return 32;
  int32_t size = 32;
  while (size > 1 && dim % size) size >>= 1;
  return size;
}
}  // namespace

extern "C" {

const char *hq_version(void) { return "hq 1.0 gfx950"; }

int32_t hq_job_path(int32_t kind, int32_t n, int32_t count, int64_t frame, int64_t sframe) {
  g_error = HQ_OK;
  if (kind < 0 || kind >= kKinds || kind_name((hq::Kind)kind)[0] == '?')
    return fail(HQ_ERR_KIND, "hq_job_path: kind %d is not run here", kind), -1;
  hq::Job j{};
  j.n = n, j.count = count, j.frame = frame, j.sframe = sframe;
  return path_of((hq::Kind)kind, j);
}

int32_t hq_init(void) {
  g_error = HQ_OK;
  if (int32_t st = ensure_device()) return st;
  char *staging = nullptr;  // hq_matmuls_static's staging on this device, looked up now (outside any capture)
  return scratch_of(&staging);
}

int32_t hq_set_stream(void *stream) {
  g_stream.store(stream);
  return HQ_OK;
}

void *hq_get_stream(void) { return g_stream.load(); }

int32_t hq_synchronize(void) {
  return hip_status(hipStreamSynchronize(stream_of(g_stream.load())), "hipStreamSynchronize");
}

int32_t hq_last_error(void) { return g_error; }
const char *hq_last_error_message(void) { return g_error ? g_message : ""; }
void hq_clear_error(void) {
  g_error = HQ_OK;
  g_message[0] = 0;
}

// ---- activations and corrections -----------------------------------------------------------------------------
int32_t hq_quantize_x_batch(void *xq, void *xs, const void *x, int32_t n, int32_t bias, int32_t count, int32_t frame,
                            int32_t x_stride, void *stream) {
  g_error = HQ_OK;
  if (n <= 0 || n % 32) return fail(HQ_ERR_ARGUMENT, "quantize_x: n = %d is not a positive multiple of 32", n);
  if (count < 0) return fail(HQ_ERR_ARGUMENT, "quantize_x: count = %d", count);
  if (count == 0) return HQ_OK;
  if (!xq || !xs || !x) return fail(HQ_ERR_NULL, "quantize_x: a NULL pointer");
  if (!aligned(xs, 4) || !aligned(x, 4)) return fail(HQ_ERR_ALIGNMENT, "quantize_x: xs or x not 4-byte aligned");
  if (count > 1 && (frame < 0 || frame % 4 || x_stride < 0 || x_stride % 4))
    return fail(HQ_ERR_ALIGNMENT, "quantize_x: frame or x_stride not a multiple of 4");
  if (int32_t st = ensure_device()) return st;
  return hip_status(hq::launch_quantize_x((char *)xq, (char *)xs, (const char *)x, n, bias, count, frame, x_stride,
                                          stream_of(stream)),
                    "quantize_x");
}

int32_t hq_quantize_x_ex(void *xq, void *xs, const void *x, int32_t n, int32_t bias, void *stream) {
  return hq_quantize_x_batch(xq, xs, x, n, bias, 1, 0, 0, stream);
}

int32_t hq_interleave_batch(void *xq, void *xs, int32_t n, int32_t count, int32_t frame, void *stream) {
  g_error = HQ_OK;
  if (n <= 0 || n % 64) return fail(HQ_ERR_ARGUMENT, "interleave: n = %d is not a positive multiple of 64", n);
  if (count < 0) return fail(HQ_ERR_ARGUMENT, "interleave: count = %d", count);
  if (count == 0) return HQ_OK;
  if (!xq || !xs) return fail(HQ_ERR_NULL, "interleave: a NULL pointer");
  if (!aligned(xq, 16) || !aligned(xs, 4)) return fail(HQ_ERR_ALIGNMENT, "interleave: xq not 16- or xs not 4-byte aligned");
  if (count > 1 && (frame < 0 || frame % 16)) return fail(HQ_ERR_ALIGNMENT, "interleave: frame not a multiple of 16");
  if (int32_t st = ensure_device()) return st;
  return hip_status(hq::launch_interleave((char *)xq, (char *)xs, n, count, frame, stream_of(stream)), "interleave");
}

int32_t hq_interleave_ex(void *xq, void *xs, int32_t n, void *stream) {
  return hq_interleave_batch(xq, xs, n, 1, 0, stream);
}

int32_t hq_int8_sums_ex(void *out, const void *w, int32_t groups, void *stream) {
  g_error = HQ_OK;
  if (groups < 0) return fail(HQ_ERR_ARGUMENT, "int8_sums: groups = %d", groups);
  if (groups == 0) return HQ_OK;
  if (!out || !w) return fail(HQ_ERR_NULL, "int8_sums: a NULL pointer");
  if (!aligned(w, 16) || !aligned(out, 4)) return fail(HQ_ERR_ALIGNMENT, "int8_sums: w not 16- or out not 4-byte aligned");
  if (int32_t st = ensure_device()) return st;
  return hip_status(hq::launch_int8_sums((int32_t *)out, (const char *)w, groups, stream_of(stream)), "int8_sums");
}

int32_t hq_six_sums_ex(void *out, const void *w, int32_t groups, void *stream) {
  g_error = HQ_OK;
  if (groups < 0) return fail(HQ_ERR_ARGUMENT, "six_sums: groups = %d", groups);
  if (groups == 0) return HQ_OK;
  if (!out || !w) return fail(HQ_ERR_NULL, "six_sums: a NULL pointer");
  if (!aligned(w, 8) || !aligned(out, 4)) return fail(HQ_ERR_ALIGNMENT, "six_sums: w not 8- or out not 4-byte aligned");
  if (int32_t st = ensure_device()) return st;
  return hip_status(hq::launch_six_sums((int32_t *)out, (const char *)w, groups, stream_of(stream)), "six_sums");
}

// ---- the products ---------------------------------------------------------------------------------------------
int32_t hq_matmul_q8r_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, const void *wc,
                         int32_t n, int32_t r0, int32_t r1, void *stream) {
  return matmul(hq::Q8R, xout, xq, xs, wq, ws, wc, n, r0, r1, 1, 0, 0, 3, stream);
}
int32_t hq_matmul_q8_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n,
                        int32_t r0, int32_t r1, void *stream) {
  return matmul(hq::Q8, xout, xq, xs, wq, ws, nullptr, n, r0, r1, 1, 0, 0, 3, stream);
}
int32_t hq_matmul_q8r_tile_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws,
                              const void *wc, int32_t n, int32_t r0, int32_t r1, int32_t count, int32_t os,
                              int32_t frame, void *stream) {
  return matmul(hq::Q8R, xout, xq, xs, wq, ws, wc, n, r0, r1, count, os, frame, 3, stream);
}
int32_t hq_tol_min_tiles(int32_t tiles) {
  g_error = HQ_OK;
  if (tiles < -1) return fail(HQ_ERR_ARGUMENT, "hq_tol_min_tiles: %d tiles", tiles);
  return g_tol_min_tiles.exchange(tiles);
}
int64_t hq_tol_work_bytes(int32_t n, int32_t count) {
  g_error = HQ_OK;
  if (n <= 0 || n % 32 || count < 0) return fail(HQ_ERR_ARGUMENT, "hq_tol_work_bytes: n = %d, count = %d", n, count), -1;
  return hq::tol_work_bytes(n, count);
}
int32_t hq_matmul_q8r_tile_tol_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws,
                                  int32_t n, int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame,
                                  void *work, int64_t work_bytes, void *stream) {
  g_error = HQ_OK;
  const char *name = "hq_matmul_q8r_tile_tol_ex";
  hq::Job j{(char *)xout, (const char *)xq, (const char *)xs, (const char *)wq, (const char *)ws, nullptr, n, r0, r1,
            count, os, frame, frame};
  if (int32_t st = check_job(hq::Q8R, j, 3)) return st;
  if (j.r1 == j.r0 || j.count == 0) return HQ_OK;
  if (!aligned(xs, 4) || !aligned(ws, 4)) return fail(HQ_ERR_ALIGNMENT, "%s: xs or ws not 4-byte aligned", name);
  if (!work) return fail(HQ_ERR_NULL, "%s: work is NULL", name);
  if (!aligned(work, 256)) return fail(HQ_ERR_ALIGNMENT, "%s: work not 256-byte aligned", name);
  const int64_t need = hq::tol_work_bytes(n, count);
  if (work_bytes < need)
    return fail(HQ_ERR_ARGUMENT, "%s: a workspace of %lld bytes (n = %d, %d tokens need %lld)", name,
                (long long)work_bytes, n, count, (long long)need);
  // a tile's loads keep 32-bit offsets from its first row and token: 128 rows of n bytes, 128 tokens of 2 n bytes,
  // and the scales' n / 32 groups x count words
  if ((int64_t)n * 256 >= ((int64_t)1 << 32) || (int64_t)(n / 32) * (count + 3) * 4 >= ((int64_t)1 << 32))
    return fail(HQ_ERR_ARGUMENT, "%s: n = %d with %d tokens is past the tiles' 32-bit offsets", name, n, count);
  if (int32_t st = ensure_device()) return st;
  // a launch of fewer tiles than the setting asks takes the bit-exact kernels (their numbers are the reference's)
  const int32_t least = g_tol_min_tiles.load();
  const int64_t min_tiles = least >= 0 ? least : 2 * (int64_t)hq::cu_count();
  if (hq::tol_tiles(j.r1 - j.r0, j.count) < min_tiles) return run_jobs(hq::Q8R, {j}, stream_of(stream));
  return hip_status(hq::launch_gemm_tol(j, (char *)work, stream_of(stream)), name);
}
int32_t hq_matmul_q6r_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, const void *wc,
                         int32_t n, int32_t r0, int32_t r1, void *stream) {
  return matmul(hq::Q6R, xout, xq, xs, wq, ws, wc, n, r0, r1, 1, 0, 0, 3, stream);
}
int32_t hq_matmul_q6_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n,
                        int32_t r0, int32_t r1, void *stream) {
  return matmul(hq::Q6, xout, xq, xs, wq, ws, nullptr, n, r0, r1, 1, 0, 0, 3, stream);
}
int32_t hq_matmul_t2r_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n,
                         int32_t r0, int32_t r1, int32_t three, void *stream) {
  return matmul(hq::T2R, xout, xq, xs, wq, ws, nullptr, n, r0, r1, 1, 0, 0, three, stream);
}
int32_t hq_matmul_t2r_tile_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n,
                              int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame, int32_t three,
                              void *stream) {
  return matmul(hq::T2R, xout, xq, xs, wq, ws, nullptr, n, r0, r1, count, os, frame, three, stream);
}
int32_t hq_matmul_b1r_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n,
                         int32_t r0, int32_t r1, int32_t two, void *stream) {
  return matmul(hq::B1R, xout, xq, xs, wq, ws, nullptr, n, r0, r1, 1, 0, 0, two, stream);
}
int32_t hq_matmul_b1r_tile_ex(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n,
                              int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame, int32_t two,
                              void *stream) {
  return matmul(hq::B1R, xout, xq, xs, wq, ws, nullptr, n, r0, r1, count, os, frame, two, stream);
}

// ---- llama.cpp's blocks (kernels/blocks/) -----------------------------------------------------------------------
int32_t hq_sb_tables_ex(void *area, const void *codebooks, void *stream) {
  g_error = HQ_OK;
  if (!area || !codebooks) return fail(HQ_ERR_NULL, "sb_tables: a NULL pointer");
  if (!aligned(area, 16)) return fail(HQ_ERR_ALIGNMENT, "sb_tables: the area not 16-byte aligned");
  if (int32_t st = ensure_device()) return st;
  return hip_status(hq::launch_sb_tables((uint8_t *)area, (const uint8_t *)codebooks, stream_of(stream)), "sb_tables");
}

int32_t hq_sums_x_batch(void *xs, const void *xq, int32_t n, int32_t count, int32_t frame, void *stream) {
  g_error = HQ_OK;
  if (n <= 0 || n % 32) return fail(HQ_ERR_ARGUMENT, "sums_x: n = %d is not a positive multiple of 32", n);
  if (count < 0) return fail(HQ_ERR_ARGUMENT, "sums_x: count = %d", count);
  if (count == 0) return HQ_OK;
  if (!xs || !xq) return fail(HQ_ERR_NULL, "sums_x: a NULL pointer");
  if (!aligned(xs, 4)) return fail(HQ_ERR_ALIGNMENT, "sums_x: xs not 4-byte aligned");
  if (count > 1 && (frame < 0 || frame % 4)) return fail(HQ_ERR_ALIGNMENT, "sums_x: frame not a multiple of 4");
  if (int32_t st = ensure_device()) return st;
  return hip_status(hq::launch_sums_x((char *)xs, (const char *)xq, n, count, frame, stream_of(stream)), "sums_x");
}

int32_t hq_matmul_sbr_ex(void *xout, const void *xq, const void *xs, const void *w, const void *tab, int32_t n,
                         int32_t r0, int32_t r1, int32_t type, void *stream) {
  return matmul_blocks(hq::SBR, xout, xq, xs, w, tab, n, r0, r1, 1, 0, 0, type, stream);
}
int32_t hq_matmul_sbr_tile_ex(void *xout, const void *xq, const void *xs, const void *w, const void *tab, int32_t n,
                              int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame, int32_t type,
                              void *stream) {
  return matmul_blocks(hq::SBR, xout, xq, xs, w, tab, n, r0, r1, count, os, frame, type, stream);
}

int32_t hq_sb_row_ex(void *out, const void *w, const void *tab, int32_t n, int32_t type, void *stream) {
  g_error = HQ_OK;
  if (!hq::sb_block_bytes(type)) return fail(HQ_ERR_ARGUMENT, "sb_row: type %d is not one of the ten block types", type);
  if (n < 0 || n % 256) return fail(HQ_ERR_ARGUMENT, "sb_row: n = %d is not a multiple of 256", n);
  if (n == 0) return HQ_OK;
  if (!out || !w || !tab) return fail(HQ_ERR_NULL, "sb_row: a NULL pointer");
  if (!aligned(out, 16) || !aligned(w, 2) || !aligned(tab, 16))
    return fail(HQ_ERR_ALIGNMENT, "sb_row: out or the tables not 16-, or w not 2-byte aligned");
  if (int32_t st = ensure_device()) return st;
  return hip_status(hq::launch_sb_row((float *)out, (const char *)w, (const uint8_t *)tab, n, type, stream_of(stream)),
                    "sb_row");
}

// ---- the classifier's outlier channels (tensors.ts:170-187, engine.ts:459-466, matmul.ts:246-266) --------------
int32_t hq_add_columns_ex(void *y, const void *rows, const void *a, int32_t count, int32_t n, void *stream) {
  g_error = HQ_OK;
  if (n < 0 || count < 0) return fail(HQ_ERR_ARGUMENT, "add_columns: count = %d, n = %d", count, n);
  if (n == 0 || count == 0) return HQ_OK;
  if (!y || !rows || !a) return fail(HQ_ERR_NULL, "add_columns: a NULL pointer");
  if (!aligned(y, 4) || !aligned(rows, 4) || !aligned(a, 4))
    return fail(HQ_ERR_ALIGNMENT, "add_columns: y, rows or a not 4-byte aligned");
  if (int32_t st = ensure_device()) return st;
  return hip_status(hq::launch_add_columns((float *)y, (const float *)rows, (const float *)a, count, n,
                                           stream_of(stream)),
                    "add_columns");
}

int32_t hq_outlier_columns_ex(void *columns, const void *values, const void *scales, int32_t packing,
                              const int32_t *channels, int32_t count, int32_t vocab, int32_t dim, void *stream) {
  g_error = HQ_OK;
  if (packing < hq::kPackInt8 || packing > hq::kPackBinary)
    return fail(HQ_ERR_ARGUMENT, "outlier_columns: packing %d is none of int8, int6, ternary, binary", packing);
  if (vocab < 0 || dim <= 0) return fail(HQ_ERR_ARGUMENT, "outlier_columns: vocab = %d, dim = %d", vocab, dim);
  const int32_t group = group_of(packing, dim);
  if (dim % group) return fail(HQ_ERR_ARGUMENT, "outlier_columns: dim = %d is not whole groups of %d", dim, group);
  hq::Channels ch{};
  if (int32_t st = channels_of("outlier_columns", channels, count, dim, ch)) return st;
  if (count == 0 || vocab == 0) return HQ_OK;
  if (!columns || !values || !scales) return fail(HQ_ERR_NULL, "outlier_columns: a NULL pointer");
  const uintptr_t sa = (packing == hq::kPackTernary || packing == hq::kPackBinary) ? 2 : 4;
  if (!aligned(columns, 4) || !aligned(scales, sa))
    return fail(HQ_ERR_ALIGNMENT, "outlier_columns: columns not 4-, or scales not %d-byte aligned", (int)sa);
  if (int32_t st = ensure_device()) return st;
  return hip_status(hq::launch_outlier_columns((float *)columns, (const uint8_t *)values, (const uint8_t *)scales,
                                               packing, ch, vocab, dim, group, stream_of(stream)),
                    "outlier_columns");
}

int32_t hq_take_channels_ex(void *picked, void *x, const int32_t *channels, int32_t count, void *stream) {
  g_error = HQ_OK;
  hq::Channels ch{};
  if (int32_t st = channels_of("take_channels", channels, count, INT32_MAX, ch)) return st;
  if (count == 0) return HQ_OK;
  if (!picked || !x) return fail(HQ_ERR_NULL, "take_channels: a NULL pointer");
  if (!aligned(picked, 4) || !aligned(x, 4)) return fail(HQ_ERR_ALIGNMENT, "take_channels: picked or x not 4-byte aligned");
  if (int32_t st = ensure_device()) return st;
  return hip_status(hq::launch_take_channels((float *)picked, (float *)x, ch, stream_of(stream)), "take_channels");
}

// ---- binary weights from float32 (kernels/kernel/quantize.ts:232-247) -------------------------------------------
int32_t hq_quantize6_x_ex(void *out, void *xs, const void *x, int32_t n, void *stream) {
  g_error = HQ_OK;
  if (n < 0 || n % 32) return fail(HQ_ERR_ARGUMENT, "quantize6_x: n = %d is not a multiple of 32", n);
  if (n == 0) return HQ_OK;
  if (!out || !xs || !x) return fail(HQ_ERR_NULL, "quantize6_x: a NULL pointer");
  if (!aligned(x, 4) || !aligned(xs, 4)) return fail(HQ_ERR_ALIGNMENT, "quantize6_x: x or xs not 4-byte aligned");
  if (int32_t st = ensure_device()) return st;
  return hip_status(hq::launch_quantize6_x((uint8_t *)out, (float *)xs, (const float *)x, n / 32, stream_of(stream)),
                    "quantize6_x");
}

int32_t hq_ternary_x_ex(void *out, void *xs, const void *x, int32_t n, void *bad, void *stream) {
  g_error = HQ_OK;
  if (n < 0 || n % 128) return fail(HQ_ERR_ARGUMENT, "ternary_x: n = %d is not a multiple of 128", n);
  if (n == 0) return HQ_OK;
  if (!out || !xs || !x) return fail(HQ_ERR_NULL, "ternary_x: a NULL pointer");
  if (!aligned(x, 16) || !aligned(xs, 4) || (bad && !aligned(bad, 4)))
    return fail(HQ_ERR_ALIGNMENT, "ternary_x: x not 16-, xs or bad not 4-byte aligned");
  if (int32_t st = ensure_device()) return st;
  return hip_status(hq::launch_ternary_x((uint8_t *)out, (float *)xs, (const float *)x, n / 128, (int32_t *)bad,
                                         stream_of(stream)),
                    "ternary_x");
}

int32_t hq_binary_x_ex(void *out, void *xs, const void *x, int32_t n, void *bad, void *stream) {
  g_error = HQ_OK;
  if (n < 0 || n % 128) return fail(HQ_ERR_ARGUMENT, "binary_x: n = %d is not a multiple of 128", n);
  if (n == 0) return HQ_OK;
  if (!out || !xs || !x) return fail(HQ_ERR_NULL, "binary_x: a NULL pointer");
  if (!aligned(x, 16) || !aligned(xs, 4) || (bad && !aligned(bad, 4)))
    return fail(HQ_ERR_ALIGNMENT, "binary_x: x not 16-, xs or bad not 4-byte aligned");
  if (int32_t st = ensure_device()) return st;
  return hip_status(hq::launch_binary_x((uint8_t *)out, (float *)xs, (const float *)x, n / 128, (int32_t *)bad,
                                        stream_of(stream)),
                    "binary_x");
}

// ---- a phase of jobs in the reference's table form ------------------------------------------------------------
}  // extern "C"

namespace {

// [kind, out, a, b, a4, a5, a6, a7, a8, rows, count, os, as, bs] (src/runtime/jobs.ts:46, 207-333) -> a Job
// the frame of a token's readied activations in a staging area: n bytes, then the largest scale area a kind reads
// (llama.cpp's blocks: n/8 of scales, n/8 of sums of 16, n/4 of sums of 8), each from a 256-byte boundary
int64_t staging_bytes_of(int32_t n) { return ((int64_t)n + 255) & ~(int64_t)255; }
int64_t staging_frame(int32_t n) { return staging_bytes_of(n) + (((int64_t)n / 2 + 255) & ~(int64_t)255); }

// staging (not NULL): every job's a / b are the staging's (its tokens staging_frame(n) apart) and the table's a, b,
// as and bs are not read
int32_t parse_jobs(const double *jobs, int32_t count, int32_t stride, std::vector<hq::Job> by_kind[kKinds],
                   const char *who, const char *staging = nullptr) {
  if (count < 0 || (count > 0 && (!jobs || stride < 14)))
    return fail(HQ_ERR_ARGUMENT, "%s: count %d, stride %d (a job has 14 numbers at least)", who, count, stride);
  for (int32_t i = 0; i < count; i++) {
    const double *e = jobs + (int64_t)i * stride;
    for (int q = 0; q < 14; q++) {
      if (!(e[q] >= 0.0 && e[q] < 9007199254740992.0 && e[q] == std::floor(e[q])))
        return fail(HQ_ERR_ARGUMENT, "%s: job %d's number %d (%g) is not an address or count", who, i, q, e[q]);
    }
    const int32_t kind = (int32_t)e[0];
    auto at = [&](int q) { return (const char *)(uintptr_t)(uint64_t)e[q]; };
    hq::Job j{(char *)at(1), at(2), at(3), at(4), at(5), nullptr, (int32_t)e[7], 0, (int32_t)e[9], (int32_t)e[10],
              (int64_t)e[11], (int64_t)e[12], (int64_t)e[13]};
    hq::Kind k;
    switch (kind) {
    case hq::Q8R: k = hq::Q8R; j.wc = at(6); j.sframe = j.count > 1 ? j.frame : j.sframe; break;  // its tile
    case hq::Q8: k = hq::Q8; break;
    case hq::Q6R: k = hq::Q6R; j.wc = at(6); break;
    case hq::Q6: k = hq::Q6; break;
    case hq::T2R: k = hq::T2R; j.sframe = j.count > 1 ? j.frame : j.sframe; break;  // its tile
    case hq::T2: k = hq::T2; break;
    case hq::B1R: k = hq::B1R; j.sframe = j.count > 1 ? j.frame : j.sframe; break;  // its tile
    case hq::B1: k = hq::B1; break;
    case hq::SBR:
    case hq::SBW:  // their tiles take a prompt's tokens a frame apart (jobs.ts:206, 297-301)
      k = (hq::Kind)kind;
      j.type = (int32_t)e[6];
      j.sframe = j.count > 1 ? j.frame : j.sframe;
      break;
    case hq::SB: k = hq::SB; j.type = (int32_t)e[6]; break;
    default: return fail(HQ_ERR_KIND, "%s: job %d is of kind %d, which this library does not run", who, i, kind);
    }
    if (staging) {
      j.xq = staging, j.xs = staging + staging_bytes_of(j.n > 0 ? j.n : 0);
      j.frame = j.sframe = staging_frame(j.n > 0 ? j.n : 0);
    }
    if (int32_t st = check_job(k, j, hq::binary_kind(k) ? 2 : 3)) return st;
    by_kind[kind].push_back(j);
  }
  return HQ_OK;
}

// ready() of `tokens` tokens of one input into xq / xs (frame bytes apart) as a job of `kind` takes them: quantize_x
// at the kind's bias, then interleave for ternary and binary, sums_x for llama.cpp's blocks (jobs.ts:376-395,
// 421-424)
int32_t ready_acts(hq::Kind k, char *xq, char *xs, const char *x, int32_t n, int32_t tokens, int64_t frame,
                   int64_t x_stride, hipStream_t s) {
  const int32_t bias = relaxed(k) ? 64 : 0;
  if (int32_t st = hip_status(hq::launch_quantize_x(xq, xs, x, n, bias, tokens, frame, x_stride, s), "quantize_x"))
    return st;
  if (ternary(k))
    if (int32_t st = hip_status(hq::launch_interleave(xq, xs, n, tokens, frame, s), "interleave")) return st;
  if (hq::blocks_kind(k))
    if (int32_t st = hip_status(hq::launch_sums_x(xs, xq, n, tokens, frame, s), "sums_x")) return st;
  return HQ_OK;
}

// matmulsAlike (src/runtime/forward/engine.ts:398-407): a kind at a time, the input readied as that kind's jobs take
// it, then those jobs run as hq_phase runs them.  staging NULL: into the jobs' own a / b (a pair several jobs share
// readied once); else into staging (every job's a / b replaced by it, its tokens `frame` bytes apart), kind after
// kind in stream order.  A job of no rows computes nothing and takes no part: check_job passes it without looking
// at its pointers, so its a / b are never written.
int32_t matmuls_alike(const void *x, int32_t x_stride, std::vector<hq::Job> by_kind[kKinds], char *staging,
                      int64_t staging_bytes, hipStream_t s, const char *who) {
  for (int kind = 0; kind < kKinds; kind++) {
    auto &list = by_kind[kind];
    list.erase(std::remove_if(list.begin(), list.end(), [](const hq::Job &j) { return j.r1 == j.r0; }), list.end());
  }
  // one input: every job of one n and one token count
  int32_t n = -1, tokens = -1;
  for (int kind = 0; kind < kKinds; kind++)
    for (const hq::Job &j : by_kind[kind]) {
      if (n < 0) n = j.n, tokens = j.count;
      if (j.n != n || j.count != tokens)
        return fail(HQ_ERR_ARGUMENT, "%s: the jobs take one input (n %d and %d tokens, and %d, %d)", who, n, tokens,
                    j.n, j.count);
      // the readied activations of a token are one frame apart, bytes and scales alike (the reference's S)
      if (!staging && tokens > 1 && j.frame != j.sframe)
        return fail(HQ_ERR_ARGUMENT, "%s: a job's a and b advance by %lld and %lld bytes a token (one frame)", who,
                    (long long)j.frame, (long long)j.sframe);
    }
  if (n < 0 || tokens == 0) return HQ_OK;
  if (!x) return fail(HQ_ERR_NULL, "%s: x is NULL", who);
  if (!aligned(x, 16) || (tokens > 1 && (x_stride < 0 || x_stride % 16)))
    return fail(HQ_ERR_ALIGNMENT, "%s: x or x_stride not 16-byte aligned", who);
  const int64_t qbytes = staging_bytes_of(n), frame = staging_frame(n);
  if (staging && (int64_t)tokens * frame > staging_bytes)
    return fail(HQ_ERR_ARGUMENT, "%s: %d tokens of %d activations take %lld bytes of staging (at most %lld)", who,
                tokens, n, (long long)(tokens * frame), (long long)staging_bytes);
  if (int32_t st = ensure_device()) return st;
  for (int kind = 0; kind < kKinds; kind++) {
    auto &list = by_kind[kind];
    if (list.empty()) continue;
    const hq::Kind k = (hq::Kind)kind;
    if (staging) {
      if (int32_t st = ready_acts(k, staging, staging + qbytes, (const char *)x, n, tokens, frame, x_stride, s))
        return st;
      for (hq::Job &j : list) j.xq = staging, j.xs = staging + qbytes, j.frame = frame, j.sframe = frame;
    } else {
      for (size_t i = 0; i < list.size(); i++) {
        const hq::Job &j = list[i];
        bool seen = false;
        for (size_t e = 0; e < i && !seen; e++) seen = list[e].xq == j.xq && list[e].xs == j.xs && list[e].frame == j.frame;
        if (seen) continue;
        if (int32_t st = ready_acts(k, (char *)j.xq, (char *)j.xs, (const char *)x, n, tokens, j.frame, x_stride, s))
          return st;
      }
    }
    if (int32_t st = run_jobs(k, list, s)) return st;
  }
  return HQ_OK;
}

}  // namespace

extern "C" {

int32_t hq_phase(const double *jobs, int32_t count, int32_t stride, void *stream) {
  g_error = HQ_OK;
  std::vector<hq::Job> by_kind[kKinds];
  if (int32_t st = parse_jobs(jobs, count, stride, by_kind, "hq_phase")) return st;
  if (count > 0) {
    if (int32_t st = ensure_device()) return st;
  }
  for (int kind = 0; kind < kKinds; kind++) {
    if (by_kind[kind].empty()) continue;
    if (int32_t st = run_jobs((hq::Kind)kind, by_kind[kind], stream_of(stream))) return st;
  }
  return HQ_OK;
}

int32_t hq_matmuls(const void *x, int32_t x_stride, const double *jobs, int32_t count, int32_t stride, void *stream) {
  g_error = HQ_OK;
  std::vector<hq::Job> by_kind[kKinds];
  if (int32_t st = parse_jobs(jobs, count, stride, by_kind, "hq_matmuls")) return st;
  return matmuls_alike(x, x_stride, by_kind, nullptr, 0, stream_of(stream), "hq_matmuls");
}

int32_t hq_matmuls_static(const void *x, int32_t x_stride, const double *jobs, int32_t count, int32_t stride,
                          void *stream) {
  g_error = HQ_OK;
  std::vector<hq::Job> by_kind[kKinds];
  // parsed against a stand-in (the staging's device address is looked up below, after the host checks)
  char *const stand_in = (char *)(uintptr_t)4096;
  if (int32_t st = parse_jobs(jobs, count, stride, by_kind, "hq_matmuls_static", stand_in)) return st;
  for (auto &list : by_kind)
    for (const hq::Job &j : list)
      if ((int64_t)j.count * staging_frame(j.n) > kStagingBytes)
        return fail(HQ_ERR_ARGUMENT, "hq_matmuls_static: %d tokens of %d activations take %lld bytes of staging (at "
                    "most %lld)", j.count, j.n, (long long)(j.count * staging_frame(j.n)), (long long)kStagingBytes);
  bool work = false;  // jobs of no rows or no tokens compute nothing: with only those, no device is needed
  for (auto &list : by_kind)
    for (const hq::Job &j : list) work = work || (j.r1 > j.r0 && j.count > 0);
  if (!work) return HQ_OK;
  char *staging = nullptr;
  if (int32_t st = scratch_of(&staging)) return st;
  return matmuls_alike(x, x_stride, by_kind, staging, kStagingBytes, stream_of(stream), "hq_matmuls_static");
}

// ---- the ceilings ---------------------------------------------------------------------------------------------
int32_t hq_ceiling_read(const void *p, int64_t bytes, void *sink, void *stream) {
  g_error = HQ_OK;
  if (bytes <= 0 || bytes % 16) return fail(HQ_ERR_ARGUMENT, "hq_ceiling_read: bytes = %lld", (long long)bytes);
  if (!p || !sink) return fail(HQ_ERR_NULL, "hq_ceiling_read: a NULL pointer");
  if (!aligned(p, 16) || !aligned(sink, 4)) return fail(HQ_ERR_ALIGNMENT, "hq_ceiling_read: misaligned");
  if (int32_t st = ensure_device()) return st;
  return hip_status(hq::launch_ceiling_read((const char *)p, bytes, (uint32_t *)sink, stream_of(stream)), "ceiling_read");
}

int32_t hq_ceiling_mfma(int32_t blocks, int32_t iterations, void *sink, void *stream) {
  g_error = HQ_OK;
  if (blocks <= 0 || iterations <= 0) return fail(HQ_ERR_ARGUMENT, "hq_ceiling_mfma: %d blocks, %d iterations", blocks, iterations);
  if (!sink || !aligned(sink, 4)) return fail(HQ_ERR_NULL, "hq_ceiling_mfma: sink");
  if (int32_t st = ensure_device()) return st;
  return hip_status(hq::launch_ceiling_mfma(blocks, iterations, (int32_t *)sink, stream_of(stream)), "ceiling_mfma");
}

int32_t hq_ceiling_epilogue(int32_t form, int32_t blocks, int32_t iterations, void *sink, void *stream) {
  g_error = HQ_OK;
  if (form < 0 || form > 1 || blocks <= 0 || iterations <= 0)
    return fail(HQ_ERR_ARGUMENT, "hq_ceiling_epilogue: form %d, %d blocks, %d iterations", form, blocks, iterations);
  if (!sink || !aligned(sink, 4)) return fail(HQ_ERR_NULL, "hq_ceiling_epilogue: sink");
  if (int32_t st = ensure_device()) return st;
  return hip_status(hq::launch_ceiling_epilogue(form, blocks, iterations, (int32_t *)sink, stream_of(stream)),
                    "ceiling_epilogue");
}

// ---- the drop-in names: the library's stream, errors kept for hq_last_error() ---------------------------------
void quantize_x(void *xq, void *xs, const void *x, int32_t n, int32_t bias) {
  hq_quantize_x_ex(xq, xs, x, n, bias, g_stream.load());
}
void int8_sums(void *out, const void *w, int32_t groups) { hq_int8_sums_ex(out, w, groups, g_stream.load()); }
void six_sums(void *out, const void *w, int32_t groups) { hq_six_sums_ex(out, w, groups, g_stream.load()); }
void interleave(void *xq, void *xs, int32_t n) { hq_interleave_ex(xq, xs, n, g_stream.load()); }
void matmul_q8r(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, const void *wc, int32_t n,
                int32_t r0, int32_t r1) {
  hq_matmul_q8r_ex(xout, xq, xs, wq, ws, wc, n, r0, r1, g_stream.load());
}
void matmul_q8(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n, int32_t r0,
               int32_t r1) {
  hq_matmul_q8_ex(xout, xq, xs, wq, ws, n, r0, r1, g_stream.load());
}
void matmul_q8r_tile(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, const void *wc,
                     int32_t n, int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame) {
  hq_matmul_q8r_tile_ex(xout, xq, xs, wq, ws, wc, n, r0, r1, count, os, frame, g_stream.load());
}
void matmul_q6r(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, const void *wc, int32_t n,
                int32_t r0, int32_t r1) {
  hq_matmul_q6r_ex(xout, xq, xs, wq, ws, wc, n, r0, r1, g_stream.load());
}
void matmul_q6(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n, int32_t r0,
               int32_t r1) {
  hq_matmul_q6_ex(xout, xq, xs, wq, ws, n, r0, r1, g_stream.load());
}
void matmul_t2r(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n, int32_t r0,
                int32_t r1, int32_t three) {
  hq_matmul_t2r_ex(xout, xq, xs, wq, ws, n, r0, r1, three, g_stream.load());
}
void matmul_t2(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n, int32_t r0,
               int32_t r1, int32_t three) {
  matmul(hq::T2, xout, xq, xs, wq, ws, nullptr, n, r0, r1, 1, 0, 0, three, g_stream.load());
}
void matmul_t2r_tile(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n,
                     int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame, int32_t three) {
  hq_matmul_t2r_tile_ex(xout, xq, xs, wq, ws, n, r0, r1, count, os, frame, three, g_stream.load());
}
void matmul_b1r(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n, int32_t r0,
                int32_t r1, int32_t two) {
  hq_matmul_b1r_ex(xout, xq, xs, wq, ws, n, r0, r1, two, g_stream.load());
}
void matmul_b1(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n, int32_t r0,
               int32_t r1, int32_t two) {
  matmul(hq::B1, xout, xq, xs, wq, ws, nullptr, n, r0, r1, 1, 0, 0, two, g_stream.load());
}
void matmul_b1r_tile(void *xout, const void *xq, const void *xs, const void *wq, const void *ws, int32_t n,
                     int32_t r0, int32_t r1, int32_t count, int32_t os, int32_t frame, int32_t two) {
  hq_matmul_b1r_tile_ex(xout, xq, xs, wq, ws, n, r0, r1, count, os, frame, two, g_stream.load());
}
int32_t sb_tables(void *area, const void *codebooks) {
  hq_sb_tables_ex(area, codebooks, g_stream.load());
  return hq::kSbTables;
}
void sums_x(void *xs, const void *xq, int32_t n) { hq_sums_x_batch(xs, xq, n, 1, 0, g_stream.load()); }
void matmul_sbr(void *xout, const void *xq, const void *xs, const void *w, const void *tab, int32_t n, int32_t r0,
                int32_t r1, int32_t type) {
  hq_matmul_sbr_ex(xout, xq, xs, w, tab, n, r0, r1, type, g_stream.load());
}
void matmul_sb(void *xout, const void *xq, const void *xs, const void *w, const void *tab, int32_t n, int32_t r0,
               int32_t r1, int32_t type) {
  matmul_blocks(hq::SB, xout, xq, xs, w, tab, n, r0, r1, 1, 0, 0, type, g_stream.load());
}
void matmul_sbr_tile(void *xout, const void *xq, const void *xs, const void *w, const void *tab, int32_t n, int32_t r0,
                     int32_t r1, int32_t count, int32_t os, int32_t frame, int32_t type) {
  hq_matmul_sbr_tile_ex(xout, xq, xs, w, tab, n, r0, r1, count, os, frame, type, g_stream.load());
}
// the reference's tile for engines whose dot product multiplies signed by signed, with a scratch area of the
// caller's for a row spread once: the same numbers, and this library needs no scratch
void matmul_sbw_tile(void *xout, const void *xq, const void *xs, const void *w, const void *tab, int32_t n, int32_t r0,
                     int32_t r1, int32_t count, int32_t os, int32_t frame, int32_t type, void *scratch) {
  (void)scratch;
  matmul_blocks(hq::SBW, xout, xq, xs, w, tab, n, r0, r1, count, os, frame, type, g_stream.load());
}
void signed_dots(void *out, const void *a, const void *b) {
  g_error = HQ_OK;
  if (!out || !a || !b) {
    fail(HQ_ERR_NULL, "signed_dots: a NULL pointer");
    return;
  }
  if (!aligned(out, 4)) {
    fail(HQ_ERR_ALIGNMENT, "signed_dots: out not 4-byte aligned");
    return;
  }
  if (ensure_device()) return;
  hip_status(hq::launch_signed_dots((int32_t *)out, (const int8_t *)a, (const int8_t *)b, stream_of(g_stream.load())),
             "signed_dots");
}
void sb_row(void *out, const void *w, const void *tab, int32_t n, int32_t type) {
  hq_sb_row_ex(out, w, tab, n, type, g_stream.load());
}
void add_columns(void *y, const void *rows, const void *a, int32_t count, int32_t n) {
  hq_add_columns_ex(y, rows, a, count, n, g_stream.load());
}
// the reference's binary_x and ternary_x return their refusal: these wait for the library's stream to give it (a
// word of device memory the library keeps for them, one a device, cleared before each call); 1 also when the call
// fails (hq_last_error says why)
static int32_t refusal_of(const char *who, int32_t (*run)(void *, void *, const void *, int32_t, void *, void *), void *out,
                   void *xs, const void *x, int32_t n) {
  static std::mutex lock;
  static int32_t *word[64];
  std::lock_guard<std::mutex> hold(lock);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    fail(HQ_ERR_DEVICE, "%s: no device", who);
    return 1;
  }
  if (!word[dev] && hip_status(hipMalloc((void **)&word[dev], 4), "hipMalloc")) return 1;
  const hipStream_t s = stream_of(g_stream.load());
  if (hip_status(hipMemsetAsync(word[dev], 0, 4, s), "hipMemsetAsync")) return 1;
  if (run(out, xs, x, n, word[dev], s)) return 1;
  int32_t bad = 1;
  if (hip_status(hipMemcpyAsync(&bad, word[dev], 4, hipMemcpyDeviceToHost, s), "hipMemcpyAsync")) return 1;
  if (hip_status(hipStreamSynchronize(s), "hipStreamSynchronize")) return 1;
  return bad;
}
int32_t binary_x(void *out, void *xs, const void *x, int32_t n) {
  return refusal_of("binary_x", hq_binary_x_ex, out, xs, x, n);
}
int32_t ternary_x(void *out, void *xs, const void *x, int32_t n) {
  return refusal_of("ternary_x", hq_ternary_x_ex, out, xs, x, n);
}
void quantize6_x(void *out, void *xs, const void *x, int32_t n) { hq_quantize6_x_ex(out, xs, x, n, g_stream.load()); }

}  // extern "C"
