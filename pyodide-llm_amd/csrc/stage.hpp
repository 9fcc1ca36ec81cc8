// stage.hpp — what the matrix-core tiles (gemm.hip, gemm_tol.hip) share: buffer-to-LDS loads of a stage, the wait
// for a stage's loads, the XOR swizzle of 16-byte chunks in LDS, and the XCD-aware order of a launch's tiles.
#pragma once
#include "common.hpp"

namespace hq {

// ---- loads -----------------------------------------------------------------------------------------------------
// A block's rows, tokens and scales are each one buffer resource (common.hpp's resource(): base and size in scalar
// registers): a thread's offsets are set once, a stage moves them by a scalar offset, and a load past the size reads
// nothing and returns zeros (the tiles past the last row or token, the groups past the last one: their results are
// never stored).
// Direct loads into LDS: lane l's `size` bytes land at dst + size * l (dst the same in the whole wave; 2-byte loads
// land zero-extended in 4-byte slots).  The stage buffers are distinct __shared__ objects, so the compiler can tell
// that a load into one buffer does not write the one being read, and waits for these loads only where the stage
// barriers say so.  A generic address of LDS is the LDS offset in its low 32 bits: taken that way, not by an
// address-space cast (which tests for the null pointer), M0 is a constant for every load into a stage buffer.
#define HQ_LDS(p) ((__attribute__((address_space(3))) void *)(uintptr_t)(uint32_t)(uintptr_t)(p))
HQ_DEV void dma16(__amdgpu_buffer_rsrc_t r, void *dst, uint32_t vo, uint32_t so) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, HQ_LDS(dst), 16, vo, so, 0, 0);
}
HQ_DEV void dma4(__amdgpu_buffer_rsrc_t r, void *dst, uint32_t vo, uint32_t so) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, HQ_LDS(dst), 4, vo, so, 0, 0);
}
HQ_DEV void dma2(__amdgpu_buffer_rsrc_t r, void *dst, uint32_t vo, uint32_t so) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, HQ_LDS(dst), 2, vo, so, 0, 0);
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
// stage s of `total` loaded stages is ready, N loads a wave a stage, the loads of stages up to s + `ahead` issued
template <int N>
HQ_DEV void wait_for(int s, int total, int ahead) {
  const int later = min(ahead, total - 1 - s);
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

// the LDS address of p (a __shared__ object's byte)
HQ_DEV uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)p;
}

}  // namespace hq
