// fold.hpp — the order of the kinds whose reference lanes each take one part of every group (ternary, binary: part k
// of each group of 128; llama.cpp's blocks: lane k of each block of 256), for rows of L lanes, a group or block a
// lane a step: the lanes write their parts to LDS, and lane k (k < 4) of each row adds part k of the row's L groups
// in order.
#pragma once
#include "common.hpp"

namespace hq {

// rows of L lanes (64 / L rows a wave), two steps' parts (the lanes of a step write while the last step is read)
template <int T, int L>
struct FoldL {
  float v[2][64 / L][T][4][L];
};
template <int T, int L>
HQ_DEV void fold_step_l(const FoldL<T, L> &f, int buf, int slot, int lane, float acc[T]) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int k = lane & 3;
#pragma unroll
  for (int t = 0; t < T; t++) {
    const float4 *src = (const float4 *)f.v[buf][slot][t][k];
    float a = acc[t];
#pragma unroll
    for (int q = 0; q < L / 4; q++) {
      const float4 v = src[q];
      a = fadd(fadd(fadd(fadd(a, v.x), v.y), v.z), v.w);
    }
    acc[t] = a;
  }
}

}  // namespace hq
