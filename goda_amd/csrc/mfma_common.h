// Helpers shared by the matrix-core attention kernels (prefill forward and
// backward).
#pragma once

#include "common.h"

namespace goda {

template <typename T>
struct Vec;
template <>
struct Vec<bf16> {
  typedef bf16x8 v8;
  typedef bf16x4 v4;
};
template <>
struct Vec<f16> {
  typedef f16x8 v8;
  typedef f16x4 v4;
};
template <>
struct Vec<float> {
  typedef f32x8 v8;
  typedef f32x4 v4;
};
// Matrix instructions issued per mfma32() call (a 32x32 tile, 16 steps of K).
template <typename T>
constexpr int kMfmaPerStep = sizeof(T) == 4 ? 8 : 1;

// 32x32 MFMA accumulator layout (gfx9 family): lane l, register r holds row
// 8*(r/4) + 4*(l/32) + r%4, column l%32; the K dimension of the A and B
// operands is split the same way (lane half h holds k = 8h..8h+7 of each
// 16-step). So the 8 accumulator registers 8g..8g+7 of one column, packed,
// form a B (or A) operand whose k index p maps to accumulator row
// 16g + kPermKey(p): a transposed operand image built in that order (an
// "image" with its 16-row groups permuted by kPermKey) multiplies the packed
// registers directly, with no register shuffles.
__host__ __device__ constexpr int kPermKey(int p) { return 8 * ((p % 8) / 4) + 4 * (p / 8) + p % 4; }

// Workgroup barrier for the tile rings. __syncthreads() would also wait for
// every outstanding global access (vmcnt(0)), i.e. for the registers of the
// tile being prefetched; a ring only needs this wave's LDS accesses retired.
// The "memory" clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void ring_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

}  // namespace goda
