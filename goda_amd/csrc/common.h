// Device-side helpers shared by the attention kernels (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "goda_attn.h"

namespace goda {

typedef __bf16 bf16;
typedef _Float16 f16;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_huge_valf();

// ---- element type traits -------------------------------------------------
template <typename T>
struct Elem;

template <>
struct Elem<float> {
  static __device__ __forceinline__ float to_f32(float x) { return x; }
  static __device__ __forceinline__ float from_f32(float x) { return x; }
};

template <>
struct Elem<bf16> {
  static __device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
  static __device__ __forceinline__ bf16 from_f32(float x) { return (bf16)x; }
  typedef bf16x8 vec8;
  typedef bf16x4 vec4;
};

template <>
struct Elem<f16> {
  static __device__ __forceinline__ float to_f32(f16 x) { return (float)x; }
  static __device__ __forceinline__ f16 from_f32(float x) { return (f16)x; }
  typedef f16x8 vec8;
  typedef f16x4 vec4;
};

// 32x32x16 MFMA with fp32 accumulation on 8-element operands.
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
// fp32 operands: the same 32x32 tile and 16-step of K as the 16-bit forms,
// as eight v_mfma_f32_32x32x2_f32. Step e takes element e of each lane's
// chunk: lane half h holds k = 8h + e, so the k-to-(lane, element) mapping,
// and with it every operand image and packed-accumulator operand, is the
// one of the 16-bit forms.
__device__ __forceinline__ f32x16 mfma32(f32x8 a, f32x8 b, f32x16 c) {
#pragma unroll
  for (int e = 0; e < 8; ++e) c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], b[e], c, 0, 0, 0);
  return c;
}
// 16x16x32 MFMA with fp32 accumulation on 8-element operands.
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
// fp32: eight 16x16x4 products, element e of every lane's 8-element chunk
// feeding the e-th (the same assignment on both operands, so their dot
// product over the chunk is unchanged).
__device__ __forceinline__ f32x4 mfma16(f32x8 a, f32x8 b, f32x4 c) {
#pragma unroll
  for (int e = 0; e < 8; ++e) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[e], c, 0, 0, 0);
  return c;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

// Sum over aligned groups of N consecutive lanes (N a power of two <= 64).
template <int N>
__device__ __forceinline__ float lane_group_sum(float v) {
#pragma unroll
  for (int m = 1; m < N; m <<= 1) v += shfl_xor_f(v, m);
  return v;
}

// 16-byte and 8-byte vector memory helpers on raw element pointers.
template <typename V, typename T>
__device__ __forceinline__ V ld_vec(const T* p) {
  return *reinterpret_cast<const V*>(p);
}
template <typename V, typename T>
__device__ __forceinline__ void st_vec(T* p, V v) {
  *reinterpret_cast<V*>(p) = v;
}
// Loads of data a kernel reads exactly once (cached K/V rows in decode, the
// raw q/k/v/o/dO rows of the pre-pass kernels): nontemporal, so they stream
// without allocating in the caches. A streaming-read probe over 4 GiB read
// 6.9-7.0 TB/s this way against 6.2-6.3 TB/s with ordinary loads.
template <typename V, typename T>
__device__ __forceinline__ V ld_stream(const T* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const V*>(p));
}

// goda's RMSNorm (mint/nn/norm.py:17-27) of a row with sum of squares `ss`
// over `n` elements: x -> x * rms_scale(ss, n, eps) * (1 + w).
__device__ __forceinline__ float rms_scale(float ss, int n, float eps) { return rsqrtf(ss / (float)n + eps); }

// Four consecutive elements as fp32, and back.
template <typename T>
__device__ __forceinline__ void load4f(const T* p, float (&out)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) out[j] = Elem<T>::to_f32(p[j]);
}
template <>
__device__ __forceinline__ void load4f<float>(const float* p, float (&out)[4]) {
  const f32x4 v = ld_vec<f32x4>(p);
  out[0] = v[0];
  out[1] = v[1];
  out[2] = v[2];
  out[3] = v[3];
}
template <typename T>
__device__ __forceinline__ void store4f(T* p, const float (&v)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) p[j] = Elem<T>::from_f32(v[j]);
}
template <>
__device__ __forceinline__ void store4f<float>(float* p, const float (&v)[4]) {
  st_vec<f32x4>(p, f32x4{v[0], v[1], v[2], v[3]});
}

// Per-sequence geometry shared by every kernel: row offsets of sequence b in
// q/k storage and its query / key counts.
struct SeqGeom {
  int64_t q_row0;  // first query row (varlen) or 0
  int64_t k_row0;
  int lq, lk;
};

__device__ __forceinline__ SeqGeom seq_geom(int b, int seqlen_q, int seqlen_k,
                                            const int32_t* cu_q, const int32_t* cu_k,
                                            const int32_t* seqused_k) {
  SeqGeom g;
  if (cu_q) {
    g.q_row0 = cu_q[b];
    g.lq = cu_q[b + 1] - cu_q[b];
  } else {
    g.q_row0 = 0;
    g.lq = seqlen_q;
  }
  if (cu_k) {
    g.k_row0 = cu_k[b];
    g.lk = cu_k[b + 1] - cu_k[b];
  } else {
    g.k_row0 = 0;
    g.lk = seqlen_k;
  }
  // Device-side lengths are clamped to the rows the launch was sized for
  // (seqlen_q / seqlen_k, the maxima the host validated), so a bad value can
  // shrink the work but never move a read out of bounds.
  g.lq = max(0, min(g.lq, seqlen_q));
  g.lk = max(0, min(g.lk, seqlen_k));
  if (seqused_k) g.lk = max(0, min(seqused_k[b], g.lk));
  return g;
}

// RoPE position of query row i (0-based within its sequence; diag = Lk - Lq):
// rope_q_offset + diag + i, or rope_q_offset + i with rope_pos_abs (a
// caller-given start position), clamped into the table the host validated.
__device__ __forceinline__ int rope_qpos(const goda_prefill_args& a, int diag, int i) {
  return min(max(a.rope_q_offset + (a.rope_pos_abs ? 0 : diag) + i, 0), a.rope_len - 1);
}

// Row (b, query head h, query row i) of the bit-packed mask: bit j % 32 of
// word j / 32 is key j's visibility.
__device__ __forceinline__ const uint32_t* mask_row(const goda_prefill_args& a, int b, int h, int i) {
  return a.mask_bits + (int64_t)b * a.mask_stride_b + (int64_t)h * a.mask_stride_h + (int64_t)i * a.mask_stride_q;
}
__device__ __forceinline__ bool mask_bit(const uint32_t* row, int j) { return (row[j >> 5] >> (j & 31)) & 1u; }

// Bits lo..hi of a 32-bit word (0 when lo > hi; lo and hi may lie outside
// 0..31). Branch-free: 64-bit shifts by 0..32.
__device__ __forceinline__ uint32_t range_bits(int lo, int hi) {
  const int l = min(max(lo, 0), 32);
  const int h = min(max(hi, -1), 31) + 1;
  return (uint32_t)(~0ull << l) & ~(uint32_t)(~0ull << h);
}

// Keep `x` where the 1-bit field `bit` of `w` is set, else `repl`: one
// bit-field extract (0 or all ones) and one bit-field select, no compare.
__device__ __forceinline__ float keep_if_bit(float x, uint32_t w, int bit, float repl) {
  const uint32_t sel = (uint32_t)__builtin_amdgcn_sbfe((int)w, bit, 1);
  return __uint_as_float((__float_as_uint(x) & sel) | (__float_as_uint(repl) & ~sel));
}

}  // namespace goda
