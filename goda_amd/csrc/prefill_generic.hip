// Generic prefill attention on the vector ALUs, fp32 arithmetic throughout.
// The product path for fp32 at head_dim 256 (goda's default model dtype is
// fp32, mint/nn/models.py:23), whose operands do not fit the matrix-core
// kernel's register and LDS budgets; every other dtype / head_dim runs on
// prefill_mfma.hip.
//
// Work split: one workgroup of 256 threads per (64-query block, query head,
// sequence). Four threads share a query row; thread `part` owns head-dim
// elements {16*i + 4*part + j : j < 4}, so each thread holds D/4 values of the
// query row and of the output accumulator. Keys are staged 32 at a time in LDS
// as fp32 (RoPE applied while staging).

#include "common.h"
#include "launch.h"

namespace goda {
namespace {

constexpr int kRows = 64;   // query rows per workgroup
constexpr int kKeys = 32;   // keys per LDS tile
constexpr int kThreads = 256;

template <typename T>
__device__ __forceinline__ void load4(const T* p, float (&out)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) out[j] = Elem<T>::to_f32(p[j]);
}
template <>
__device__ __forceinline__ void load4<float>(const float* p, float (&out)[4]) {
  f32x4 v = ld_vec<f32x4>(p);
  out[0] = v[0];
  out[1] = v[1];
  out[2] = v[2];
  out[3] = v[3];
}

template <typename T, int D>
__global__ void __launch_bounds__(kThreads)
prefill_generic_kernel(const PrefillParams p) {
  const goda_prefill_args& a = p.a;
  constexpr int NPER = D / 4;      // elements per thread
  constexpr int NGRP = D / 16;     // groups of 4 per thread
  __shared__ float Ks[kKeys][D];
  __shared__ float Vs[kKeys][D];

  const int b = blockIdx.z;
  const int hq = blockIdx.y;
  const int hk = hq / p.group;
  const SeqGeom g = seq_geom(b, a.seqlen_q, a.seqlen_k, a.cu_seqlens_q, a.cu_seqlens_k,
                             a.seqused_k);
  const int q0 = blockIdx.x * kRows;
  if (q0 >= g.lq) return;

  const int tid = threadIdx.x;
  const int row = tid >> 2;
  const int part = tid & 3;
  const int i = q0 + row;             // query row within the sequence
  const bool row_valid = i < g.lq;
  const int diag = g.lk - g.lq;       // bottom-right alignment
  const bool use_window = a.window_left >= 0 && (a.causal || g.lq == 1);

  const T* qbase = reinterpret_cast<const T*>(a.q);
  const T* kbase = reinterpret_cast<const T*>(a.k);
  const T* vbase = reinterpret_cast<const T*>(a.v);
  const int64_t qb_off = a.cu_seqlens_q ? 0 : (int64_t)b * a.q_stride_b;
  const int64_t kb_off = a.cu_seqlens_k ? 0 : (int64_t)b * a.k_stride_b;
  const int64_t vb_off = a.cu_seqlens_k ? 0 : (int64_t)b * a.v_stride_b;

  // ---- query row (rotated) --------------------------------------------
  float q[NPER];
  if (row_valid) {
    const T* qrow = qbase + qb_off + (g.q_row0 + i) * a.q_stride_t + (int64_t)hq * a.q_stride_h;
#pragma unroll
    for (int gi = 0; gi < NGRP; ++gi) {
      float t4[4];
      load4<T>(qrow + 16 * gi + 4 * part, t4);
#pragma unroll
      for (int j = 0; j < 4; ++j) q[4 * gi + j] = t4[j];
    }
    if (a.q_norm_weight) {
      // Fused QK-RMSNorm over the row held by the 4 threads of the row.
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < NPER; ++e) ss = fmaf(q[e], q[e], ss);
      ss += shfl_xor_f(ss, 1);
      ss += shfl_xor_f(ss, 2);
      const float inv = rms_scale(ss, D, a.norm_eps);
#pragma unroll
      for (int gi = 0; gi < NGRP; ++gi)
#pragma unroll
        for (int j = 0; j < 4; ++j) q[4 * gi + j] *= inv * (1.f + a.q_norm_weight[16 * gi + 4 * part + j]);
    }
    if (a.rope_q) {
      const int pos = rope_qpos(a, diag, i);
      const float* cs = a.rope_cos + (int64_t)pos * (D / 2);
      const float* sn = a.rope_sin + (int64_t)pos * (D / 2);
#pragma unroll
      for (int gi = 0; gi < NGRP / 2; ++gi) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int f = 16 * gi + 4 * part + j;  // frequency index (< D/2)
          const float c = cs[f], s = sn[f];
          const float x1 = q[4 * gi + j], x2 = q[4 * (gi + NGRP / 2) + j];
          q[4 * gi + j] = x1 * c - x2 * s;
          q[4 * (gi + NGRP / 2) + j] = x1 * s + x2 * c;
        }
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < NPER; ++e) q[e] = 0.f;
  }

  const float slope_log2 = a.alibi_slopes ? a.alibi_slopes[hq] * kLog2e : 0.f;
  const int iabs = diag + i;  // absolute position of this query
  const uint32_t* mrow = a.mask_bits ? mask_row(a, b, hq, row_valid ? i : 0) : nullptr;

  // ---- key range of the workgroup ----------------------------------------
  const int i_last = min(q0 + kRows, g.lq) - 1;
  int kv_hi = g.lk;
  if (a.causal) kv_hi = min(kv_hi, diag + i_last + 1);
  int kv_lo = 0;
  if (use_window) kv_lo = max(0, diag + q0 - a.window_left);

  float o[NPER];
#pragma unroll
  for (int e = 0; e < NPER; ++e) o[e] = 0.f;
  float m = kNegInf, l = 0.f;

  for (int kv0 = (kv_lo / kKeys) * kKeys; kv0 < kv_hi; kv0 += kKeys) {
    __syncthreads();
    // Stage K (rotated) and V rows [kv0, kv0+kKeys) as fp32.
    constexpr int HALF4 = D / 8;  // 4-element groups in half a row
    for (int idx = tid; idx < kKeys * HALF4; idx += kThreads) {
      const int jr = idx / HALF4;
      const int c4 = (idx % HALF4) * 4;
      const int j = kv0 + jr;
      float k1[4] = {0.f, 0.f, 0.f, 0.f}, k2[4] = {0.f, 0.f, 0.f, 0.f};
      float v1[4] = {0.f, 0.f, 0.f, 0.f}, v2[4] = {0.f, 0.f, 0.f, 0.f};
      if (j < g.lk) {
        const T* krow = kbase + kb_off + (g.k_row0 + j) * a.k_stride_t + (int64_t)hk * a.k_stride_h;
        const T* vrow = vbase + vb_off + (g.k_row0 + j) * a.v_stride_t + (int64_t)hk * a.v_stride_h;
        load4<T>(krow + c4, k1);
        load4<T>(krow + c4 + D / 2, k2);
        load4<T>(vrow + c4, v1);
        load4<T>(vrow + c4 + D / 2, v2);
        if (a.rope_k && !a.k_norm_weight) {  // with the norm: rotated after it
          const int pos = a.rope_k_offset + j;
          const float* cs = a.rope_cos + (int64_t)pos * (D / 2) + c4;
          const float* sn = a.rope_sin + (int64_t)pos * (D / 2) + c4;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float x1 = k1[e], x2 = k2[e];
            k1[e] = x1 * cs[e] - x2 * sn[e];
            k2[e] = x1 * sn[e] + x2 * cs[e];
          }
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        Ks[jr][c4 + e] = k1[e];
        Ks[jr][c4 + D / 2 + e] = k2[e];
        Vs[jr][c4 + e] = v1[e];
        Vs[jr][c4 + D / 2 + e] = v2[e];
      }
    }
    if (a.k_norm_weight) {
      // Fused QK-RMSNorm of the staged key rows (staged unrotated on this
      // path), then their rotation: 8 threads per row.
      __syncthreads();
      const int jr = tid >> 3, p8 = tid & 7;
      float ss = 0.f;
      for (int d = p8; d < D; d += 8) ss = fmaf(Ks[jr][d], Ks[jr][d], ss);
      ss += shfl_xor_f(ss, 1);
      ss += shfl_xor_f(ss, 2);
      ss += shfl_xor_f(ss, 4);
      const float inv = rms_scale(ss, D, a.norm_eps);
      const int j = kv0 + jr;
      const int pos = a.rope_k_offset + j;
      for (int f = p8; f < D / 2; f += 8) {
        float x1 = Ks[jr][f] * inv * (1.f + a.k_norm_weight[f]);
        float x2 = Ks[jr][f + D / 2] * inv * (1.f + a.k_norm_weight[f + D / 2]);
        if (a.rope_k && j < g.lk) {
          const float c = a.rope_cos[(int64_t)pos * (D / 2) + f], sn = a.rope_sin[(int64_t)pos * (D / 2) + f];
          const float y1 = x1 * c - x2 * sn;
          x2 = x1 * sn + x2 * c;
          x1 = y1;
        }
        Ks[jr][f] = x1;
        Ks[jr][f + D / 2] = x2;
      }
    }
    __syncthreads();

    // Scores of this row against the tile (log2 domain, masked to -inf).
    float x[kKeys];
    float tmax = kNegInf;
#pragma unroll
    for (int jr = 0; jr < kKeys; ++jr) {
      float s = 0.f;
#pragma unroll
      for (int gi = 0; gi < NGRP; ++gi) {
        const f32x4 kv = ld_vec<f32x4>(&Ks[jr][16 * gi + 4 * part]);
        s = fmaf(q[4 * gi + 0], kv[0], s);
        s = fmaf(q[4 * gi + 1], kv[1], s);
        s = fmaf(q[4 * gi + 2], kv[2], s);
        s = fmaf(q[4 * gi + 3], kv[3], s);
      }
      s += shfl_xor_f(s, 1);
      s += shfl_xor_f(s, 2);
      const int j = kv0 + jr;
      bool vis = row_valid && j < g.lk && j >= kv_lo;
      if (a.causal) vis = vis && (j <= iabs);
      if (use_window) vis = vis && (iabs - j <= a.window_left);
      if (vis && mrow) vis = mask_bit(mrow, j);
      float t = s * p.scale_log2;
      if (a.alibi_slopes) t = fmaf(slope_log2, (float)(j - iabs), t);
      x[jr] = vis ? t : kNegInf;
      tmax = fmaxf(tmax, x[jr]);
    }
    const float m_new = fmaxf(m, tmax);
    const float m_use = (m_new == kNegInf) ? 0.f : m_new;
    const float alpha = exp2f(m - m_use);
    m = m_new;
    l *= alpha;
#pragma unroll
    for (int e = 0; e < NPER; ++e) o[e] *= alpha;
#pragma unroll
    for (int jr = 0; jr < kKeys; ++jr) {
      const float pj = exp2f(x[jr] - m_use);
      l += pj;
#pragma unroll
      for (int gi = 0; gi < NGRP; ++gi) {
        const f32x4 vv = ld_vec<f32x4>(&Vs[jr][16 * gi + 4 * part]);
        o[4 * gi + 0] = fmaf(pj, vv[0], o[4 * gi + 0]);
        o[4 * gi + 1] = fmaf(pj, vv[1], o[4 * gi + 1]);
        o[4 * gi + 2] = fmaf(pj, vv[2], o[4 * gi + 2]);
        o[4 * gi + 3] = fmaf(pj, vv[3], o[4 * gi + 3]);
      }
    }
  }

  if (!row_valid) return;
  const float inv = (l > 0.f) ? 1.f / l : 0.f;
  T* obase = reinterpret_cast<T*>(a.o);
  const int64_t ob_off = a.cu_seqlens_q ? 0 : (int64_t)b * a.o_stride_b;
  T* orow = obase + ob_off + (g.q_row0 + i) * a.o_stride_t + (int64_t)hq * a.o_stride_h;
#pragma unroll
  for (int gi = 0; gi < NGRP; ++gi) {
#pragma unroll
    for (int j = 0; j < 4; ++j) orow[16 * gi + 4 * part + j] = Elem<T>::from_f32(o[4 * gi + j] * inv);
  }
  if (a.lse && part == 0) {
    const float lse = (l > 0.f) ? (m + log2f(l)) * kLn2 : kNegInf;
    if (a.cu_seqlens_q)
      a.lse[(int64_t)hq * a.lse_stride_h + g.q_row0 + i] = lse;
    else
      a.lse[(int64_t)b * a.lse_stride_b + (int64_t)hq * a.lse_stride_h + i] = lse;
  }
}

template <typename T>
hipError_t launch_t(const PrefillParams& p, hipStream_t s) {
  const goda_prefill_args& a = p.a;
  dim3 grid((a.seqlen_q + kRows - 1) / kRows, a.heads_q, a.batch);
  hipError_t e = record_timing(a.timing_begin, s);
  if (e != hipSuccess) return e;
  switch (a.head_dim) {
    case 64:
      prefill_generic_kernel<T, 64><<<grid, kThreads, 0, s>>>(p);
      break;
    case 128:
      prefill_generic_kernel<T, 128><<<grid, kThreads, 0, s>>>(p);
      break;
    case 256:
      prefill_generic_kernel<T, 256><<<grid, kThreads, 0, s>>>(p);
      break;
    default:
      return hipErrorNotSupported;
  }
  if ((e = hipGetLastError()) != hipSuccess) return e;
  return record_timing(a.timing_end, s);
}

}  // namespace

hipError_t launch_prefill_generic(const PrefillParams& p, hipStream_t s) {
  switch (p.a.dtype) {
    case GODA_DTYPE_F32:
      return launch_t<float>(p, s);
    case GODA_DTYPE_F16:
      return launch_t<f16>(p, s);
    case GODA_DTYPE_BF16:
      return launch_t<bf16>(p, s);
    default:
      return hipErrorNotSupported;
  }
}

}  // namespace goda
