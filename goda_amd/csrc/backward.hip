// Backward of prefill attention: dq, dk, dv from dO and the forward's saved o
// and log-sum-exp (kernels_/flash_attn_gqa/cuda.py:577-658 computes the same
// quantities: D = rowsum(dO * O), P = exp(scale * q k^T - M),
// dV = P^T dO, dS = P * (dO V^T - D), dQ = scale * dS K, dK = scale * dS^T Q).
//
// This file holds the generic kernels: fp32 arithmetic on the vector ALUs,
// the path for fp32 at head_dim 256 (goda's default model dtype is fp32,
// mint/nn/models.py:23), whose operands do not fit the matrix-core kernels;
// every other dtype / head_dim runs on backward_mfma.hip. Three launches:
//   1. bwd_delta_kernel   delta[hq][row] = sum_d dO * O (fp32 workspace);
//   2. bwd_dkv_kernel     one workgroup per (key block, KV head, sequence):
//                         keys stay in registers, query rows of every head of
//                         the KV head's group stream through LDS, so the GQA
//                         reduction of dk/dv happens in registers and each
//                         dk/dv row is written once (no atomics);
//   3. bwd_dq_kernel      one workgroup per (query block, query head,
//                         sequence): query rows stay in registers, keys
//                         stream through LDS.
// Masks, ALiBi and RoPE follow the forward exactly: scores are recomputed
// from the rotated q and k, and the gradients of the rotated rows are rotated
// back (the transpose of the rotation) before they are written.

#include "common.h"
#include "launch.h"

namespace goda {
namespace {

constexpr int kThreads = 256;

// Row split: TPR = D/32 consecutive threads share a row (a query or a key);
// thread `part` holds the 32 head-dim elements 4*(TPR*g + part) + j (g < 8,
// j < 4), so adjacent threads read adjacent 16-byte pieces of a row, and
// group g < 4 pairs with group g + 4 (offset D/2) for RoPE.
template <int D>
struct Split {
  static constexpr int TPR = D / 32;
  static constexpr int ROWS = kThreads / TPR;  // rows per workgroup
  static constexpr int STAGE = 4096 / D;       // rows staged in LDS per step (2 x 16 KB)
  static __device__ __forceinline__ int col(int part, int g) { return 4 * (TPR * g + part); }
};

template <typename T, int D>
__device__ __forceinline__ void load_part(const T* row, int part, float (&x)[32]) {
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    float t[4];
    load4f<T>(row + Split<D>::col(part, g), t);
#pragma unroll
    for (int j = 0; j < 4; ++j) x[4 * g + j] = t[j];
  }
}

template <typename T, int D>
__device__ __forceinline__ void store_part(T* row, int part, const float (&x)[32]) {
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const float t[4] = {x[4 * g], x[4 * g + 1], x[4 * g + 2], x[4 * g + 3]};
    store4f<T>(row + Split<D>::col(part, g), t);
  }
}

// Half-split rotation of a row part by the table row (cos_row, sin_row)
// (mint/nn/pos.py:90-98); `inverse` applies the transpose, which takes the
// gradient of a rotated row back to the unrotated input.
template <int D>
__device__ __forceinline__ void rope_part(float (&x)[32], const float* cos_row, const float* sin_row,
                                          int part, bool inverse) {
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int f = Split<D>::col(part, g) + j;
      const float c = cos_row[f];
      const float s = inverse ? -sin_row[f] : sin_row[f];
      const float x1 = x[4 * g + j], x2 = x[4 * (g + 4) + j];
      x[4 * g + j] = x1 * c - x2 * s;
      x[4 * (g + 4) + j] = x1 * s + x2 * c;
    }
}

// Dot product of a row held in parts with an LDS row, summed over the TPR
// threads of the row.
template <int D>
__device__ __forceinline__ float row_dot(const float (&x)[32], const float* y, int part) {
  float s = 0.f;
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const f32x4 v = ld_vec<f32x4>(y + Split<D>::col(part, g));
    s = fmaf(x[4 * g + 0], v[0], s);
    s = fmaf(x[4 * g + 1], v[1], s);
    s = fmaf(x[4 * g + 2], v[2], s);
    s = fmaf(x[4 * g + 3], v[3], s);
  }
#pragma unroll
  for (int o = 1; o < Split<D>::TPR; o <<= 1) s += shfl_xor_f(s, o);
  return s;
}

// x += w * y for an LDS row y.
template <int D>
__device__ __forceinline__ void row_axpy(float (&x)[32], float w, const float* y, int part) {
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const f32x4 v = ld_vec<f32x4>(y + Split<D>::col(part, g));
    x[4 * g + 0] = fmaf(w, v[0], x[4 * g + 0]);
    x[4 * g + 1] = fmaf(w, v[1], x[4 * g + 1]);
    x[4 * g + 2] = fmaf(w, v[2], x[4 * g + 2]);
    x[4 * g + 3] = fmaf(w, v[3], x[4 * g + 3]);
  }
}

// Index of query row i of sequence b, head hq in the lse tensor and in the
// delta buffer.
__device__ __forceinline__ int64_t lse_index(const goda_prefill_args& a, const SeqGeom& g, int b, int hq,
                                             int i) {
  if (a.cu_seqlens_q) return (int64_t)hq * a.lse_stride_h + g.q_row0 + i;
  return (int64_t)b * a.lse_stride_b + (int64_t)hq * a.lse_stride_h + i;
}
__device__ __forceinline__ int64_t delta_index(const BwdParams& p, const SeqGeom& g, int b, int hq, int i) {
  const int64_t row = p.a.cu_seqlens_q ? g.q_row0 + i : (int64_t)b * p.a.seqlen_q + i;
  return (int64_t)hq * p.delta_rows + row;
}

template <typename T>
__device__ __forceinline__ const T* row_ptr(const void* base, int64_t sb, int64_t st, int64_t sh, bool varlen,
                                            int b, int64_t row, int h) {
  return reinterpret_cast<const T*>(base) + (varlen ? 0 : (int64_t)b * sb) + row * st + (int64_t)h * sh;
}
template <typename T>
__device__ __forceinline__ T* row_ptr_w(void* base, int64_t sb, int64_t st, int64_t sh, bool varlen, int b,
                                        int64_t row, int h) {
  return reinterpret_cast<T*>(base) + (varlen ? 0 : (int64_t)b * sb) + row * st + (int64_t)h * sh;
}

// ---------------------------------------------------------------------------
// 1. delta = rowsum(dO * O)
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ void __launch_bounds__(kThreads) bwd_delta_kernel(const BwdParams p) {
  typedef Split<D> S;
  const goda_prefill_args& a = p.a;
  const int b = blockIdx.z, hq = blockIdx.y;
  const SeqGeom g = seq_geom(b, a.seqlen_q, a.seqlen_k, a.cu_seqlens_q, a.cu_seqlens_k, a.seqused_k);
  const int row = threadIdx.x / S::TPR, part = threadIdx.x % S::TPR;
  const int i = blockIdx.x * S::ROWS + row;
  if (i >= g.lq) return;  // the TPR threads of a row leave together
  const bool varlen = a.cu_seqlens_q != nullptr;
  float o[32], d_o[32];
  load_part<T, D>(row_ptr<T>(a.o, a.o_stride_b, a.o_stride_t, a.o_stride_h, varlen, b, g.q_row0 + i, hq), part, o);
  load_part<T, D>(row_ptr<T>(p.g.d_o, p.g.do_stride_b, p.g.do_stride_t, p.g.do_stride_h, varlen, b, g.q_row0 + i, hq),
                  part, d_o);
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 32; ++e) s = fmaf(o[e], d_o[e], s);
#pragma unroll
  for (int off = 1; off < S::TPR; off <<= 1) s += shfl_xor_f(s, off);
  if (part == 0) p.delta[delta_index(p, g, b, hq, i)] = s;
}

// ---------------------------------------------------------------------------
// 2. dk, dv
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ void __launch_bounds__(kThreads) bwd_dkv_kernel(const BwdParams p) {
  typedef Split<D> S;
  const goda_prefill_args& a = p.a;
  const goda_prefill_grads& gr = p.g;
  __shared__ __align__(16) float Qs[S::STAGE][D];
  __shared__ __align__(16) float Gs[S::STAGE][D];  // dO rows
  __shared__ float Ls[S::STAGE];                   // lse, log2 units
  __shared__ float Dl[S::STAGE];                   // delta

  const int b = blockIdx.z, hk = blockIdx.y;
  const SeqGeom g = seq_geom(b, a.seqlen_q, a.seqlen_k, a.cu_seqlens_q, a.cu_seqlens_k, a.seqused_k);
  const bool varlen = a.cu_seqlens_q != nullptr;
  // Rows this launch owns: the keys of the sequence (varlen), or every row of
  // the dense k tensor, where rows past the used keys get zero gradients.
  const int kend = varlen ? g.lk : a.seqlen_k;
  const int kv0 = blockIdx.x * S::ROWS;
  if (kv0 >= kend) return;

  const int tid = threadIdx.x;
  const int row = tid / S::TPR, part = tid % S::TPR;
  const int j = kv0 + row;
  const bool key_valid = j < g.lk;
  const int diag = g.lk - g.lq;
  const bool use_window = a.window_left >= 0 && (a.causal || g.lq == 1);

  float k[32], v[32], dk[32], dv[32];
#pragma unroll
  for (int e = 0; e < 32; ++e) dk[e] = dv[e] = k[e] = v[e] = 0.f;
  if (key_valid) {
    load_part<T, D>(row_ptr<T>(a.k, a.k_stride_b, a.k_stride_t, a.k_stride_h, varlen, b, g.k_row0 + j, hk), part, k);
    load_part<T, D>(row_ptr<T>(a.v, a.v_stride_b, a.v_stride_t, a.v_stride_h, varlen, b, g.k_row0 + j, hk), part, v);
    if (a.rope_k) {
      const int pos = a.rope_k_offset + j;
      rope_part<D>(k, a.rope_cos + (int64_t)pos * (D / 2), a.rope_sin + (int64_t)pos * (D / 2), part, false);
    }
  }

  // Query rows that can see a key of this block.
  const int kv_last = min(kv0 + S::ROWS, g.lk) - 1;
  int i_lo = 0, i_hi = g.lq;
  if (a.causal) i_lo = max(0, kv0 - diag);
  if (use_window) i_hi = min(g.lq, kv_last + a.window_left - diag + 1);
  if (kv0 >= g.lk) i_hi = i_lo;

  const float c = p.scale_log2;
  for (int h = 0; h < p.group; ++h) {
    const int hq = hk * p.group + h;
    const float slope2 = a.alibi_slopes ? a.alibi_slopes[hq] * kLog2e : 0.f;
    for (int i0 = i_lo; i0 < i_hi; i0 += S::STAGE) {
      __syncthreads();
      // Stage query rows i0.. (rotated q, dO) and their lse / delta.
      constexpr int HALF4 = D / 8;
      for (int idx = tid; idx < S::STAGE * HALF4; idx += kThreads) {
        const int ir = idx / HALF4;
        const int c4 = (idx % HALF4) * 4;
        const int i = i0 + ir;
        float q1[4] = {0.f, 0.f, 0.f, 0.f}, q2[4] = {0.f, 0.f, 0.f, 0.f};
        float g1[4] = {0.f, 0.f, 0.f, 0.f}, g2[4] = {0.f, 0.f, 0.f, 0.f};
        if (i < i_hi) {
          const T* qr = row_ptr<T>(a.q, a.q_stride_b, a.q_stride_t, a.q_stride_h, varlen, b, g.q_row0 + i, hq);
          const T* dr = row_ptr<T>(gr.d_o, gr.do_stride_b, gr.do_stride_t, gr.do_stride_h, varlen, b, g.q_row0 + i, hq);
          load4f<T>(qr + c4, q1);
          load4f<T>(qr + c4 + D / 2, q2);
          load4f<T>(dr + c4, g1);
          load4f<T>(dr + c4 + D / 2, g2);
          if (a.rope_q) {
            const int pos = rope_qpos(a, diag, i);
            const float* cs = a.rope_cos + (int64_t)pos * (D / 2) + c4;
            const float* sn = a.rope_sin + (int64_t)pos * (D / 2) + c4;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float x1 = q1[e], x2 = q2[e];
              q1[e] = x1 * cs[e] - x2 * sn[e];
              q2[e] = x1 * sn[e] + x2 * cs[e];
            }
          }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          Qs[ir][c4 + e] = q1[e];
          Qs[ir][c4 + D / 2 + e] = q2[e];
          Gs[ir][c4 + e] = g1[e];
          Gs[ir][c4 + D / 2 + e] = g2[e];
        }
      }
      for (int ir = tid; ir < S::STAGE; ir += kThreads) {
        const int i = i0 + ir;
        float l2 = kNegInf, dl = 0.f;
        if (i < i_hi) {
          l2 = a.lse[lse_index(a, g, b, hq, i)] * kLog2e;
          dl = p.delta[delta_index(p, g, b, hq, i)];
        }
        Ls[ir] = l2;
        Dl[ir] = dl;
      }
      __syncthreads();

      for (int ir = 0; ir < S::STAGE; ++ir) {
        const int i = i0 + ir;
        const int iabs = diag + i;
        const float s = row_dot<D>(k, Qs[ir], part);
        bool vis = key_valid && i < i_hi && Ls[ir] != kNegInf;
        if (a.causal) vis = vis && j <= iabs;
        if (use_window) vis = vis && iabs - j <= a.window_left;
        if (vis && a.mask_bits) vis = mask_bit(mask_row(a, b, hq, i), j);
        float t = s * c;
        if (a.alibi_slopes) t = fmaf(slope2, (float)(j - iabs), t);
        const float pr = vis ? exp2f(t - Ls[ir]) : 0.f;
        row_axpy<D>(dv, pr, Gs[ir], part);
        const float dp = row_dot<D>(v, Gs[ir], part);
        const float ds = pr * (dp - Dl[ir]);
        row_axpy<D>(dk, ds, Qs[ir], part);
      }
    }
  }

  if (j >= kend) return;
#pragma unroll
  for (int e = 0; e < 32; ++e) dk[e] *= a.softmax_scale;
  if (a.rope_k && key_valid) {
    const int pos = a.rope_k_offset + j;
    rope_part<D>(dk, a.rope_cos + (int64_t)pos * (D / 2), a.rope_sin + (int64_t)pos * (D / 2), part, true);
  }
  store_part<T, D>(row_ptr_w<T>(gr.dk, gr.dk_stride_b, gr.dk_stride_t, gr.dk_stride_h, varlen, b, g.k_row0 + j, hk),
                   part, dk);
  store_part<T, D>(row_ptr_w<T>(gr.dv, gr.dv_stride_b, gr.dv_stride_t, gr.dv_stride_h, varlen, b, g.k_row0 + j, hk),
                   part, dv);
}

// ---------------------------------------------------------------------------
// 3. dq
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ void __launch_bounds__(kThreads) bwd_dq_kernel(const BwdParams p) {
  typedef Split<D> S;
  const goda_prefill_args& a = p.a;
  const goda_prefill_grads& gr = p.g;
  __shared__ __align__(16) float Ks[S::STAGE][D];
  __shared__ __align__(16) float Vs[S::STAGE][D];

  const int b = blockIdx.z, hq = blockIdx.y;
  const int hk = hq / p.group;
  const SeqGeom g = seq_geom(b, a.seqlen_q, a.seqlen_k, a.cu_seqlens_q, a.cu_seqlens_k, a.seqused_k);
  const bool varlen = a.cu_seqlens_q != nullptr;
  const int q0 = blockIdx.x * S::ROWS;
  if (q0 >= g.lq) return;

  const int tid = threadIdx.x;
  const int row = tid / S::TPR, part = tid % S::TPR;
  const int i = q0 + row;
  const bool row_valid = i < g.lq;
  const int diag = g.lk - g.lq;
  const bool use_window = a.window_left >= 0 && (a.causal || g.lq == 1);
  const int iabs = diag + i;

  float q[32], d_o[32], dq[32];
  float l2 = kNegInf, dl = 0.f;
#pragma unroll
  for (int e = 0; e < 32; ++e) q[e] = d_o[e] = dq[e] = 0.f;
  const int qpos = row_valid ? rope_qpos(a, diag, i) : 0;
  if (row_valid) {
    load_part<T, D>(row_ptr<T>(a.q, a.q_stride_b, a.q_stride_t, a.q_stride_h, varlen, b, g.q_row0 + i, hq), part, q);
    load_part<T, D>(row_ptr<T>(gr.d_o, gr.do_stride_b, gr.do_stride_t, gr.do_stride_h, varlen, b, g.q_row0 + i, hq),
                    part, d_o);
    if (a.rope_q)
      rope_part<D>(q, a.rope_cos + (int64_t)qpos * (D / 2), a.rope_sin + (int64_t)qpos * (D / 2), part, false);
    l2 = a.lse[lse_index(a, g, b, hq, i)] * kLog2e;
    dl = p.delta[delta_index(p, g, b, hq, i)];
  }
  const float slope2 = a.alibi_slopes ? a.alibi_slopes[hq] * kLog2e : 0.f;
  const float c = p.scale_log2;

  // Keys that a row of this block can see.
  const int i_last = min(q0 + S::ROWS, g.lq) - 1;
  int kv_hi = g.lk;
  if (a.causal) kv_hi = min(kv_hi, diag + i_last + 1);
  int kv_lo = 0;
  if (use_window) kv_lo = max(0, diag + q0 - a.window_left);

  for (int kv0 = kv_lo; kv0 < kv_hi; kv0 += S::STAGE) {
    __syncthreads();
    constexpr int HALF4 = D / 8;
    for (int idx = tid; idx < S::STAGE * HALF4; idx += kThreads) {
      const int jr = idx / HALF4;
      const int c4 = (idx % HALF4) * 4;
      const int j = kv0 + jr;
      float k1[4] = {0.f, 0.f, 0.f, 0.f}, k2[4] = {0.f, 0.f, 0.f, 0.f};
      float v1[4] = {0.f, 0.f, 0.f, 0.f}, v2[4] = {0.f, 0.f, 0.f, 0.f};
      if (j < kv_hi) {
        const T* kr = row_ptr<T>(a.k, a.k_stride_b, a.k_stride_t, a.k_stride_h, varlen, b, g.k_row0 + j, hk);
        const T* vr = row_ptr<T>(a.v, a.v_stride_b, a.v_stride_t, a.v_stride_h, varlen, b, g.k_row0 + j, hk);
        load4f<T>(kr + c4, k1);
        load4f<T>(kr + c4 + D / 2, k2);
        load4f<T>(vr + c4, v1);
        load4f<T>(vr + c4 + D / 2, v2);
        if (a.rope_k) {
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
    __syncthreads();

    for (int jr = 0; jr < S::STAGE; ++jr) {
      const int j = kv0 + jr;
      const float s = row_dot<D>(q, Ks[jr], part);
      bool vis = row_valid && j < kv_hi && l2 != kNegInf;
      if (a.causal) vis = vis && j <= iabs;
      if (use_window) vis = vis && iabs - j <= a.window_left;
      if (vis && a.mask_bits) vis = mask_bit(mask_row(a, b, hq, i), j);
      float t = s * c;
      if (a.alibi_slopes) t = fmaf(slope2, (float)(j - iabs), t);
      const float pr = vis ? exp2f(t - l2) : 0.f;
      const float dp = row_dot<D>(d_o, Vs[jr], part);
      row_axpy<D>(dq, pr * (dp - dl), Ks[jr], part);
    }
  }

  if (!row_valid) return;
#pragma unroll
  for (int e = 0; e < 32; ++e) dq[e] *= a.softmax_scale;
  if (a.rope_q)
    rope_part<D>(dq, a.rope_cos + (int64_t)qpos * (D / 2), a.rope_sin + (int64_t)qpos * (D / 2), part, true);
  store_part<T, D>(row_ptr_w<T>(gr.dq, gr.dq_stride_b, gr.dq_stride_t, gr.dq_stride_h, varlen, b, g.q_row0 + i, hq),
                   part, dq);
}

template <typename T, int D>
hipError_t launch_generic_d(const BwdParams& p, hipStream_t s) {
  typedef Split<D> S;
  const goda_prefill_args& a = p.a;
  hipError_t e;
  const dim3 gq((a.seqlen_q + S::ROWS - 1) / S::ROWS, a.heads_q, a.batch);
  if (a.seqlen_q > 0) {
    bwd_delta_kernel<T, D><<<gq, kThreads, 0, s>>>(p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if ((e = record_timing(p.g.timing_begin, s)) != hipSuccess) return e;
  if (a.seqlen_k > 0) {
    const dim3 gk((a.seqlen_k + S::ROWS - 1) / S::ROWS, a.heads_kv, a.batch);
    bwd_dkv_kernel<T, D><<<gk, kThreads, 0, s>>>(p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if (a.seqlen_q > 0) {
    bwd_dq_kernel<T, D><<<gq, kThreads, 0, s>>>(p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  return record_timing(p.g.timing_end, s);
}

template <typename T>
hipError_t launch_generic_t(const BwdParams& p, hipStream_t s) {
  switch (p.a.head_dim) {
    case 64:
      return launch_generic_d<T, 64>(p, s);
    case 128:
      return launch_generic_d<T, 128>(p, s);
    case 256:
      return launch_generic_d<T, 256>(p, s);
    default:
      return hipErrorNotSupported;
  }
}

}  // namespace

namespace {

int64_t align_up(int64_t x) { return (x + 255) / 256 * 256; }

// Workspace layout: the kernels' own region, then with the fused QK-RMSNorm
// the dw partials and, for the generic kernels (which read q / k rows
// themselves), the normalized q and k rows.
struct BwdLayout {
  int64_t norm_part = 0, q_rows = 0, k_rows = 0, bytes = 0;
};

BwdLayout bwd_layout(const goda_prefill_args& a) {
  BwdLayout l;
  const bool mf = prefill_bwd_mfma_supported(a);
  l.bytes = mf ? prefill_bwd_mfma_workspace_bytes(a) : (int64_t)a.heads_q * a.batch * a.seqlen_q * (int64_t)sizeof(float);
  if (!a.q_norm_weight && !a.k_norm_weight) return l;
  l.norm_part = align_up(l.bytes);
  l.bytes = l.norm_part + norm_bwd_part_bytes(a);
  if (!mf) {
    const int64_t es = a.dtype == GODA_DTYPE_F32 ? 4 : 2;
    if (a.q_norm_weight) {
      l.q_rows = align_up(l.bytes);
      l.bytes = l.q_rows + (int64_t)a.batch * a.seqlen_q * a.heads_q * a.head_dim * es;
    }
    if (a.k_norm_weight) {
      l.k_rows = align_up(l.bytes);
      l.bytes = l.k_rows + (int64_t)a.batch * a.seqlen_k * a.heads_kv * a.head_dim * es;
    }
  }
  return l;
}

}  // namespace

int64_t prefill_bwd_workspace_bytes(const goda_prefill_args& a) { return bwd_layout(a).bytes; }

hipError_t launch_prefill_bwd(const BwdParams& p0, hipStream_t s) {
  const goda_prefill_args& a = p0.a;
  const bool norm = a.q_norm_weight || a.k_norm_weight;
  const bool mf = prefill_bwd_mfma_supported(a);
  const BwdLayout l = bwd_layout(a);
  unsigned char* ws = reinterpret_cast<unsigned char*>(p0.g.workspace);
  BwdParams p = p0;
  hipError_t e;
  if (norm && !mf) {
    // The generic kernels read q / k rows themselves: hand them the
    // normalized rows (RoPE stays theirs), so dq / dk come out as the
    // gradients of those rows, as on the MFMA path.
    if (a.q_norm_weight) {
      if ((e = launch_norm_rows(a, true, ws + l.q_rows, s)) != hipSuccess) return e;
      p.a.q = ws + l.q_rows;
      p.a.q_stride_h = a.head_dim;
      p.a.q_stride_t = (int64_t)a.heads_q * a.head_dim;
      p.a.q_stride_b = (int64_t)a.seqlen_q * p.a.q_stride_t;
    }
    if (a.k_norm_weight) {
      if ((e = launch_norm_rows(a, false, ws + l.k_rows, s)) != hipSuccess) return e;
      p.a.k = ws + l.k_rows;
      p.a.k_stride_h = a.head_dim;
      p.a.k_stride_t = (int64_t)a.heads_kv * a.head_dim;
      p.a.k_stride_b = (int64_t)a.seqlen_k * p.a.k_stride_t;
    }
    p.a.q_norm_weight = p.a.k_norm_weight = nullptr;
  }
  if (mf) {
    e = launch_prefill_bwd_mfma(p, s);
  } else {
    switch (a.dtype) {
      case GODA_DTYPE_F32:
        e = launch_generic_t<float>(p, s);
        break;
      case GODA_DTYPE_F16:
        e = launch_generic_t<f16>(p, s);
        break;
      case GODA_DTYPE_BF16:
        e = launch_generic_t<bf16>(p, s);
        break;
      default:
        e = hipErrorNotSupported;
    }
  }
  if (e != hipSuccess || !norm) return e;
  // dx and dw from the caller's rows (p0.a: the un-normalized q, k).
  return launch_norm_bwd(a, p0.g, reinterpret_cast<float*>(ws + l.norm_part), s);
}

}  // namespace goda
