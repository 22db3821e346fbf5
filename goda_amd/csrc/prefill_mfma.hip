// Causal / non-causal GQA-MQA prefill attention on gfx950 matrix cores
// (bf16 or fp16 operands, fp32 accumulation).
//
// Two launches per call:
//   1. pack_kv_kernel: reads every K/V row of a KV head exactly once, applies
//      RoPE to K (half-split rotation, mint/nn/pos.py:90-98), and writes
//      tile-major copies to the workspace: K' tiles [BKV][D] and V^T tiles
//      [D][BKV]. Rotating K here instead of inside the attention loop means
//      each key is rotated once, not once per query tile and per query head.
//   2. prefill_mfma_kernel: one workgroup per (query tile, query-head slice,
//      sequence). All waves of a workgroup belong to query heads of ONE KV
//      head, so every K/V tile brought into LDS serves HG query heads ("read
//      once per query-head group"). Per wave: 32*NT query rows of one head.
//
// GEMM shapes per wave and KV tile (32x32x16 MFMA):
//   S^T[kv][q] = K'[kv][d] . Q^T[d][q]     A = K' from LDS, B = Q^T in VGPRs
//   O^T[d][q] += V^T[d][kv] . P^T[kv][q]   A = V^T from LDS, B = P^T in VGPRs
// Computing the transposed products keeps every query row in one lane pair
// (lanes l and l^32), so the online softmax needs a single cross-lane max per
// tile and the output rescale is lane-local.
//
// MFMA 32x32 accumulator layout (gfx9 family): lane l, register r holds
// row 8*(r/4) + 4*(l/32) + r%4, column l%32. The layout of the K dimension
// inside the A/B operands is the same function for A and B, so any
// consistent assignment of k indices to (lane half, element) is valid; the
// P^T operand reuses the S^T accumulator layout and V^T is read with that
// same assignment.

#include "common.h"
#include "launch.h"

namespace goda {
namespace {

constexpr int kWaves = 4;

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

template <int D, int BKV>
struct Tile {
  static constexpr int KLD = D + 8;    // K' LDS row stride (elements), 16-B aligned rows
  static constexpr int VLD = BKV + 4;  // V^T LDS row stride: rows shift by 2 banks
  static constexpr int K_ELEMS = BKV * KLD;
  static constexpr int V_ELEMS = D * VLD;
  static constexpr int STAGE_ELEMS = K_ELEMS + V_ELEMS;
};

// Shared by both launches: index of workspace tile j of sequence b, KV head hk.
__device__ __forceinline__ int64_t ws_tile(int b, int j, int hk, int ntiles, int hkv) {
  return ((int64_t)b * ntiles + j) * hkv + hk;
}

// ---------------------------------------------------------------------------
// 1. pack K (rotated) and V^T into tile-major workspace
// ---------------------------------------------------------------------------
template <typename T, int D, int BKV>
__global__ void __launch_bounds__(256) pack_kv_kernel(const PrefillParams p) {
  typedef typename Vec<T>::v8 v8;
  const goda_prefill_args& a = p.a;
  const int j = blockIdx.x;
  const int hk = blockIdx.y;
  const int b = blockIdx.z;
  const SeqGeom g = seq_geom(b, a.seqlen_q, a.seqlen_k, a.cu_seqlens_q, a.cu_seqlens_k,
                             a.seqused_k);
  const int kv0 = j * BKV;
  if (kv0 >= g.lk) return;

  T* kp = reinterpret_cast<T*>(a.workspace);
  const int64_t tile_elems = (int64_t)BKV * D;
  const int64_t ntot = (int64_t)a.batch * p.ntiles_k * a.heads_kv;
  T* vt = kp + ntot * tile_elems;
  const int64_t t = ws_tile(b, j, hk, p.ntiles_k, a.heads_kv);
  T* kdst = kp + t * tile_elems;
  T* vdst = vt + t * tile_elems;

  const T* kbase = reinterpret_cast<const T*>(a.k) +
                   (a.cu_seqlens_k ? 0 : (int64_t)b * a.k_stride_b) + (int64_t)hk * a.k_stride_h;
  const T* vbase = reinterpret_cast<const T*>(a.v) +
                   (a.cu_seqlens_k ? 0 : (int64_t)b * a.v_stride_b) + (int64_t)hk * a.v_stride_h;

  // V rows staged for the transpose; +8 elements keep columns off one bank.
  __shared__ T vs[BKV][D + 8];

  const int tid = threadIdx.x;
  constexpr int HALF8 = D / 16;  // 8-element chunks per half row
  for (int idx = tid; idx < BKV * HALF8; idx += 256) {
    const int r = idx / HALF8;
    const int c = (idx % HALF8) * 8;
    const int row = kv0 + r;
    v8 k1 = {}, k2 = {}, v1 = {}, v2 = {};
    if (row < g.lk) {
      const int64_t roff = (g.k_row0 + row);
      const T* kr = kbase + roff * a.k_stride_t;
      const T* vr = vbase + roff * a.v_stride_t;
      k1 = ld_vec<v8>(kr + c);
      k2 = ld_vec<v8>(kr + c + D / 2);
      v1 = ld_vec<v8>(vr + c);
      v2 = ld_vec<v8>(vr + c + D / 2);
      if (a.rope_k) {
        const int pos = a.rope_k_offset + row;
        const float* cs = a.rope_cos + (int64_t)pos * (D / 2) + c;
        const float* sn = a.rope_sin + (int64_t)pos * (D / 2) + c;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x1 = (float)k1[e], x2 = (float)k2[e];
          const float cc = cs[e], ss = sn[e];
          k1[e] = (T)(x1 * cc - x2 * ss);
          k2[e] = (T)(x1 * ss + x2 * cc);
        }
      }
    }
    st_vec<v8>(kdst + r * D + c, k1);
    st_vec<v8>(kdst + r * D + c + D / 2, k2);
    st_vec<v8>(&vs[r][c], v1);
    st_vec<v8>(&vs[r][c + D / 2], v2);
  }
  __syncthreads();
  // V^T: thread writes 8 consecutive keys of one head-dim row.
  constexpr int RCH = BKV / 8;
  for (int idx = tid; idx < D * RCH; idx += 256) {
    const int d = idx / RCH;
    const int r0 = (idx % RCH) * 8;
    v8 out;
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = vs[r0 + e][d];
    st_vec<v8>(vdst + (int64_t)d * BKV + r0, out);
  }
}

// ---------------------------------------------------------------------------
// 2. attention
// ---------------------------------------------------------------------------
template <typename T, int D, int BKV, int NT, bool ALIBI>
__global__ void __launch_bounds__(kWaves * 64, 1) prefill_mfma_kernel(const PrefillParams p) {
  typedef typename Vec<T>::v8 v8;
  typedef typename Vec<T>::v4 v4;
  typedef Tile<D, BKV> TL;
  constexpr int MT = BKV / 32;   // 32-key row tiles of S^T
  constexpr int KS = D / 16;     // k-steps of QK^T
  constexpr int MD = D / 32;     // 32-wide head-dim tiles of O^T
  constexpr int KS2 = BKV / 16;  // k-steps of PV
  constexpr int THREADS = kWaves * 64;

  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* smem = reinterpret_cast<T*>(smem_raw);

  const goda_prefill_args& a = p.a;
  const int hg = p.heads_per_wg;
  const int nslices = p.group / hg;
  const int qb_rows = (kWaves / hg) * 32 * NT;  // query rows per workgroup
  const int nqt = (a.seqlen_q + qb_rows - 1) / qb_rows;

  // XCD-aware order: consecutive dispatch slots rotate over the 8 XCDs; give
  // each XCD a contiguous range of (sequence, head-slice) pairs so that the
  // workgroups sharing K/V tiles share that XCD's L2. Heavy causal query
  // tiles go first.
  const int nblk = gridDim.x;
  const int lin = blockIdx.x;
  const int vid = (nblk % 8 == 0) ? (lin % 8) * (nblk / 8) + lin / 8 : lin;
  const int pair = vid / nqt;
  const int qt = nqt - 1 - (vid % nqt);
  const int b = pair / (a.heads_kv * nslices);
  const int rem = pair % (a.heads_kv * nslices);
  const int hk = rem / nslices;
  const int sl = rem % nslices;

  const SeqGeom g = seq_geom(b, a.seqlen_q, a.seqlen_k, a.cu_seqlens_q, a.cu_seqlens_k,
                             a.seqused_k);
  const int qr0 = qt * qb_rows;
  if (qr0 >= g.lq) return;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int hi = lane >> 5;  // lane half
  const int hq = hk * p.group + sl * hg + (wave % hg);
  const int wrow0 = qr0 + (wave / hg) * 32 * NT;  // first query row of this wave
  const int diag = g.lk - g.lq;
  const bool use_window = a.window_left >= 0 && (a.causal || g.lq == 1);

  // ---- Q^T operand fragments (rotated) -------------------------------------
  v8 qf[NT][KS];
  {
    const T* qbase = reinterpret_cast<const T*>(a.q) +
                     (a.cu_seqlens_q ? 0 : (int64_t)b * a.q_stride_b) + (int64_t)hq * a.q_stride_h;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int qi = wrow0 + 32 * nt + l32;
      if (qi < g.lq) {
        const T* qr = qbase + (g.q_row0 + qi) * a.q_stride_t;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) qf[nt][ks] = ld_vec<v8>(qr + 16 * ks + 8 * hi);
        if (a.rope_q) {
          const int pos = min(max(a.rope_q_offset + diag + qi, 0), a.rope_len - 1);
#pragma unroll
          for (int ks = 0; ks < KS / 2; ++ks) {
            const int f0 = 16 * ks + 8 * hi;
            const float* cs = a.rope_cos + (int64_t)pos * (D / 2) + f0;
            const float* sn = a.rope_sin + (int64_t)pos * (D / 2) + f0;
            const f32x4 c0 = ld_vec<f32x4>(cs), c1 = ld_vec<f32x4>(cs + 4);
            const f32x4 s0 = ld_vec<f32x4>(sn), s1 = ld_vec<f32x4>(sn + 4);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float cc = e < 4 ? c0[e & 3] : c1[e & 3];
              const float ss = e < 4 ? s0[e & 3] : s1[e & 3];
              const float x1 = (float)qf[nt][ks][e], x2 = (float)qf[nt][ks + KS / 2][e];
              qf[nt][ks][e] = (T)(x1 * cc - x2 * ss);
              qf[nt][ks + KS / 2][e] = (T)(x1 * ss + x2 * cc);
            }
          }
        }
      } else {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) qf[nt][ks] = v8{};
      }
    }
  }

  // ---- key tile range ---------------------------------------------------------
  const int q_last = min(qr0 + qb_rows, g.lq) - 1;
  int kv_hi = g.lk;
  if (a.causal) kv_hi = min(kv_hi, diag + q_last + 1);
  int kv_lo = 0;
  if (use_window) kv_lo = max(0, diag + qr0 - a.window_left);
  const int j_lo = kv_lo / BKV;
  const int j_hi = kv_hi > 0 ? (kv_hi + BKV - 1) / BKV : 0;

  const T* kp = reinterpret_cast<const T*>(a.workspace);
  const int64_t tile_elems = (int64_t)BKV * D;
  const int64_t ntot = (int64_t)a.batch * p.ntiles_k * a.heads_kv;
  const T* vt = kp + ntot * tile_elems;

  // Global -> register staging of one K'/V^T tile pair.
  constexpr int NVEC = BKV * D / 8 / THREADS;  // 16-byte vectors per thread per tensor
  static_assert(NVEC >= 1 && (BKV * D / 8) % THREADS == 0, "tile not divisible");
  v8 kreg[NVEC], vreg[NVEC];
  auto load_tile = [&](int j) {
    const int64_t t = ws_tile(b, j, hk, p.ntiles_k, a.heads_kv);
    const T* ks = kp + t * tile_elems;
    const T* vs = vt + t * tile_elems;
#pragma unroll
    for (int i = 0; i < NVEC; ++i) {
      const int v = tid + i * THREADS;
      kreg[i] = ld_vec<v8>(ks + v * 8);
      vreg[i] = ld_vec<v8>(vs + v * 8);
    }
  };
  auto store_tile = [&](int buf) {
    T* kl = smem + buf * TL::STAGE_ELEMS;
    T* vl = kl + TL::K_ELEMS;
#pragma unroll
    for (int i = 0; i < NVEC; ++i) {
      const int v = tid + i * THREADS;
      const int kr = v / (D / 8), kc = (v % (D / 8)) * 8;
      st_vec<v8>(kl + kr * TL::KLD + kc, kreg[i]);
      const int vr = v / (BKV / 8), vc = (v % (BKV / 8)) * 8;
      const v4 lo = {vreg[i][0], vreg[i][1], vreg[i][2], vreg[i][3]};
      const v4 hi4 = {vreg[i][4], vreg[i][5], vreg[i][6], vreg[i][7]};
      st_vec<v4>(vl + vr * TL::VLD + vc, lo);
      st_vec<v4>(vl + vr * TL::VLD + vc + 4, hi4);
    }
  };

  f32x16 oacc[MD][NT];
#pragma unroll
  for (int md = 0; md < MD; ++md)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) oacc[md][nt] = f32x16{};
  float m_run[NT], l_run[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    m_run[nt] = kNegInf;
    l_run[nt] = 0.f;
  }
  const float c = p.scale_log2;
  const float slope2 = ALIBI ? a.alibi_slopes[hq] * kLog2e : 0.f;

  if (j_lo < j_hi) {
    load_tile(j_lo);
    store_tile(0);
  }
  __syncthreads();

  for (int j = j_lo; j < j_hi; ++j) {
    const int buf = (j - j_lo) & 1;
    if (j + 1 < j_hi) load_tile(j + 1);
    const T* kl = smem + buf * TL::STAGE_ELEMS;
    const T* vl = kl + TL::K_ELEMS;

    // S^T = K' Q^T
    f32x16 sacc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) sacc[mt][nt] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const v8 av = ld_vec<v8>(kl + (32 * mt + l32) * TL::KLD + 16 * ks + 8 * hi);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) sacc[mt][nt] = mfma32(av, qf[nt][ks], sacc[mt][nt]);
      }
    }

    // Mask, online softmax, P^T fragments.
    const int kvb = j * BKV;
    const bool need_mask = (kvb + BKV > g.lk) ||
                           (a.causal && kvb + BKV - 1 > diag + wrow0) ||
                           (use_window && kvb < diag + wrow0 + 32 * NT - 1 - a.window_left);
    v8 pf[NT][KS2];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int qi = wrow0 + 32 * nt + l32;
      const int iabs = diag + qi;
      if (need_mask || ALIBI) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int kv = kvb + 32 * mt + 8 * (r >> 2) + 4 * hi + (r & 3);
            bool vis = kv < g.lk;
            if (a.causal) vis = vis && kv <= iabs;
            if (use_window) vis = vis && (iabs - kv <= a.window_left);
            float t = sacc[mt][nt][r];
            if (ALIBI) t = fmaf(t, c, slope2 * (float)(kv - iabs));
            sacc[mt][nt][r] = vis ? t : kNegInf;
          }
      }
      float mx = kNegInf;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[mt][nt][r]);
      mx = fmaxf(mx, shfl_xor_f(mx, 32));
      const float m_new = fmaxf(m_run[nt], ALIBI ? mx : mx * c);
      const float m_use = (m_new == kNegInf) ? 0.f : m_new;
      const float alpha = fast_exp2(m_run[nt] - m_use);
      m_run[nt] = m_new;
      float lsum = 0.f;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float s = sacc[mt][nt][r];
          const float pv = ALIBI ? fast_exp2(s - m_use) : fast_exp2(fmaf(s, c, -m_use));
          lsum += pv;
          pf[nt][2 * mt + (r >> 3)][r & 7] = (T)pv;
        }
      }
      l_run[nt] = l_run[nt] * alpha + lsum;
#pragma unroll
      for (int md = 0; md < MD; ++md) oacc[md][nt] *= alpha;
    }

    // O^T += V^T P^T
#pragma unroll
    for (int ks2 = 0; ks2 < KS2; ++ks2) {
#pragma unroll
      for (int md = 0; md < MD; ++md) {
        const T* vp = vl + (32 * md + l32) * TL::VLD + 16 * ks2 + 4 * hi;
        const v4 a0 = ld_vec<v4>(vp);
        const v4 a1 = ld_vec<v4>(vp + 8);
        const v8 av = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) oacc[md][nt] = mfma32(av, pf[nt][ks2], oacc[md][nt]);
      }
    }

    if (j + 1 < j_hi) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue ------------------------------------------------------------
  T* obase = reinterpret_cast<T*>(a.o) + (a.cu_seqlens_q ? 0 : (int64_t)b * a.o_stride_b) +
             (int64_t)hq * a.o_stride_h;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const float ltot = l_run[nt] + shfl_xor_f(l_run[nt], 32);
    const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
    const int qi = wrow0 + 32 * nt + l32;
    if (qi < g.lq) {
      T* orow = obase + (g.q_row0 + qi) * a.o_stride_t;
#pragma unroll
      for (int md = 0; md < MD; ++md)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int d0 = 32 * md + 8 * rr + 4 * hi;
          const v4 ov = {(T)(oacc[md][nt][4 * rr + 0] * inv), (T)(oacc[md][nt][4 * rr + 1] * inv),
                         (T)(oacc[md][nt][4 * rr + 2] * inv), (T)(oacc[md][nt][4 * rr + 3] * inv)};
          st_vec<v4>(orow + d0, ov);
        }
      if (a.lse && hi == 0) {
        const float lse = ltot > 0.f ? (m_run[nt] + log2f(ltot)) * kLn2 : kNegInf;
        if (a.cu_seqlens_q)
          a.lse[(int64_t)hq * a.lse_stride_h + g.q_row0 + qi] = lse;
        else
          a.lse[(int64_t)b * a.lse_stride_b + (int64_t)hq * a.lse_stride_h + qi] = lse;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
int kv_tile_for(int d) { return 64; }
int nt_for(int d) { return d >= 256 ? 1 : 2; }

int gcd_int(int x, int y) {
  while (y) {
    int t = x % y;
    x = y;
    y = t;
  }
  return x;
}

template <typename T, int D, int BKV, int NT, bool ALIBI>
hipError_t launch_attn(PrefillParams p, hipStream_t s) {
  const goda_prefill_args& a = p.a;
  const int hg = gcd_int(p.group, kWaves);
  p.heads_per_wg = hg;
  const int qb_rows = (kWaves / hg) * 32 * NT;
  const int nqt = (a.seqlen_q + qb_rows - 1) / qb_rows;
  const int64_t nblk = (int64_t)nqt * a.batch * a.heads_kv * (p.group / hg);
  if (nblk <= 0) return hipSuccess;
  if (nblk > 0x7fffffff) return hipErrorInvalidValue;
  const size_t lds = 2 * Tile<D, BKV>::STAGE_ELEMS * sizeof(T);
  auto kern = prefill_mfma_kernel<T, D, BKV, NT, ALIBI>;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)lds);
  if (e != hipSuccess) return e;
  if ((e = record_timing(a.timing_begin, s)) != hipSuccess) return e;
  kern<<<dim3((unsigned)nblk), dim3(kWaves * 64), lds, s>>>(p);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  return record_timing(a.timing_end, s);
}

template <typename T, int D>
hipError_t launch_d(PrefillParams p, hipStream_t s) {
  constexpr int BKV = 64;
  const goda_prefill_args& a = p.a;
  p.kv_tile = BKV;
  p.ntiles_k = (a.seqlen_k + BKV - 1) / BKV;
  if (p.ntiles_k > 0) {
    dim3 grid(p.ntiles_k, a.heads_kv, a.batch);
    pack_kv_kernel<T, D, BKV><<<grid, 256, 0, s>>>(p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  constexpr int NT = D >= 256 ? 1 : 2;
  if (a.alibi_slopes) return launch_attn<T, D, BKV, NT, true>(p, s);
  return launch_attn<T, D, BKV, NT, false>(p, s);
}

template <typename T>
hipError_t launch_t(const PrefillParams& p, hipStream_t s) {
  switch (p.a.head_dim) {
    case 64:
      return launch_d<T, 64>(p, s);
    case 128:
      return launch_d<T, 128>(p, s);
    case 256:
      return launch_d<T, 256>(p, s);
    default:
      return hipErrorNotSupported;
  }
}

}  // namespace

bool prefill_mfma_supported(const goda_prefill_args& a) {
  if (a.dtype != GODA_DTYPE_BF16 && a.dtype != GODA_DTYPE_F16) return false;
  return a.head_dim == 64 || a.head_dim == 128 || a.head_dim == 256;
}

int64_t prefill_mfma_workspace_bytes(const goda_prefill_args& a) {
  const int bkv = kv_tile_for(a.head_dim);
  const int64_t ntiles = (a.seqlen_k + bkv - 1) / bkv;
  return 2 * (int64_t)a.batch * ntiles * a.heads_kv * bkv * a.head_dim * 2;
}

hipError_t launch_prefill_mfma(const PrefillParams& p, hipStream_t s) {
  if (p.a.dtype == GODA_DTYPE_BF16) return launch_t<bf16>(p, s);
  if (p.a.dtype == GODA_DTYPE_F16) return launch_t<f16>(p, s);
  return hipErrorNotSupported;
}

}  // namespace goda
