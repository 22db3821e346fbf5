// One-token decode attention over a contiguous KV cache (bf16 / fp16),
// split-K over the cached keys with a log-sum-exp merge, plus the KV append.
//
// decode_splitk_kernel: one workgroup per (split, KV head x head slice,
// sequence). The split covers `split` consecutive keys of the sequence's valid
// range; the workgroup's 4 waves take 16-key chunks of it in turn, each with
// its own online-softmax state, and merge through LDS at the end.
//   scores  S^T[16 keys][16 heads] = K[16 keys][D] . Q^T[D][heads]
//           on 16x16x32 MFMA; K rows are loaded straight from the cache into
//           the A operand (16 bytes per lane), Q^T lives in VGPRs. All query
//           heads of the KV head's group are served by the same K/V bytes.
//   values  O[head][d] += p[head][key] * V[key][d] on the vector ALUs: each
//           lane owns 8 consecutive head-dim elements (16-byte loads, a wave
//           instruction reads whole cache rows), p is broadcast through LDS.
// A sequence whose keys fit in one split is written directly; otherwise each
// split writes (o_s normalised, lse_s) to the workspace and merge_kernel
// combines them: lse = log sum_s exp(lse_s), o = sum_s exp(lse_s - lse) o_s.

#include "common.h"
#include "launch.h"

namespace goda {
namespace {

constexpr int kWaves = 4;
constexpr int kChunk = 16;  // keys per wave step

template <typename T>
struct V8;
template <>
struct V8<bf16> {
  typedef bf16x8 t;
};
template <>
struct V8<f16> {
  typedef f16x8 t;
};

// Valid key range [kbeg, kend) of sequence b and its split count.
struct KeyRange {
  int kbeg, kend, nsplit;
};
__device__ __forceinline__ KeyRange key_range(const DecodeParams& p, int b) {
  const goda_decode_args& a = p.a;
  int L = a.cache_seqlens[b];
  L = max(0, min(L, a.max_seqlen));
  KeyRange r;
  r.kend = L;
  r.kbeg = (a.window_left >= 0) ? max(0, L - 1 - a.window_left) : 0;
  const int n = r.kend - r.kbeg;
  r.nsplit = n > 0 ? (n + p.split - 1) / p.split : 0;
  return r;
}

template <typename T, int D, int HMAX>
__global__ void __launch_bounds__(kWaves * 64) decode_splitk_kernel(const DecodeParams p) {
  typedef typename V8<T>::t v8;
  constexpr int KS = D / 32;    // k-steps of the 16x16x32 score MFMA
  constexpr int CPL = D / 128;  // 8-element head-dim chunks per lane in PV
  static_assert(CPL >= 1, "head_dim >= 128");
  const goda_decode_args& a = p.a;

  __shared__ float p_lds[kWaves][kChunk][16];
  __shared__ float alpha_lds[kWaves][16];
  __shared__ float red_m[kWaves][HMAX];
  __shared__ float red_l[kWaves][HMAX];
  __shared__ float red_o[kWaves][HMAX][D];

  const int s = blockIdx.x;
  const int nhs = (p.group + HMAX - 1) / HMAX;
  const int hk = blockIdx.y / nhs;
  const int hs = blockIdx.y % nhs;
  const int b = blockIdx.z;
  const int hq0 = hk * p.group + hs * HMAX;
  const int nh = min(HMAX, p.group - hs * HMAX);

  const KeyRange kr = key_range(p, b);
  const int tid = threadIdx.x;
  T* obase = reinterpret_cast<T*>(a.o) + (int64_t)b * a.o_stride_b;
  if (kr.nsplit == 0) {
    // No visible key: o = 0, lse = -inf (written once, by split 0).
    if (s == 0) {
      for (int idx = tid; idx < nh * D; idx += kWaves * 64) {
        const int h = idx / D, d = idx % D;
        obase[(int64_t)(hq0 + h) * a.o_stride_h + d] = (T)0.f;
      }
      if (a.lse && tid < nh) a.lse[(int64_t)b * a.lse_stride_b + hq0 + tid] = kNegInf;
    }
    return;
  }
  if (s >= kr.nsplit) return;
  const int sbeg = kr.kbeg + s * p.split;
  const int send = min(kr.kend, sbeg + p.split);

  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l16 = lane & 15;
  const int kg = lane >> 4;  // 4 lane groups of 16
  const bool head_ok = l16 < nh;
  const int qpos = kr.kend - 1;  // absolute position of the query token

  // Q^T operand: lane -> head l16, head-dim 32*ks + 8*kg + e.
  v8 qf[KS];
  {
    const T* qr = reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_stride_b +
                  (int64_t)(hq0 + min(l16, nh - 1)) * a.q_stride_h;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = head_ok ? ld_vec<v8>(qr + 32 * ks + 8 * kg) : v8{};
    if (a.rope_q && head_ok) {
      const int pos = qpos + a.rope_q_offset;
#pragma unroll
      for (int ks = 0; ks < KS / 2; ++ks) {
        const int f0 = 32 * ks + 8 * kg;
        const float* cs = a.rope_cos + (int64_t)pos * (D / 2) + f0;
        const float* sn = a.rope_sin + (int64_t)pos * (D / 2) + f0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x1 = (float)qf[ks][e], x2 = (float)qf[ks + KS / 2][e];
          qf[ks][e] = (T)(x1 * cs[e] - x2 * sn[e]);
          qf[ks + KS / 2][e] = (T)(x1 * sn[e] + x2 * cs[e]);
        }
      }
    }
  }
  const float c = p.scale_log2;
  const bool alibi = a.alibi_slopes != nullptr;
  const float slope2 = (alibi && head_ok) ? a.alibi_slopes[hq0 + l16] * kLog2e : 0.f;

  const T* kbase = reinterpret_cast<const T*>(a.k_cache) + (int64_t)b * a.k_stride_b +
                   (int64_t)hk * a.k_stride_h;
  const T* vbase = reinterpret_cast<const T*>(a.v_cache) + (int64_t)b * a.v_stride_b +
                   (int64_t)hk * a.v_stride_h;

  float acc[HMAX][CPL][8];
#pragma unroll
  for (int h = 0; h < HMAX; ++h)
#pragma unroll
    for (int i = 0; i < CPL; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][i][e] = 0.f;
  float m_run = kNegInf, l_run = 0.f;  // for head l16 over this lane's keys

  const int nchunks = (send - sbeg + kChunk - 1) / kChunk;
  for (int ch = wave; ch < nchunks; ch += kWaves) {
    const int k0 = sbeg + ch * kChunk;
    // K operand rows (clamped inside the sequence; masked below).
    const int krow = min(k0 + l16, send - 1);
    v8 kf[KS];
    const T* kp = kbase + (int64_t)krow * a.k_stride_t;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kf[ks] = ld_vec<v8>(kp + 32 * ks + 8 * kg);
    // V rows for the PV step: keys k0 + 4*kg + kk, head-dim chunk l16 (+16 i).
    v8 vf[4][CPL];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int vrow = min(k0 + 4 * kg + kk, send - 1);
      const T* vp = vbase + (int64_t)vrow * a.v_stride_t;
#pragma unroll
      for (int i = 0; i < CPL; ++i) vf[kk][i] = ld_vec<v8>(vp + 8 * (l16 + 16 * i));
    }

    f32x4 sc = f32x4{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) sc = mfma16(kf[ks], qf[ks], sc);

    // sc[r]: head l16, key k0 + 4*kg + r.
    float t[4];
    float mx = kNegInf;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = k0 + 4 * kg + r;
      float x = sc[r] * c;
      if (alibi) x = fmaf(slope2, (float)(key - qpos), x);
      t[r] = (key < send) ? x : kNegInf;
      mx = fmaxf(mx, t[r]);
    }
    mx = fmaxf(mx, shfl_xor_f(mx, 16));
    mx = fmaxf(mx, shfl_xor_f(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == kNegInf) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    m_run = m_new;
    float lsum = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float pr = fast_exp2(t[r] - m_use);
      lsum += pr;
      p_lds[wave][4 * kg + r][l16] = pr;
    }
    l_run = l_run * alpha + lsum;
    if (kg == 0) alpha_lds[wave][l16] = alpha;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // Rescale and accumulate this lane's 4 keys for every head of the slice.
#pragma unroll
    for (int h4 = 0; h4 < HMAX / 4; ++h4) {
      const f32x4 al = ld_vec<f32x4>(&alpha_lds[wave][4 * h4]);
#pragma unroll
      for (int hh = 0; hh < 4; ++hh)
#pragma unroll
        for (int i = 0; i < CPL; ++i)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[4 * h4 + hh][i][e] *= al[hh];
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      float vv[CPL][8];
#pragma unroll
      for (int i = 0; i < CPL; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) vv[i][e] = (float)vf[kk][i][e];
#pragma unroll
      for (int h4 = 0; h4 < HMAX / 4; ++h4) {
        const f32x4 pv = ld_vec<f32x4>(&p_lds[wave][4 * kg + kk][4 * h4]);
#pragma unroll
        for (int hh = 0; hh < 4; ++hh)
#pragma unroll
          for (int i = 0; i < CPL; ++i)
#pragma unroll
            for (int e = 0; e < 8; ++e)
              acc[4 * h4 + hh][i][e] = fmaf(pv[hh], vv[i][e], acc[4 * h4 + hh][i][e]);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // ---- reduce within the wave -------------------------------------------------
  l_run += shfl_xor_f(l_run, 16);
  l_run += shfl_xor_f(l_run, 32);
#pragma unroll
  for (int h = 0; h < HMAX; ++h)
#pragma unroll
    for (int i = 0; i < CPL; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float v = acc[h][i][e];
        v += shfl_xor_f(v, 16);
        v += shfl_xor_f(v, 32);
        acc[h][i][e] = v;
      }
  if (kg == 0) {
    if (l16 < HMAX) {
      red_m[wave][l16] = m_run;
      red_l[wave][l16] = l_run;
    }
#pragma unroll
    for (int h = 0; h < HMAX; ++h)
#pragma unroll
      for (int i = 0; i < CPL; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) red_o[wave][h][8 * (l16 + 16 * i) + e] = acc[h][i][e];
  }
  __syncthreads();

  // ---- merge the waves, write output or split partial --------------------------
  const bool single = kr.nsplit == 1;
  float* part_o = reinterpret_cast<float*>(a.workspace);
  float* part_lse = part_o + (int64_t)a.batch * a.heads_q * p.nsplit_max * D;
  for (int idx = tid; idx < nh * D; idx += kWaves * 64) {
    const int h = idx / D, d = idx % D;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, red_m[w][h]);
    const float Mu = (M == kNegInf) ? 0.f : M;
    float lsum = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = fast_exp2(red_m[w][h] - Mu);
      lsum = fmaf(f, red_l[w][h], lsum);
      o = fmaf(f, red_o[w][h][d], o);
    }
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    const float lse = lsum > 0.f ? (M + log2f(lsum)) * kLn2 : kNegInf;
    const int hq = hq0 + h;
    if (single) {
      obase[(int64_t)hq * a.o_stride_h + d] = (T)(o * inv);
      if (a.lse && d == 0) a.lse[(int64_t)b * a.lse_stride_b + hq] = lse;
    } else {
      const int64_t slot = ((int64_t)b * a.heads_q + hq) * p.nsplit_max + s;
      part_o[slot * D + d] = o * inv;
      if (d == 0) part_lse[slot] = lse;
    }
  }
}

template <typename T, int D>
__global__ void __launch_bounds__(D) merge_kernel(const DecodeParams p) {
  const goda_decode_args& a = p.a;
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const KeyRange kr = key_range(p, b);
  if (kr.nsplit <= 1) return;
  const int d = threadIdx.x;
  const float* part_o = reinterpret_cast<const float*>(a.workspace);
  const float* part_lse = part_o + (int64_t)a.batch * a.heads_q * p.nsplit_max * D;
  const int64_t slot0 = ((int64_t)b * a.heads_q + hq) * p.nsplit_max;
  float M = kNegInf;
  for (int s = 0; s < kr.nsplit; ++s) M = fmaxf(M, part_lse[slot0 + s]);
  const float Mu = (M == kNegInf) ? 0.f : M;
  float wsum = 0.f, o = 0.f;
  for (int s = 0; s < kr.nsplit; ++s) {
    const float w = __expf(part_lse[slot0 + s] - Mu);
    wsum += w;
    o = fmaf(w, part_o[(slot0 + s) * D + d], o);
  }
  T* out = reinterpret_cast<T*>(a.o) + (int64_t)b * a.o_stride_b + (int64_t)hq * a.o_stride_h;
  out[d] = (T)(wsum > 0.f ? o / wsum : 0.f);
  if (a.lse && d == 0) a.lse[(int64_t)b * a.lse_stride_b + hq] = wsum > 0.f ? Mu + logf(wsum) : kNegInf;
}

template <typename T, int D, int HMAX>
hipError_t launch_hd(const DecodeParams& p, hipStream_t s) {
  const goda_decode_args& a = p.a;
  const int nhs = (p.group + HMAX - 1) / HMAX;
  dim3 grid(p.nsplit_max, a.heads_kv * nhs, a.batch);
  hipError_t e = record_timing(a.timing_begin, s);
  if (e != hipSuccess) return e;
  decode_splitk_kernel<T, D, HMAX><<<grid, kWaves * 64, 0, s>>>(p);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if ((e = record_timing(a.timing_end, s)) != hipSuccess) return e;
  if (p.nsplit_max <= 1) return hipSuccess;
  merge_kernel<T, D><<<dim3(a.heads_q, a.batch), D, 0, s>>>(p);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_d(const DecodeParams& p, hipStream_t s) {
  if (p.group <= 4) return launch_hd<T, D, 4>(p, s);
  if (p.group <= 8 || D > 128) return launch_hd<T, D, 8>(p, s);
  return launch_hd<T, D, 16>(p, s);
}

template <typename T>
hipError_t launch_t(const DecodeParams& p, hipStream_t s) {
  if (p.a.head_dim == 128) return launch_d<T, 128>(p, s);
  if (p.a.head_dim == 256) return launch_d<T, 256>(p, s);
  return hipErrorNotSupported;
}

// ---------------------------------------------------------------------------
// KV append: rows [pos_b, pos_b + T_new) of sequence b receive the new k
// (rotated at its absolute position) and v, with pos_b = cache_seqlens[b] read
// on the device. One workgroup per (new row, sequence). The lengths are
// advanced by a second launch on the same stream, so every workgroup of the
// first one has read the old positions before they change.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void kv_append_kernel(const goda_kv_append_args a) {
  const int t = blockIdx.x;
  const int b = blockIdx.y;
  const int D = a.head_dim;
  const int pos = a.cache_seqlens[b] + t;
  if (pos < 0 || pos >= a.max_seqlen) return;
  const T* kn = reinterpret_cast<const T*>(a.k_new) + (int64_t)b * a.kn_stride_b +
                (int64_t)t * a.kn_stride_t;
  const T* vn = reinterpret_cast<const T*>(a.v_new) + (int64_t)b * a.vn_stride_b +
                (int64_t)t * a.vn_stride_t;
  T* kc = reinterpret_cast<T*>(a.k_cache) + (int64_t)b * a.k_stride_b + (int64_t)pos * a.k_stride_t;
  T* vc = reinterpret_cast<T*>(a.v_cache) + (int64_t)b * a.v_stride_b + (int64_t)pos * a.v_stride_t;
  const int half = D / 2;
  for (int idx = threadIdx.x; idx < a.heads_kv * half; idx += blockDim.x) {
    const int h = idx / half, i = idx % half;
    const float x1 = Elem<T>::to_f32(kn[(int64_t)h * a.kn_stride_h + i]);
    const float x2 = Elem<T>::to_f32(kn[(int64_t)h * a.kn_stride_h + i + half]);
    float y1 = x1, y2 = x2;
    if (a.rope_k) {
      const int rp = pos + a.rope_k_offset;
      const float cc = a.rope_cos[(int64_t)rp * half + i], ss = a.rope_sin[(int64_t)rp * half + i];
      y1 = x1 * cc - x2 * ss;
      y2 = x1 * ss + x2 * cc;
    }
    kc[(int64_t)h * a.k_stride_h + i] = Elem<T>::from_f32(y1);
    kc[(int64_t)h * a.k_stride_h + i + half] = Elem<T>::from_f32(y2);
    vc[(int64_t)h * a.v_stride_h + i] = vn[(int64_t)h * a.vn_stride_h + i];
    vc[(int64_t)h * a.v_stride_h + i + half] = vn[(int64_t)h * a.vn_stride_h + i + half];
  }
}

__global__ void kv_bump_kernel(int32_t* seqlens, int n, int add) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b < n) seqlens[b] += add;
}

template <typename T>
hipError_t launch_append_t(const goda_kv_append_args& a, hipStream_t s) {
  if (a.seqlen_new > 0) {
    kv_append_kernel<T><<<dim3(a.seqlen_new, a.batch), 256, 0, s>>>(a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  kv_bump_kernel<<<(a.batch + 255) / 256, 256, 0, s>>>(a.cache_seqlens, a.batch, a.seqlen_new);
  return hipGetLastError();
}

}  // namespace

bool decode_mfma_supported(const goda_decode_args& a) {
  if (a.dtype != GODA_DTYPE_BF16 && a.dtype != GODA_DTYPE_F16) return false;
  return a.head_dim == 128 || a.head_dim == 256;
}

int decode_default_split(const goda_decode_args& a) {
  // Aim for ~4096 workgroups with the cache assumed half full; splits are a
  // multiple of one workgroup step (4 waves x 16 keys).
  const int group = a.heads_q / a.heads_kv;
  const int hmax = group <= 4 ? 4 : (group <= 8 || a.head_dim > 128) ? 8 : 16;
  const int64_t units = (int64_t)a.batch * a.heads_kv * ((group + hmax - 1) / hmax);
  const int64_t keys = units * ((int64_t)a.max_seqlen / 2 + 1);
  int split = 256;
  while (split < 4096 && keys / split > 4096) split *= 2;
  return split;
}

int64_t decode_workspace_bytes(const goda_decode_args& a, int split) {
  const int64_t nsplit = ((int64_t)a.max_seqlen + split - 1) / split;
  if (nsplit <= 1) return 0;
  return (int64_t)a.batch * a.heads_q * nsplit * (a.head_dim + 1) * 4;
}

hipError_t launch_decode(const DecodeParams& p, hipStream_t s) {
  if (p.a.dtype == GODA_DTYPE_BF16) return launch_t<bf16>(p, s);
  if (p.a.dtype == GODA_DTYPE_F16) return launch_t<f16>(p, s);
  return hipErrorNotSupported;
}

hipError_t launch_kv_append(const goda_kv_append_args& a, hipStream_t s) {
  switch (a.dtype) {
    case GODA_DTYPE_F32:
      return launch_append_t<float>(a, s);
    case GODA_DTYPE_F16:
      return launch_append_t<f16>(a, s);
    case GODA_DTYPE_BF16:
      return launch_append_t<bf16>(a, s);
    default:
      return hipErrorNotSupported;
  }
}

}  // namespace goda
