// Host-side launcher declarations shared between the C-ABI layer (api.hip)
// and the kernel translation units. Internal to libgoda_attn.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "goda_attn.h"

namespace goda {

// Launch-ready prefill parameters: the caller's arguments plus values derived
// once on the host.
struct PrefillParams {
  goda_prefill_args a;
  int group;          // heads_q / heads_kv
  float scale_log2;   // softmax_scale * log2(e)
  int kv_tile;        // keys per workspace tile (MFMA path)
  int ntiles_k;       // ceil(seqlen_k / kv_tile)
  int heads_per_wg;   // query heads sharing one workgroup (MFMA path)
};

struct DecodeParams {
  goda_decode_args a;
  int group;
  float scale_log2;
  int split;          // keys per work range; 0: balanced over the grid
  int grid;           // persistent workgroups (set by the launcher)
  int64_t nslots;     // partial slots in the workspace
};

// Generic (VALU) prefill: any dtype, head_dim in {64,128,256}.
hipError_t launch_prefill_generic(const PrefillParams& p, hipStream_t s);

// MFMA prefill for bf16/fp16, head_dim in {64,128,256}. Returns
// hipErrorNotSupported when no tuned instance covers the arguments.
bool prefill_mfma_supported(const goda_prefill_args& a);
int64_t prefill_mfma_workspace_bytes(const goda_prefill_args& a);
hipError_t launch_prefill_mfma(const PrefillParams& p, hipStream_t s);

// Split-K decode for bf16/fp16; fp32 decode goes through the generic prefill.
bool decode_mfma_supported(const goda_decode_args& a);
int64_t decode_slots(const goda_decode_args& a);
int64_t decode_workspace_bytes(const goda_decode_args& a);
hipError_t launch_decode(const DecodeParams& p, hipStream_t s);

hipError_t launch_kv_append(const goda_kv_append_args& a, hipStream_t s);

// Records the caller's optional timing event (a hipEvent_t or NULL) on s.
inline hipError_t record_timing(void* ev, hipStream_t s) {
  if (!ev) return hipSuccess;
  return hipEventRecord(reinterpret_cast<hipEvent_t>(ev), s);
}

}  // namespace goda
