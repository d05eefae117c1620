// Kernel argument block and host-side launch declarations for the attention kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_sched.hpp"

namespace sps {

// Element strides of a [B, H, N, D] view whose D axis is contiguous.
struct Strides3 {
  int64_t b, h, n;
};

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;
  const uint16_t* dO;
  uint16_t* out;  // forward: O; unused by the backward kernels
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  Strides3 sq, sk, sv, so, sdo, sout, sdq, sdk, sdv;
  float* lse;          // [B, H, N] log2-domain log-sum-exp of the scaled scores
  float* delta;        // [B, H, N] rowsum(O * dO) (backward)
  const void* docs;    // [B, N] int32 or int64 document ids (unit stride along N), or null
  int docs_i64;
  int64_t docs_sb;
  int64_t* gmin;  // [B, NG] per-granule min/max document id (written by the prepass)
  int64_t* gmax;
  int NG;
  int B, H;
  float sm_scale;
  float scale2;  // sm_scale * log2(e)
  MaskSpec m;
  uint8_t* mask_out;  // mask-dump kernels: [B, N, N]
};

__device__ __forceinline__ int64_t load_doc(const AttnArgs& a, int b, int pos) {
  if (a.docs_i64) return reinterpret_cast<const int64_t*>(a.docs)[b * a.docs_sb + pos];
  return reinterpret_cast<const int32_t*>(a.docs)[b * a.docs_sb + pos];
}

// Host launchers (each defined next to its kernels). All launches are asynchronous on `stream`.
hipError_t launch_doc_granules(const AttnArgs& a, hipStream_t stream);
hipError_t launch_attn_fwd(const AttnArgs& a, int D, int is_f16, hipStream_t stream);
// Backward passes (bit mask): kBwdDq computes Delta = rowsum(O * dO) and dQ; kBwdDkdv computes dK and dV
// from the Delta the dQ pass stored.
constexpr int kBwdDq = 1;
constexpr int kBwdDkdv = 2;
hipError_t launch_attn_bwd(const AttnArgs& a, int D, int is_f16, int passes, hipStream_t stream);
hipError_t launch_mask_dump(const AttnArgs& a, int schedule, hipStream_t stream);

}  // namespace sps
