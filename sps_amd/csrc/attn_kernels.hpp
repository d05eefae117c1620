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

// Work plan of one workgroup, written by the prepass (when documents are given) in dispatch order,
// heaviest first, so a workgroup needs one load to start fetching its first tiles.
struct TilePlan {
  int tile;    // query tile (forward, dQ) or key tile (dK/dV) of the row
  int mono;    // 1 when the row's ids are non-decreasing
  int b0, n0;  // query tile: stream-0 key blocks b0 .. b0 + n0 - 1; key tile: query chunks
  int b1, n1;  // query tile: temporary-stream key blocks b1 .. b1 + n1 - 1; key tile: unused
  int pad0, pad1;
};

// First block and block count of the 32-row blocks covering the index interval [lo, hi] (lo >= 0).
__host__ __device__ __forceinline__ void cover_blocks(int lo, int hi, int& first, int& count) {
  first = hi >= lo ? lo / kBlock : 0;
  count = hi >= lo ? hi / kBlock - first + 1 : 0;
}

// Workgroup barrier ordering LDS accesses only (fences limited to the local address space):
// global stores issued before it keep draining, where __syncthreads() would wait for them.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;
  const uint16_t* dO;
  uint16_t* out;  // forward: O
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  Strides3 sq, sk, sv, so, sdo, sout, sdq, sdk, sdv;
  float* lse;        // [B, H, N] log2-domain log-sum-exp of the scaled scores
  float* seeds;      // [B, H, 2, N] backward: -LSE (0 where LSE = -inf) and -Delta = -rowsum(O * dO)
  const void* docs;  // [B, N] int32 or int64 document ids (unit stride along N), or null
  int docs_i64;
  int64_t docs_sb;
  // Row layout written by the prepass when docs are given (workspace), else null:
  int* run_start;  // [B, N] first position of the run of equal ids containing each position
  int* run_end;    // [B, N] last position of that run
  int* row_mono;   // [B] 1 when the row's ids are non-decreasing (runs are the documents)
  TilePlan* q_plan;  // [B, q_tiles] query-tile plans, heaviest first
  TilePlan* k_plan;  // [B, k_tiles] key-tile plans, heaviest first
  int B, H;
  FastDiv div_bh, div_b, div_h;  // B H, B and H (workgroup -> row, head, rank)
  float sm_scale;
  float scale2;  // sm_scale * log2(e)
  MaskSpec m;
  uint8_t* mask_out;  // mask-dump kernels: [B, N, N]
};

__device__ __forceinline__ int64_t load_doc(const AttnArgs& a, int b, int pos) {
  if (a.docs_i64) return reinterpret_cast<const int64_t*>(a.docs)[b * a.docs_sb + pos];
  return reinterpret_cast<const int32_t*>(a.docs)[b * a.docs_sb + pos];
}

// Row view used by the kernels: run bounds of a position and whether ids need an exact check.
struct RowView {
  const int* start;  // null: no documents (one run covering the row)
  const int* end;
  bool mono;
  __device__ __forceinline__ int run_start(int p) const { return start ? start[p] : 0; }
  __device__ __forceinline__ int run_end(int p, int N) const { return end ? end[p] : N - 1; }
};

// mono < 0: read the row's flag from the prepass output.
__device__ __forceinline__ RowView row_view(const AttnArgs& a, int b, int mono = -1) {
  RowView r;
  if (a.m.has_docs) {
    r.start = a.run_start + (int64_t)b * a.m.N;
    r.end = a.run_end + (int64_t)b * a.m.N;
    r.mono = (mono < 0 ? a.row_mono[b] : mono) != 0;
  } else {
    r.start = nullptr;
    r.end = nullptr;
    r.mono = true;
  }
  return r;
}

// Plan of workgroup rank `rank` of row b (heaviest first). Without documents no prepass runs: the
// tile follows the closed-form order (later query tiles see more keys, earlier key tiles are seen
// by more queries) and the block ranges are left for the kernel to derive (n0 = -1).
__device__ __forceinline__ TilePlan q_plan_of(const AttnArgs& a, int b, int rank) {
  const int nqt = q_tiles(a.m.N);
  if (a.m.has_docs) return a.q_plan[(int64_t)b * nqt + rank];
  return TilePlan{nqt - 1 - rank, 1, 0, -1, 0, 0, 0, 0};
}

__device__ __forceinline__ TilePlan k_plan_of(const AttnArgs& a, int b, int rank) {
  const int nkt = k_tiles(a.m.family, a.m.N, a.m.P);
  if (a.m.has_docs) return a.k_plan[(int64_t)b * nkt + rank];
  return TilePlan{rank, 1, 0, -1, 0, 0, 0, 0};
}

// Backward passes (bit mask): kBwdDq computes Delta = rowsum(O * dO) and dQ; kBwdDkdv computes dK and dV
// from the Delta the dQ pass stored.
constexpr int kBwdDq = 1;
constexpr int kBwdDkdv = 2;

// Host launchers (each defined next to its kernels). All launches are asynchronous on `stream`.
hipError_t launch_row_layout(const AttnArgs& a, hipStream_t stream);
hipError_t launch_attn_fwd(const AttnArgs& a, int D, int is_f16, hipStream_t stream);
hipError_t launch_attn_bwd(const AttnArgs& a, int D, int is_f16, int passes, hipStream_t stream);
hipError_t launch_mask_dump(const AttnArgs& a, int schedule, hipStream_t stream);

}  // namespace sps
