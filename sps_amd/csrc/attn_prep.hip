// Row-layout prepass of the attention kernels (one workgroup per batch row).
//
// From a row's document ids it writes, for every position, the first and last position of the
// maximal run of equal ids containing it, and whether the row's ids are non-decreasing. In a
// non-decreasing row every document is one run, so the attention kernels turn the document mask
// into interval bounds (see attn_sched.hpp). A row with decreasing steps is recorded as one run
// covering the row (start 0, end N - 1) and the kernels compare ids pair by pair there.
//
// It also writes the row's query tiles and key tiles in decreasing order of their (approximate)
// number of MFMA blocks, so the heaviest workgroups are dispatched first. The order only affects
// speed: it is always a permutation of the tiles.
#include "attn_kernels.hpp"

namespace sps {

constexpr int kPrepThreads = 1024;
constexpr int kRegIds = 8;  // ids per thread held in registers (rows up to kPrepThreads * kRegIds positions)
constexpr int kMaxSortTiles = 2048;  // rows with more tiles keep the closed-form order
constexpr int kLdsRow = kPrepThreads * kRegIds;  // rows up to this length keep their runs in LDS

__device__ __forceinline__ int blocks_in(int lo, int hi) {
  return hi >= lo ? (hi >> 5) - (lo >> 5) + 1 : 0;
}

// Run bounds of a position, from the LDS copy (rows up to kLdsRow) or from global memory.
struct RunBounds {
  const short* s_lds;
  const short* e_lds;
  const int* s_glb;
  const int* e_glb;
  __device__ __forceinline__ int start(int p) const { return s_lds ? s_lds[p] : s_glb[p]; }
  __device__ __forceinline__ int end(int p) const { return e_lds ? e_lds[p] : e_glb[p]; }
};

// Key blocks of the query tile qt (both streams), from its first and last queries' intervals.
__device__ int q_tile_cost(const MaskSpec& m, const RunBounds& rb, int qt) {
  const int qa = qt * kTile, qz = imin(qa + kTile - 1, m.N - 1);
  Interval a0, a1, z0, z1;
  query_intervals(m, qa, rb.start(qa), a0, a1);
  query_intervals(m, qz, rb.start(qz), z0, z1);
  return blocks_in(imin(a0.lo, z0.lo), imax(a0.hi, z0.hi)) + blocks_in(imin(a1.lo, z1.lo), imax(a1.hi, z1.hi));
}

// Query chunks of the key tile kt, from its first key and the last query of its last key.
__device__ int k_tile_cost(const MaskSpec& m, const RunBounds& rb, int kt) {
  int stream, first;
  k_tile_run(m, kt, stream, first);
  const int len = stream_len(m.family, m.N, stream, m.P);
  const int last = imin(first + kTile - 1, len - 1);
  const int k0 = stream_pos(m, stream, first), k1 = stream_pos(m, stream, last);
  return blocks_in(k0, key_last_query(m, stream, k1, rb.end(k1)));
}

// Exclusive scan of the per-thread chunk summaries in thread order (reverse: in reverse thread
// order) for an associative, commutative op: a shuffle scan inside each wave, then the waves'
// totals through LDS (two barriers in all).
constexpr int kPrepWaves = kPrepThreads / 64;

template <class Op>
__device__ int block_exclusive_scan(int* s, int x, int identity, Op op, bool reverse) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int v = x;  // inclusive scan within the wave
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = reverse ? __shfl_down(v, o) : __shfl_up(v, o);
    if (reverse ? lane + o < 64 : lane >= o) v = op(v, y);
  }
  const int wslot = reverse ? kPrepWaves - 1 - wave : wave;
  if (reverse ? lane == 0 : lane == 63) s[wslot] = v;
  __syncthreads();
  int carry = identity;
  for (int w = 0; w < wslot; ++w) carry = op(carry, s[w]);
  int ex = reverse ? __shfl_down(v, 1) : __shfl_up(v, 1);
  if (reverse ? lane == 63 : lane == 0) ex = identity;
  __syncthreads();  // the wave totals may be overwritten by the next scan
  return op(carry, ex);
}

// Writes the order of `n` tiles by decreasing cost (ties: lower index first) into order[0..n),
// with threads [first, first + count) of the workgroup (rank sort; the cost reads are batched so
// their LDS latencies overlap).
__device__ void sort_tiles(const int* cost, int n, int* order, bool ascending_fallback, int first, int count) {
  const int tid = threadIdx.x - first;
  if (tid < 0 || tid >= count) return;
  if (n > kMaxSortTiles) {
    for (int t = tid; t < n; t += count) order[t] = ascending_fallback ? t : n - 1 - t;
    return;
  }
  for (int t = tid; t < n; t += count) {
    const int c = cost[t];
    int r = 0, j = 0;
    for (; j + 8 <= n; j += 8) {
      int x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = cost[j + u];
#pragma unroll
      for (int u = 0; u < 8; ++u) r += (x[u] > c) || (x[u] == c && j + u < t);
    }
    for (; j < n; ++j) r += (cost[j] > c) || (cost[j] == c && j < t);
    order[r] = t;
  }
}

__global__ __launch_bounds__(kPrepThreads) void row_layout_kernel(const AttnArgs a) {
  __shared__ int s_scan[kPrepThreads];
  __shared__ int s_cost[kMaxSortTiles], s_cost_k[kMaxSortTiles];
  __shared__ int s_nonmono;
  __shared__ short s_start[kLdsRow], s_end[kLdsRow];
  const MaskSpec m = a.m;
  const int b = blockIdx.x, tid = threadIdx.x, N = m.N;
  int* start = a.run_start + (int64_t)b * N;
  int* end = a.run_end + (int64_t)b * N;
  const int C = (N + kPrepThreads - 1) / kPrepThreads;
  const int p0 = imin(tid * C, N), p1 = imin(p0 + C, N);
  if (tid == 0) s_nonmono = 0;

  const bool in_regs = C <= kRegIds;
  int last = -1, first = N;
  bool dec = false;
  int64_t d[kRegIds];
  bool flag[kRegIds];
  if (in_regs) {
    // Common case: every id of this thread's chunk (and its predecessor) loaded once, together.
    const int64_t before = (p0 > 0 && p0 < N) ? load_doc(a, b, p0 - 1) : 0;
#pragma unroll
    for (int j = 0; j < kRegIds; ++j) d[j] = p0 + j < p1 ? load_doc(a, b, p0 + j) : 0;
#pragma unroll
    for (int j = 0; j < kRegIds; ++j) {
      const int p = p0 + j;
      const int64_t prev = j == 0 ? before : d[j - 1];
      flag[j] = p < p1 && (p == 0 || d[j] != prev);
      dec |= p < p1 && p > 0 && d[j] < prev;
      if (flag[j]) {
        last = p;
        first = imin(first, p);
      }
    }
  } else {
    int64_t prev = p0 > 0 ? load_doc(a, b, p0 - 1) : 0;
    for (int p = p0; p < p1; ++p) {
      const int64_t x = load_doc(a, b, p);
      if (p == 0 || x != prev) {
        last = p;
        first = imin(first, p);
      }
      dec |= (p > 0 && x < prev);
      prev = x;
    }
  }
  __syncthreads();
  if (dec) atomicOr(&s_nonmono, 1);
  const int carry_start = block_exclusive_scan(s_scan, last, -1, [](int x, int y) { return imax(x, y); }, false);
  const int carry_next = block_exclusive_scan(s_scan, first, N, [](int x, int y) { return imin(x, y); }, true);
  const bool mono = s_nonmono == 0;

  if (mono && in_regs) {
    int cur = carry_start;
#pragma unroll
    for (int j = 0; j < kRegIds; ++j) {
      if (flag[j]) cur = p0 + j;
      if (p0 + j < p1) {
        start[p0 + j] = cur;
        s_start[p0 + j] = (short)cur;
      }
    }
    int nxt = carry_next;
#pragma unroll
    for (int j = kRegIds - 1; j >= 0; --j) {
      if (p0 + j < p1) {
        end[p0 + j] = nxt - 1;
        s_end[p0 + j] = (short)(nxt - 1);
      }
      if (flag[j]) nxt = p0 + j;
    }
  } else if (mono) {
    int cur = carry_start;
    int64_t prev = p0 > 0 ? load_doc(a, b, p0 - 1) : 0;
    for (int p = p0; p < p1; ++p) {
      const int64_t x = load_doc(a, b, p);
      if (p == 0 || x != prev) cur = p;
      start[p] = cur;
      prev = x;
    }
    int nxt = carry_next;
    for (int p = p1 - 1; p >= p0; --p) {
      end[p] = nxt - 1;
      if (p == 0 || load_doc(a, b, p) != load_doc(a, b, p - 1)) nxt = p;
    }
  } else {
    for (int p = p0; p < p1; ++p) {
      start[p] = 0;
      end[p] = N - 1;
      if (in_regs) {
        s_start[p] = 0;
        s_end[p] = (short)(N - 1);
      }
    }
  }
  if (tid == 0) a.row_mono[b] = mono ? 1 : 0;
  __syncthreads();  // start/end of the whole row are visible to every thread below
  // Rows that fit read their run bounds from LDS (short: positions < kLdsRow <= 32767).
  const bool lds_ok = in_regs;
  const RunBounds rb = {lds_ok ? s_start : nullptr, lds_ok ? s_end : nullptr, start, end};

  // Query-tile and key-tile orders (independent: both cost passes, one barrier, both sorts).
  const int nqt = q_tiles(N);
  const int nkt = k_tiles(m.family, N, m.P);
  if (nqt <= kMaxSortTiles)
    for (int t = tid; t < nqt; t += kPrepThreads) s_cost[t] = q_tile_cost(m, rb, t);
  if (nkt <= kMaxSortTiles)
    for (int t = tid; t < nkt; t += kPrepThreads) s_cost_k[t] = k_tile_cost(m, rb, t);
  __syncthreads();
  sort_tiles(s_cost, nqt, a.q_order + (int64_t)b * nqt, false, 0, kPrepThreads / 2);
  sort_tiles(s_cost_k, nkt, a.k_order + (int64_t)b * nkt, true, kPrepThreads / 2, kPrepThreads / 2);
}

hipError_t launch_row_layout(const AttnArgs& a, hipStream_t stream) {
  if (a.B == 0 || a.m.N == 0 || !a.m.has_docs) return hipSuccess;
  hipLaunchKernelGGL(row_layout_kernel, dim3(a.B), dim3(kPrepThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace sps
