// Row-layout prepass of the attention kernels (one workgroup per batch row).
//
// From a row's document ids it writes, for every position, the first and last position of the
// maximal run of equal ids containing it, and whether the row's ids are non-decreasing. In a
// non-decreasing row every document is one run, so the attention kernels turn the document mask
// into interval bounds (see attn_sched.hpp). A row with decreasing steps is recorded as one run
// covering the row (start 0, end N - 1) and the kernels compare ids pair by pair there.
//
// It also writes the work plan of every query tile and key tile (the 32-row blocks covering the
// union of the tile's lanes' visible intervals, per stream: exactly what the kernels would derive
// from the run bounds, in closed form from the tile's first and last rows) in decreasing order of block count, so the heaviest workgroups are
// dispatched first and each workgroup starts its first tile loads after reading one plan. The order
// only affects speed: it is always a permutation of the tiles.
#include "attn_kernels.hpp"

namespace sps {

constexpr int kPrepThreads = 1024;
constexpr int kRegIds = 8;  // ids per thread held in registers (rows up to kPrepThreads * kRegIds positions)
constexpr int kMaxSortTiles = 2048;  // rows with more tiles keep the closed-form order
constexpr int kLdsRow = kPrepThreads * kRegIds;  // rows up to this length keep their runs in LDS

// Exclusive scans of the per-thread chunk summaries, both in one pass so their latencies overlap:
// a max-scan of `up` in thread order and a min-scan of `down` in reverse thread order. Inside each
// wave: DPP shifts within the 16-lane rows (no LDS round trips), then the rows' totals from one lane
// each; across the waves: their totals through LDS, read back as vectors (two barriers in all).
constexpr int kPrepWaves = kPrepThreads / 64;
static_assert(kPrepWaves == 16, "the wave totals are read back as four int4 vectors");

template <int CTRL>
__device__ __forceinline__ int dpp_shift(int x, int id) {
  // Lanes whose source lane lies outside the shift's range get `id`.
  return __builtin_amdgcn_update_dpp(id, x, CTRL, 0xF, 0xF, false);
}

__device__ void block_exclusive_scans(int* s_up, int* s_down, int up, int down, int up_identity, int down_identity,
                                      int& up_ex, int& down_ex) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, row = lane >> 4;
  const int iu = up_identity, id = down_identity;
  // Inclusive max-scan upward (row_shr 1, 2, 4, 8) and min-scan downward (row_shl 1, 2, 4, 8) per row.
  int u = up, d = down;
  u = imax(u, dpp_shift<0x111>(u, iu));
  d = imin(d, dpp_shift<0x101>(d, id));
  u = imax(u, dpp_shift<0x112>(u, iu));
  d = imin(d, dpp_shift<0x102>(d, id));
  u = imax(u, dpp_shift<0x114>(u, iu));
  d = imin(d, dpp_shift<0x104>(d, id));
  u = imax(u, dpp_shift<0x118>(u, iu));
  d = imin(d, dpp_shift<0x108>(d, id));
  // Across the rows: row r adds the totals of rows below it (up) / above it (down).
  const int t0 = __builtin_amdgcn_readlane(u, 15), t1 = __builtin_amdgcn_readlane(u, 31);
  const int t2 = __builtin_amdgcn_readlane(u, 47), t3 = __builtin_amdgcn_readlane(u, 63);
  const int p1 = t0, p2 = imax(t0, t1), p3 = imax(p2, t2);
  u = imax(u, row == 0 ? iu : row == 1 ? p1 : row == 2 ? p2 : p3);
  const int b0 = __builtin_amdgcn_readlane(d, 0), b1 = __builtin_amdgcn_readlane(d, 16);
  const int b2 = __builtin_amdgcn_readlane(d, 32), b3 = __builtin_amdgcn_readlane(d, 48);
  const int s2 = b3, s1 = imin(b2, b3), s0 = imin(b1, s1);
  d = imin(d, row == 3 ? id : row == 2 ? s2 : row == 1 ? s1 : s0);
  if (lane == 0) {
    s_up[wave] = imax(p3, t3);
    s_down[wave] = imin(b0, s0);
  }
  // The lane's exclusive value inside the wave: its neighbour's inclusive one (wave_shr / wave_shl 1).
  const int eu = dpp_shift<0x138>(u, iu), ed = dpp_shift<0x130>(d, id);
  __syncthreads();
  int cu = iu, cd = id;
#pragma unroll
  for (int k = 0; k < kPrepWaves / 4; ++k) {
    const int4 vu = reinterpret_cast<const int4*>(s_up)[k], vd = reinterpret_cast<const int4*>(s_down)[k];
    const int w = 4 * k;
    cu = imax(cu, w + 0 < wave ? vu.x : iu);
    cu = imax(cu, w + 1 < wave ? vu.y : iu);
    cu = imax(cu, w + 2 < wave ? vu.z : iu);
    cu = imax(cu, w + 3 < wave ? vu.w : iu);
    cd = imin(cd, w + 0 > wave ? vd.x : id);
    cd = imin(cd, w + 1 > wave ? vd.y : id);
    cd = imin(cd, w + 2 > wave ? vd.z : id);
    cd = imin(cd, w + 3 > wave ? vd.w : id);
  }
  __syncthreads();  // the wave totals may be overwritten by a later scan
  up_ex = imax(cu, eu);
  down_ex = imin(cd, ed);
}

// Minimum / maximum over each group of 8 consecutive lanes (all lanes active), held by every lane
// of the group: quad swaps, then the half-row mirror.
template <class Op>
__device__ __forceinline__ int group8_reduce(int x, Op op) {
  x = op(x, __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));   // quad_perm [1, 0, 3, 2]
  x = op(x, __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));   // quad_perm [2, 3, 0, 1]
  return op(x, __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, false));  // row_half_mirror
}
__device__ __forceinline__ int group8_min(int x) { return group8_reduce(x, [](int u, int v) { return imin(u, v); }); }
__device__ __forceinline__ int group8_max(int x) { return group8_reduce(x, [](int u, int v) { return imax(u, v); }); }

// Ranks `n` <= kMaxSortTiles tiles by decreasing cost (ties: lower index first) and calls
// emit(rank, tile) for each, with threads [first, first + count) of the workgroup (rank sort; the
// cost reads are batched so their LDS latencies overlap).
template <class Emit>
__device__ void sort_tiles(const int* cost, int n, int first, int count, Emit emit) {
  const int tid = threadIdx.x - first;
  if (tid < 0 || tid >= count) return;
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
    emit(r, t);
  }
}

__global__ __launch_bounds__(kPrepThreads) void row_layout_kernel(const AttnArgs a) {
  __shared__ __attribute__((aligned(16))) int s_scan[kPrepThreads];
  __shared__ int s_cost[kMaxSortTiles], s_cost_k[kMaxSortTiles];
  __shared__ int s_qplan[kMaxSortTiles][4], s_kplan[kMaxSortTiles][2];
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
    // Common case: every id of this thread's chunk (and its predecessor) loaded once, together: one
    // branch on the id type around straight-line loads whose positions are clamped into the row
    // (values past the chunk are never used), so all of them are in flight at once.
    int64_t before = 0;
    auto load_all = [&](auto* ids) {
      ids += (int64_t)b * a.docs_sb;
      const int64_t bv = ids[imax(imin(p0, N) - 1, 0)];
#pragma unroll
      for (int j = 0; j < kRegIds; ++j) d[j] = ids[imin(p0 + j, N - 1)];
      before = (p0 > 0 && p0 < N) ? bv : 0;
    };
    if (a.docs_i64)
      load_all(reinterpret_cast<const int64_t*>(a.docs));
    else
      load_all(reinterpret_cast<const int32_t*>(a.docs));
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
  int carry_start, carry_next;
  block_exclusive_scans(s_scan, s_scan + kPrepWaves, last, first, -1, N, carry_start, carry_next);
  const bool mono = s_nonmono == 0;

  if (mono && in_regs) {
    // LDS copies only; the global arrays are written from them below with coalesced stores.
    int cur = carry_start;
#pragma unroll
    for (int j = 0; j < kRegIds; ++j) {
      if (flag[j]) cur = p0 + j;
      if (p0 + j < p1) s_start[p0 + j] = (short)cur;
    }
    int nxt = carry_next;
#pragma unroll
    for (int j = kRegIds - 1; j >= 0; --j) {
      if (p0 + j < p1) s_end[p0 + j] = (short)(nxt - 1);
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
      if (in_regs) {
        s_start[p] = 0;
        s_end[p] = (short)(N - 1);
      } else {
        start[p] = 0;
        end[p] = N - 1;
      }
    }
  }
  if (tid == 0) a.row_mono[b] = mono ? 1 : 0;
  __syncthreads();  // start/end of the whole row are visible to every thread below
  if (in_regs) {
    // Rows held in LDS go to global memory now: one pass of consecutive positions per thread group,
    // 4 per thread (16-byte stores) when the row length allows; the stores drain while the plans
    // below are computed (the barrier before the sorts is the first to wait for them).
    if ((N & 3) == 0) {
      for (int p = 4 * tid; p < N; p += 4 * kPrepThreads) {
        *reinterpret_cast<int4*>(start + p) = make_int4(s_start[p], s_start[p + 1], s_start[p + 2], s_start[p + 3]);
        *reinterpret_cast<int4*>(end + p) = make_int4(s_end[p], s_end[p + 1], s_end[p + 2], s_end[p + 3]);
      }
    } else {
      for (int p = tid; p < N; p += kPrepThreads) {
        start[p] = s_start[p];
        end[p] = s_end[p];
      }
    }
  }
  // Rows that fit read their run bounds from LDS (short: positions < kLdsRow <= 32767).
  const bool lds_ok = in_regs;

  // Query-tile and key-tile plans, then both sorts. Rows with more than
  // kMaxSortTiles tiles keep the closed-form order (query tiles last to first, key tiles first to
  // last) and write their plans directly.
  const int nqt = q_tiles(N);
  const int nkt = k_tiles(m.family, N, m.P);
  const bool sort_q = nqt <= kMaxSortTiles, sort_k = nkt <= kMaxSortTiles;
  TilePlan* qplan = a.q_plan + (int64_t)b * nqt;
  TilePlan* kplan = a.k_plan + (int64_t)b * nkt;
  const int mono_flag = mono ? 1 : 0;
  // One 8-lane group per tile, one lane per row of the tile's first and last kTileEnds rows (the
  // rows q_tile_union / k_tile_union take), the group's intervals combined by three DPP steps:
  // query tiles on waves 0-7, key tiles on waves 8-15 (no wave runs both paths), 64 tiles per pass.
  // The run bounds come from LDS or from global memory in two separate copies of the loop: with a
  // global read anywhere in it, the loads' waits (vmcnt counts stores too) would also wait for the
  // run-bound stores above.
  static_assert(2 * kTileEnds == 8, "one lane of an 8-lane group per end row");
  const bool key_half = tid >= kPrepThreads / 2;
  const int lt = tid & (kPrepThreads / 2 - 1), grp = lt >> 3, row8 = lt & 7;
  auto plans = [&](auto st_of, auto en_of) {
    const int n = key_half ? nkt : nqt;
    for (int t0 = 0; t0 < n; t0 += kPrepThreads / 16) {
      const int t = t0 + grp;
      if (!key_half) {
        Interval i0 = {kEmptyLo, kEmptyHi}, i1 = i0;
        const int q = t < n ? q_tile_row(m, t, row8) : -1;
        if (q >= 0) query_intervals(m, q, st_of(q), i0, i1);
        const Interval u0 = {group8_min(i0.lo), group8_max(i0.hi)}, u1 = {group8_min(i1.lo), group8_max(i1.hi)};
        if (t < n && row8 == 0) {
          int b0, n0, b1, n1;
          cover_blocks(u0.lo, u0.hi, b0, n0);
          cover_blocks(u1.lo, u1.hi, b1, n1);
          if (sort_q) {
            s_cost[t] = n0 + n1;
            s_qplan[t][0] = b0;
            s_qplan[t][1] = n0;
            s_qplan[t][2] = b1;
            s_qplan[t][3] = n1;
          } else {
            qplan[nqt - 1 - t] = TilePlan{t, mono_flag, b0, n0, b1, n1, 0, 0};
          }
        }
      } else {
        Interval r = {kEmptyLo, kEmptyHi};
        int stream = STREAM_NATURAL;
        const int kp = t < n ? k_tile_row(m, t, row8, stream) : -1;
        if (kp >= 0) {
          const int last = key_last_query(m, stream, kp, en_of(kp));
          if (last >= kp) r = Interval{kp, last};
        }
        const Interval k = {group8_min(r.lo), group8_max(r.hi)};
        if (t < n && row8 == 0) {
          int c0, nc;
          cover_blocks(k.lo, k.hi, c0, nc);
          if (sort_k) {
            s_cost_k[t] = nc;
            s_kplan[t][0] = c0;
            s_kplan[t][1] = nc;
          } else {
            kplan[t] = TilePlan{t, mono_flag, c0, nc, 0, 0, 0, 0};
          }
        }
      }
    }
  };
  if (lds_ok)
    plans([&](int q) { return (int)s_start[q]; }, [&](int k) { return (int)s_end[k]; });
  else
    plans([&](int q) { return start[q]; }, [&](int k) { return end[k]; });
  lds_barrier();  // the plans and costs are in LDS; the run-bound stores above keep draining
  if (sort_q)
    sort_tiles(s_cost, nqt, 0, kPrepThreads / 2, [&](int r, int t) {
      qplan[r] = TilePlan{t, mono_flag, s_qplan[t][0], s_qplan[t][1], s_qplan[t][2], s_qplan[t][3], 0, 0};
    });
  if (sort_k)
    sort_tiles(s_cost_k, nkt, kPrepThreads / 2, kPrepThreads / 2, [&](int r, int t) {
      kplan[r] = TilePlan{t, mono_flag, s_kplan[t][0], s_kplan[t][1], 0, 0, 0, 0};
    });
}

hipError_t launch_row_layout(const AttnArgs& a, hipStream_t stream) {
  if (a.B == 0 || a.m.N == 0 || !a.m.has_docs) return hipSuccess;
  hipLaunchKernelGGL(row_layout_kernel, dim3(a.B), dim3(kPrepThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace sps
