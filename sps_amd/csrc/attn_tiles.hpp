// Global -> register -> LDS staging of 32-row tiles and the per-element visibility tests shared by
// the attention kernels and the mask-dump kernels.
#pragma once
#include <type_traits>

#include "attn_kernels.hpp"
#include "cdna4.hpp"

namespace sps {

// LDS tile geometry. Rows are padded by 16 bytes so that the 32 rows read by one MFMA fragment
// land on distinct bank groups. Head dims below 32 are zero-padded to one 32-wide d chunk so the
// 32x32 MFMA shapes apply unchanged (the pad columns are zeroed once per kernel).
template <int D>
struct TileGeom {
  static constexpr int DC = (D + 31) / 32;  // 32-wide d chunks
  static constexpr int DPAD = DC * 32;
  static constexpr int RS = DPAD + 8;       // LDS row stride (elements)
  static constexpr int CPR = D / 8;         // 16-byte chunks per row
  static constexpr int RPP = 256 / CPR;     // rows per pass of 256 threads
  static constexpr int PASSES = (kBlock + RPP - 1) / RPP;
  static constexpr int ELEMS = kBlock * RS;  // one staged tile
};

// Zeroes the pad columns [D, DPAD) of a staged tile (no-op for D >= 32).
template <int D>
__device__ __forceinline__ void zero_pad_cols(uint16_t* tile, int tid) {
  using G = TileGeom<D>;
  if constexpr (G::DPAD > D) {
    constexpr int per_row = (G::DPAD - D) / 8;
    for (int i = tid; i < kBlock * per_row; i += 256) {
      const int r = i / per_row, ch = i % per_row;
      u32x4_t z = {0u, 0u, 0u, 0u};
      lds_write_b128(tile + r * G::RS + D + ch * 8, z);
    }
  }
}

// Register staging for one 32-row tile of a [B, H, N, D] tensor: row r is sequence position
// pos0 + r * step, clamped to N - 1 (rows past the end are never visible, so their values only need
// to be finite data of the same tensor).
template <int D>
struct TileRegs {
  u32x4_t v[TileGeom<D>::PASSES];

  __device__ __forceinline__ void load(const uint16_t* base, int64_t sn, int N, int tid, int pos0, int step) {
    using G = TileGeom<D>;
#pragma unroll
    for (int p = 0; p < G::PASSES; ++p) {
      const int r = p * G::RPP + tid / G::CPR;
      const int ch = tid % G::CPR;
      if (G::PASSES * G::RPP == kBlock || r < kBlock) {
        const int kp = imin(pos0 + r * step, N - 1);
        v[p] = *reinterpret_cast<const u32x4_t*>(base + (int64_t)kp * sn + ch * 8);
      }
    }
  }

  __device__ __forceinline__ void store(uint16_t* tile, int tid) const {
    using G = TileGeom<D>;
#pragma unroll
    for (int p = 0; p < G::PASSES; ++p) {
      const int r = p * G::RPP + tid / G::CPR;
      const int ch = tid % G::CPR;
      if (G::PASSES * G::RPP == kBlock || r < kBlock) lds_write_b128(tile + r * G::RS + ch * 8, v[p]);
    }
  }
};

// Sets to -inf the elements of a 32x32 accumulator (lane half g) whose row t0 + acc_row(i, g) lies
// outside [lo, hi].
__device__ __forceinline__ void mask_outside(f32x16_t& s, int lo, int hi, int t0, int g) {
  const int a = lo - t0 - 4 * g, z = hi - t0 - 4 * g;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = 8 * (i >> 2) + (i & 3);
    s[i] = (r >= a && r <= z) ? s[i] : -INFINITY;
  }
}

// Query-stationary exact visibility bits for a lane owning query qp (document id dq) and a block
// of 32 indices of `stream` starting at t0, when the row's ids are arbitrary: interval test and
// per-pair id equality.
__device__ __forceinline__ uint32_t qs_exact_bits(const AttnArgs& a, int b, const Interval& r, int stream, int t0,
                                                  int g, int64_t dq) {
  uint32_t bits = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int t = t0 + acc_row(i, g);
    bool vis = t >= r.lo && t <= r.hi;
    if (vis) vis = load_doc(a, b, stream_pos(a.m, stream, t)) == dq;
    bits |= (uint32_t)vis << i;
  }
  return bits;
}

// Key-stationary exact visibility bits for a lane owning key kp (document id dk, last visible query
// qhi) and the query chunk starting at position qc.
__device__ __forceinline__ uint32_t ks_exact_bits(const AttnArgs& a, int b, int kp, int qhi, int qc, int g,
                                                  int64_t dk) {
  uint32_t bits = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int q = qc + acc_row(i, g);
    bool vis = q >= kp && q <= qhi;
    if (vis) vis = load_doc(a, b, q) == dk;
    bits |= (uint32_t)vis << i;
  }
  return bits;
}

// Key-block plan of a query-stationary workgroup: blocks [0, n0) are stream-0 blocks b0, b0 + 1, ...
// (natural or persistent stream), blocks [n0, n0 + n1) temporary-stream blocks b1, b1 + 1, ...
struct QPlan {
  int stream0, b0, n0, b1, n1;
  __device__ __forceinline__ int count() const { return n0 + n1; }
  __device__ __forceinline__ int stream(int i) const { return i < n0 ? stream0 : STREAM_TEMPORARY; }
  __device__ __forceinline__ int first(int i) const { return kBlock * (i < n0 ? b0 + i : b1 + i - n0); }
};

// Per-lane key intervals, per-wave spans and the workgroup plan of the query tile starting at qa.
struct QState {
  Interval r0, r1;
  WaveSpan w0, w1;
  QPlan plan;
};

__device__ __forceinline__ void q_setup(const AttnArgs& a, const RowView& row, int qp, int* s_span, QState& st) {
  const MaskSpec& m = a.m;
  const int tid = threadIdx.x, wave = tid >> 6;
  if (qp < m.N) {
    query_intervals(m, qp, row.run_start(qp), st.r0, st.r1);
  } else {
    st.r0 = Interval{kEmptyLo, kEmptyHi};
    st.r1 = st.r0;
  }
  st.w0 = wave_span(st.r0);
  st.w1 = wave_span(st.r1);
  if ((tid & 63) == 0) {
    s_span[4 * wave + 0] = st.w0.min_lo;
    s_span[4 * wave + 1] = st.w0.max_hi;
    s_span[4 * wave + 2] = st.w1.min_lo;
    s_span[4 * wave + 3] = st.w1.max_hi;
  }
  __syncthreads();
  int lo0 = kEmptyLo, hi0 = kEmptyHi, lo1 = kEmptyLo, hi1 = kEmptyHi;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    lo0 = imin(lo0, s_span[4 * w + 0]);
    hi0 = imax(hi0, s_span[4 * w + 1]);
    lo1 = imin(lo1, s_span[4 * w + 2]);
    hi1 = imax(hi1, s_span[4 * w + 3]);
  }
  QPlan& p = st.plan;
  p.stream0 = m.family == FAMILY_FULL ? STREAM_NATURAL : STREAM_PERSISTENT;
  p.b0 = wave_uniform(hi0 >= lo0 ? lo0 / kBlock : 0);
  p.n0 = wave_uniform(hi0 >= lo0 ? hi0 / kBlock - p.b0 + 1 : 0);
  p.b1 = wave_uniform(hi1 >= lo1 ? lo1 / kBlock : 0);
  p.n1 = wave_uniform(hi1 >= lo1 ? hi1 / kBlock - p.b1 + 1 : 0);
}

// Workgroup -> (row, head, query tile): ranks of the per-row heaviest-first order are outermost, so
// every (row, head) pair keeps the same XCD (dispatch is round-robin over XCDs by block index).
__device__ __forceinline__ void q_workgroup(const AttnArgs& a, int& b, int& h, int& qt) {
  const int BH = a.B * a.H;
  const int rank = blockIdx.x / BH, bh = blockIdx.x - rank * BH;
  b = bh / a.H;
  h = bh - b * a.H;
  qt = q_tile_of(a, b, rank);
}


// Query-chunk plan of a key-stationary workgroup (dK/dV): chunks c0 .. c0 + nc - 1 of 32 positions.
struct KState {
  int stream, first;  // the workgroup's key stream and first stream index
  int kp;             // this lane's key position (valid when kvalid)
  bool kvalid;
  Interval r;  // queries seeing the lane's key: [kp, last]
  WaveSpan w;
  int c0, nc;
};

__device__ __forceinline__ void k_setup(const AttnArgs& a, const RowView& row, int kt, int* s_span, KState& st) {
  const MaskSpec& m = a.m;
  const int tid = threadIdx.x, wave = tid >> 6, c32 = tid & 31;
  k_tile_run(m, kt, st.stream, st.first);
  const int t = st.first + wave * kBlock + c32;
  st.kvalid = t < stream_len(m.family, m.N, st.stream, m.P);
  st.kp = st.kvalid ? stream_pos(m, st.stream, t) : 0;
  if (st.kvalid) {
    st.r.lo = st.kp;
    st.r.hi = key_last_query(m, st.stream, st.kp, row.run_end(st.kp, m.N));
    if (st.r.hi < st.r.lo) st.r = Interval{kEmptyLo, kEmptyHi};
  } else {
    st.r = Interval{kEmptyLo, kEmptyHi};
  }
  st.w = wave_span(st.r);
  if ((tid & 63) == 0) {
    s_span[2 * wave + 0] = st.w.min_lo;
    s_span[2 * wave + 1] = st.w.max_hi;
  }
  __syncthreads();
  int lo = kEmptyLo, hi = kEmptyHi;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    lo = imin(lo, s_span[2 * w + 0]);
    hi = imax(hi, s_span[2 * w + 1]);
  }
  st.c0 = wave_uniform(hi >= lo ? lo / kBlock : 0);
  st.nc = wave_uniform(hi >= lo ? hi / kBlock - st.c0 + 1 : 0);
}

__device__ __forceinline__ void k_workgroup(const AttnArgs& a, int& b, int& h, int& kt) {
  const int BH = a.B * a.H;
  const int rank = blockIdx.x / BH, bh = blockIdx.x - rank * BH;
  b = bh / a.H;
  h = bh - b * a.H;
  kt = k_tile_of(a, b, rank);
}

// Interval bits (rows of the accumulator inside [lo, hi]) for a block starting at t0.
__device__ __forceinline__ uint32_t interval_keep_bits(int lo, int hi, int t0, int g) {
  return interval_bits(lo, hi, t0, g);
}

}  // namespace sps
