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

// Register staging for one 32-row tile of a [B, H, N, D] tensor read through a buffer descriptor
// over one (batch, head) slice: row r of the tile is sequence position pos0 + r * step. Rows past
// the end of the sequence read as zeros (they are never visible).
template <int D>
struct TileRegs {
  using G = TileGeom<D>;
  u32x4_t v[G::PASSES];

  // Byte offsets, from the tile's first row, of the 16-byte pieces this thread moves.
  struct Offsets {
    uint32_t o[G::PASSES];
  };

  static __device__ __forceinline__ Offsets offsets(int tid, uint32_t row_step_bytes) {
    Offsets f;
#pragma unroll
    for (int p = 0; p < G::PASSES; ++p) {
      const int r = p * G::RPP + tid / G::CPR;
      f.o[p] = (uint32_t)r * row_step_bytes + (uint32_t)(tid % G::CPR) * 16u;
    }
    return f;
  }

  __device__ __forceinline__ void load(BufRsrc rs, uint32_t first_row_bytes, const Offsets& f, int tid) {
#pragma unroll
    for (int p = 0; p < G::PASSES; ++p) {
      const int r = p * G::RPP + tid / G::CPR;
      if (G::PASSES * G::RPP == kBlock || r < kBlock) v[p] = buf_load_b128(rs, first_row_bytes + f.o[p]);
    }
  }

  // A block past the end of the plan: zeros, so its LDS tile (computed on, then masked) holds finite
  // values and contributes exactly 0 to the products.
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int p = 0; p < G::PASSES; ++p) v[p] = u32x4_t{0u, 0u, 0u, 0u};
  }

  __device__ __forceinline__ void store(uint16_t* tile, int tid) const {
#pragma unroll
    for (int p = 0; p < G::PASSES; ++p) {
      const int r = p * G::RPP + tid / G::CPR;
      const int ch = tid % G::CPR;
      if (G::PASSES * G::RPP == kBlock || r < kBlock) lds_write_b128(tile + r * G::RS + ch * 8, v[p]);
    }
  }
};

// Dense LDS tile filled by direct global -> LDS loads (head dims of 64 and more): 32 rows of D
// elements, no padding; the 16-byte chunks of each row are permuted by a row-dependent swizzle
// instead (swz below).
template <int D, bool kSpread = true>
struct DmaTile {
  static_assert(D == 64 || D % 128 == 0, "the swizzle permutes 8 chunks of a row at D = 64, 16 above");
  static constexpr int CPR = D / 8;                  // 16-byte chunks per row
  static constexpr int ELEMS = kBlock * D;           // one staged tile
  static constexpr int PASSES = ELEMS / (256 * 8);   // 16-byte pieces per thread (1 for D = 64)

  // Logical chunk k of row r is stored at chunk k ^ swz(r), so that both fragment reads below hit
  // distinct LDS banks (64 banks of 4 bytes): a row-fragment b128 read gives 16 lanes 16 consecutive
  // rows at one logical chunk, a transposed b64 read gives 32 lanes rows r0 .. r0 + 3 at four
  // consecutive chunks. D = 64 (a row covers half the banks): the rows of one parity among 16
  // consecutive rows get 8 different swizzles (bits 1-3 of r), and rows r, r + 2 different 4-chunk
  // groups (swizzle bit 2 = bit 1 of r). D >= 128 (a row covers every bank): 16 consecutive rows get
  // 16 different swizzles, and rows r0 .. r0 + 3 different 4-chunk groups (swizzle bits 2-3 = r & 3).
  // kSpread false keeps an older 3-bit swizzle under which rows r and r + 8 share a swizzle (so a
  // transposed fragment needs one address per lane instead of two; row-fragment reads then meet
  // 2-way bank conflicts), for kernels whose registers are the tighter limit.
  static __device__ __forceinline__ int swz(int r) {
    if constexpr (!kSpread)
      return ((r & 3) << 1) | ((r >> 2) & 1);
    else if constexpr (D == 64)
      return (((r >> 1) & 1) << 2) | (((r >> 2) & 1) << 1) | ((r >> 3) & 1);
    else
      return ((r & 3) << 2) | ((r >> 2) & 3);
  }

  // Byte offsets, from the tile's first row, of the pieces thread tid loads: piece p fills slot
  // p * 256 + tid of the tile (row slot / CPR, stored chunk slot % CPR).
  struct Src {
    uint32_t o[PASSES];
  };
  static __device__ __forceinline__ Src sources(int tid, uint32_t row_step_bytes) {
    Src s;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int slot = p * 256 + tid, r = slot / CPR, c = (slot % CPR) ^ swz(r);
      s.o[p] = (uint32_t)r * row_step_bytes + (uint32_t)c * 16u;
    }
    return s;
  }

  // Issues the loads of a tile whose first row is at byte `first` of the buffer (one instruction
  // per piece and wave, each filling the wave's contiguous 1 KiB of the tile).
  static __device__ __forceinline__ void load(BufRsrc rs, uint32_t first, const Src& s, uint16_t* tile, int wave) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) lds_dma_b128(rs, tile + (p * 256 + wave * 64) * 8, first + s.o[p]);
  }

  // Element offset of row c32's chunk 2c + g (row-major fragment: 8 consecutive columns 16c + 8g).
  // Both forms here and in frag_tr give the same offsets for the register-lean swizzle; each kernel
  // keeps the form it was tuned with, since the compiler allocates registers differently for them.
  static __device__ __forceinline__ int frag(int c32, int g, int c) {
    if constexpr (kSpread)
      return c32 * D + ((2 * c + g) ^ swz(c32)) * 8;
    else
      return c32 * D + ((2 * c) ^ (g ^ swz(c32))) * 8;
  }

  // The transposed fragment of lds_frag_tr(tile, row_stride, r0, 32 dc, lane) on this layout
  // (r0 a multiple of 8; rows r and r + 8 share a swizzle only when !kSpread).
  static __device__ __forceinline__ u32x4_t frag_tr(const uint16_t* tile, int r0, int dc, int lane) {
    const int s = lane & 15, grp = lane >> 4;
    const int row = r0 + 4 * (grp >> 1) + (s >> 2);
    const int t = 2 * (grp & 1) + ((s & 3) >> 1);  // logical chunk 4 dc + t
    const uint16_t *p, *q;
    if constexpr (kSpread) {
      p = tile + row * D + ((4 * dc + t) ^ swz(row)) * 8 + 4 * (s & 1);
      q = tile + (row + 8) * D + ((4 * dc + t) ^ swz(row + 8)) * 8 + 4 * (s & 1);
    } else {
      p = tile + row * D + ((4 * dc) ^ (t ^ swz(row))) * 8 + 4 * (s & 1);
      q = p + 8 * D;
    }
    const u32x2_t lo = lds_read_tr16(p), hi = lds_read_tr16(q);
    return u32x4_t{lo[0], lo[1], hi[0], hi[1]};
  }
};

// Descriptor over the rows [0, N) of one (batch, head) slice of a [B, H, N, D] tensor.
template <int D>
__device__ __forceinline__ BufRsrc head_rsrc(const uint16_t* head_base, int64_t sn, int N) {
  return make_rsrc(head_base, (uint32_t)(((int64_t)N - 1) * sn * 2 + D * 2));
}

// Sets to -inf the elements of a 32x32 accumulator (lane half g) whose row t0 + acc_row(i, g) lies
// outside the lane's interval [lo, hi]. cut_lo / cut_hi (wave-uniform) tell whether the lower / upper
// bound of some lane falls inside this block; usually only one does, so only one test runs.
__device__ __forceinline__ void mask_cuts(f32x16_t& s, int lo, int hi, int t0, int g, bool cut_lo, bool cut_hi) {
  if (cut_lo) {
    const int a = lo - t0 - 4 * g;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = (8 * (i >> 2) + (i & 3) >= a) ? s[i] : -INFINITY;
  }
  if (cut_hi) {
    const int z = hi - t0 - 4 * g;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = (8 * (i >> 2) + (i & 3) <= z) ? s[i] : -INFINITY;
  }
}

// Masks a partial block: interval cuts, plus the per-pair id check of rows whose ids are arbitrary
// (bits from qs_exact_bits / ks_exact_bits).
template <bool EXACT, class BitsFn>
__device__ __forceinline__ void mask_partial(f32x16_t& s, const Interval& r, const WaveSpan& w, int t0, int g,
                                             BitsFn exact_bits) {
  if constexpr (EXACT) {
    mask_cuts(s, r.lo, r.hi, t0, g, t0 < w.max_lo, t0 + kBlock - 1 > w.min_hi);
  } else {
    const uint32_t bits = exact_bits();
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = ((bits >> e) & 1u) ? s[e] : -INFINITY;
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

// Lane intervals and wave spans of query qp, whose document run starts at position s.
__device__ __forceinline__ void q_lanes(const MaskSpec& m, int qp, int s, QState& st) {
  if (qp < m.N) {
    query_intervals(m, qp, s, st.r0, st.r1);
  } else {
    st.r0 = Interval{kEmptyLo, kEmptyHi};
    st.r1 = st.r0;
  }
  st.w0 = wave_span_monotone(st.r0);
  st.w1 = wave_span_monotone(st.r1);
}

// The workgroup's key-block plan: per stream, the 32-row blocks covering the union of its lanes'
// intervals (one LDS exchange and barrier). The prepass computes the same union for every tile.
__device__ __forceinline__ void q_plan_from_spans(const MaskSpec& m, int* s_span, QState& st) {
  const int tid = threadIdx.x, wave = tid >> 6;
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
  cover_blocks(lo0, hi0, p.b0, p.n0);
  cover_blocks(lo1, hi1, p.b1, p.n1);
  p.b0 = wave_uniform(p.b0);
  p.n0 = wave_uniform(p.n0);
  p.b1 = wave_uniform(p.b1);
  p.n1 = wave_uniform(p.n1);
}

__device__ __forceinline__ void q_setup(const AttnArgs& a, const RowView& row, int qp, int* s_span, QState& st) {
  q_lanes(a.m, qp, qp < a.m.N ? row.run_start(qp) : 0, st);
  q_plan_from_spans(a.m, s_span, st);
}

// Start of a query-stationary workgroup. With a prepass plan (documents given) the block ranges come
// from it and the lane's run start is read here; the caller issues its first tile loads and then
// calls q_lanes(m, qp, run_start, st), so both loads are in flight together. Without a plan (no
// documents: every run starts at 0, nothing to read) the whole setup runs here.
__device__ __forceinline__ bool q_begin(const AttnArgs& a, const TilePlan& tp, const RowView& row, int qp,
                                        int* s_span, QState& st, int& run_start) {
  run_start = 0;
  if (tp.n0 < 0) {
    q_setup(a, row, qp, s_span, st);
    return false;
  }
  st.plan = QPlan{a.m.family == FAMILY_FULL ? STREAM_NATURAL : STREAM_PERSISTENT, tp.b0, tp.n0, tp.b1, tp.n1};
  if (qp < a.m.N) run_start = row.run_start(qp);
  return true;
}

// Workgroup -> (row, head, tile): ranks of the per-row heaviest-first order are outermost, and
// within a rank the (row, head) slots rotate by one batch row (H slots) per rank. The hardware deals
// consecutive workgroups round-robin to its XCDs and, inside an XCD, to its shader engines, and
// dispatches in order: without the rotation each engine would always receive the same batch rows;
// rows packed with different documents carry different work, and the engines holding the lighter
// rows would drain and idle while the others still hold work only they may start (measured: ~8% of
// the attention time at the benchmark shape). When H is a multiple of the XCD count the rotation
// keeps every (row, head) on one XCD, so its K/V tiles stay in that XCD's L2.
// Slot j (< B H) of rank `rank` -> (row, head) index (j + rank H) mod B H, as j + (rank mod B) H
// less B H when that reaches B H (rank H mod B H = (rank mod B) H).
__device__ __forceinline__ void workgroup_slot(const AttnArgs& a, int& b, int& h, int& rank) {
  const int BH = a.B * a.H;
  rank = (int)fast_div(blockIdx.x, a.div_bh);
  const int j = (int)blockIdx.x - rank * BH;
  int bh = j + (rank - (int)fast_div((uint32_t)rank, a.div_b) * a.B) * a.H;
  if (bh >= BH) bh -= BH;
  b = (int)fast_div((uint32_t)bh, a.div_h);
  h = bh - b * a.H;
}

__device__ __forceinline__ TilePlan uniform_plan(const TilePlan& p) {
  return TilePlan{wave_uniform(p.tile), wave_uniform(p.mono), wave_uniform(p.b0), wave_uniform(p.n0),
                  wave_uniform(p.b1),   wave_uniform(p.n1),   0,                  0};
}

__device__ __forceinline__ void q_workgroup(const AttnArgs& a, int& b, int& h, TilePlan& tp) {
  int rank;
  workgroup_slot(a, b, h, rank);
  tp = uniform_plan(q_plan_of(a, b, rank));
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

// The lane's key of key tile kt (lanes 32-63 repeat lanes 0-31).
__device__ __forceinline__ void k_lane_key(const MaskSpec& m, int kt, KState& st) {
  const int tid = threadIdx.x, wave = tid >> 6, c32 = tid & 31;
  k_tile_run(m, kt, st.stream, st.first);
  const int t = st.first + wave * kBlock + c32;
  st.kvalid = t < stream_len(m.family, m.N, st.stream, m.P);
  st.kp = st.kvalid ? stream_pos(m, st.stream, t) : 0;
}

// The lane's query interval and the wave span, given the end e of the key's document run.
// kMonotone: the span from four lane reads (wave_span_monotone), else from four reductions.
template <bool kMonotone = true>
__device__ __forceinline__ void k_lanes(const MaskSpec& m, int e, KState& st) {
  if (st.kvalid) {
    st.r.lo = st.kp;
    st.r.hi = key_last_query(m, st.stream, st.kp, e);
    if (st.r.hi < st.r.lo) st.r = Interval{kEmptyLo, kEmptyHi};
  } else {
    st.r = Interval{kEmptyLo, kEmptyHi};
  }
  st.w = kMonotone ? wave_span_monotone(st.r) : wave_span(st.r);
}

// Query chunks covering the union of the workgroup's lane intervals (one LDS exchange and barrier).
__device__ __forceinline__ void k_plan_from_spans(int* s_span, KState& st) {
  const int tid = threadIdx.x, wave = tid >> 6;
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
  cover_blocks(lo, hi, st.c0, st.nc);
  st.c0 = wave_uniform(st.c0);
  st.nc = wave_uniform(st.nc);
}

template <bool kMonotone = true>
__device__ __forceinline__ void k_setup(const AttnArgs& a, const RowView& row, int kt, int* s_span, KState& st) {
  k_lane_key(a.m, kt, st);
  k_lanes<kMonotone>(a.m, st.kvalid ? row.run_end(st.kp, a.m.N) : 0, st);
  k_plan_from_spans(s_span, st);
}

// Start of a key-stationary workgroup; as q_begin, with the lane's run end read here and consumed by
// k_lanes(m, run_end, st) after the caller's first loads are issued.
template <bool kMonotone = true>
__device__ __forceinline__ bool k_begin(const AttnArgs& a, const TilePlan& tp, const RowView& row, int* s_span,
                                        KState& st, int& run_end) {
  run_end = 0;
  if (tp.n0 < 0) {
    k_setup<kMonotone>(a, row, tp.tile, s_span, st);
    return false;
  }
  k_lane_key(a.m, tp.tile, st);
  st.c0 = tp.b0;
  st.nc = tp.n0;
  if (st.kvalid) run_end = row.run_end(st.kp, a.m.N);
  return true;
}

__device__ __forceinline__ void k_workgroup(const AttnArgs& a, int& b, int& h, TilePlan& tp) {
  int rank;
  workgroup_slot(a, b, h, rank);
  tp = uniform_plan(k_plan_of(a, b, rank));
}


// Per-wave classes of the first 128 blocks of a loop as bitmasks (bit i: block i is not SKIP / is
// FULL for this wave), so the loops test two bits per pair of blocks instead of re-deriving streams,
// spans and classes. Blocks from 128 on are classified on the fly.
struct BlockMask {
  uint64_t act0, act1, full0, full1;  // blocks 0..63 and 64..127 (separate words: no dynamic indexing)
};

// Bits [lo, hi] (inclusive; none when lo > hi) of the 64-bit word that holds bits [base, base + 63].
__host__ __device__ __forceinline__ uint64_t bit_range64(int lo, int hi, int base) {
  const int l = imax(lo - base, 0), h = imin(hi - base, 63);
  return l > h ? 0ull : ((~0ull >> (63 - imax(h, 0))) & (~0ull << imin(l, 63)));
}

__host__ __device__ __forceinline__ void set_range(uint64_t& w0, uint64_t& w1, int lo, int hi) {
  w0 |= bit_range64(lo, hi, 0);
  w1 |= bit_range64(lo, hi, 64);
}

// Adds the classes of loop blocks [i0, i0 + n), which hold the 32-row blocks bfirst, bfirst + 1, ...
// of one stream, for a wave with span w: exactly classify_block's classes in closed form. A block
// b (rows [32 b, 32 b + 31]) is not SKIP iff 32 b <= max_hi and 32 b + 31 >= min_lo, i.e. b in
// [min_lo / 32, max_hi / 32] (bounds of non-empty intervals are >= 0), and FULL iff 32 b >= max_lo
// and 32 b + 31 <= min_hi, i.e. b in [ceil(max_lo / 32), floor((min_hi + 1) / 32) - 1]; both are
// contiguous ranges, so the masks are two bit ranges instead of a loop over the blocks.
__host__ __device__ __forceinline__ void add_block_classes(BlockMask& bm, const WaveSpan& w, bool exact, int i0, int n,
                                                  int bfirst) {
  if (n <= 0) return;
  const int last = i0 + n - 1;
  if (w.min_lo <= w.max_hi) {
    const int lo = imax((w.min_lo >> 5) - bfirst + i0, i0), hi = imin((w.max_hi >> 5) - bfirst + i0, last);
    set_range(bm.act0, bm.act1, lo, hi);
  }
  if (exact && w.max_lo <= w.min_hi) {
    const int lo = imax(((w.max_lo + 31) >> 5) - bfirst + i0, i0);
    const int hi = imin(((w.min_hi + 1) >> 5) - 1 - bfirst + i0, last);
    set_range(bm.full0, bm.full1, lo, hi);
  }
}

// Masks of a query-stationary plan (stream-0 blocks, then temporary-stream blocks).
__device__ __forceinline__ BlockMask q_block_mask(const QState& st, bool exact) {
  BlockMask bm = {0ull, 0ull, 0ull, 0ull};
  add_block_classes(bm, st.w0, exact, 0, st.plan.n0, st.plan.b0);
  add_block_classes(bm, st.w1, exact, st.plan.n0, st.plan.n1, st.plan.b1);
  return bm;
}

// Masks of a key-stationary plan (query chunks c0, c0 + 1, ...).
__device__ __forceinline__ BlockMask k_block_mask(const KState& st, bool exact) {
  BlockMask bm = {0ull, 0ull, 0ull, 0ull};
  add_block_classes(bm, st.w, exact, 0, st.nc, st.c0);
  return bm;
}

// Class of block i (< 128) from the masks.
__host__ __device__ __forceinline__ int mask_class(const BlockMask& bm, int i) {
  const uint64_t a = i < 64 ? bm.act0 : bm.act1, f = i < 64 ? bm.full0 : bm.full1;
  const int sh = i & 63;
  return ((a >> sh) & 1ull) ? (((f >> sh) & 1ull) ? TILE_FULL : TILE_PARTIAL) : TILE_SKIP;
}

// G-bit activity and fullness codes of blocks i .. i + G - 1 (i a multiple of G, G a power of two
// <= 8; blocks >= nb are SKIP).
template <int G, class ClassFn>
__device__ __forceinline__ void group_codes(const BlockMask& bm, int i, int nb, ClassFn cls_of, int& act, int& full) {
  constexpr uint64_t kMask = (1ull << G) - 1;
  if (i < 128) {
    const int sh = i & 63;
    act = (int)(((i < 64 ? bm.act0 : bm.act1) >> sh) & kMask);
    full = (int)(((i < 64 ? bm.full0 : bm.full1) >> sh) & kMask);
  } else {
    act = full = 0;
#pragma unroll
    for (int y = 0; y < G; ++y) {
      const int c = i + y < nb ? cls_of(i + y) : TILE_SKIP;
      act |= (c != TILE_SKIP) << y;
      full |= (c == TILE_FULL) << y;
    }
  }
}

// Two-bit codes of blocks i, i + 1 (i even).
template <class ClassFn>
__device__ __forceinline__ void pair_codes(const BlockMask& bm, int i, int nb, ClassFn cls_of, int& act2, int& full2) {
  group_codes<2>(bm, i, nb, cls_of, act2, full2);
}

// Software pipeline over `nb` blocks taken in groups of G (32·G stream rows per iteration, one
// barrier per group). issue(j, slot) starts the global loads of group j into register slot `slot`
// (of L), put(slot, buf) writes a slot to LDS buffer `buf` (0/1), body(j, buf) computes group j
// from LDS buffer `buf`. Group j + 1 + L is loaded while group j is computed and reaches LDS L
// iterations later, so each group's loads have L full iterations to land. Unrolled by two, so
// slots and buffers are compile-time indices. run_pairs is the G = 2 form. kFirstIssued: the
// caller has already issued group 0 into slot 0 (when nb > 0), ahead of its own setup work.
template <int L, int G = 2, bool kFirstIssued = false, class Issue, class Put, class Body>
__device__ __forceinline__ void run_groups(int nb, Issue&& issue, Put&& put, Body&& body) {
  static_assert(L == 1 || L == 2, "lookahead of one or two groups");
  const int np = (nb + G - 1) / G;
  if (np > 0) {
    if (!kFirstIssued) issue(0, 0);
    put(0, 0);
  }
  vmem_wait_all();  // everything loaded before the loop is in registers
#pragma unroll
  for (int k = 1; k <= L; ++k)
    if (k < np) issue(k, k % L);
  __syncthreads();
  for (int j0 = 0; j0 < np; j0 += 2) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j = j0 + u;
      if (j < np) {
        if (j + 1 < np) put((u + 1) % L, u ^ 1);
        if (j + 1 + L < np) issue(j + 1 + L, (u + 1) % L);
        body(j, u);
        __syncthreads();
      }
    }
  }
}

// Pipeline over groups staged by direct global -> LDS loads: issue(j, buf) loads group j into LDS
// buffer `buf`. Group j + 1 goes into buffer (j + 1) % 2 while group j is computed from buffer j % 2
// (that buffer's previous group was finished at the barrier ending iteration j - 1); each wave then
// waits for its own loads and the barrier publishes the group. kFirstIssued: the caller has already
// issued group 0 into buffer 0 (when nb > 0).
template <int G, bool kFirstIssued = false, class Issue, class Body>
__device__ __forceinline__ void run_groups_dma(int nb, Issue&& issue, Body&& body) {
  const int np = (nb + G - 1) / G;
  if (!kFirstIssued && np > 0) issue(0, 0);
  vmem_wait_all();
  __syncthreads();
  for (int j0 = 0; j0 < np; j0 += 2) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j = j0 + u;
      if (j < np) {
        if (j + 1 < np) issue(j + 1, u ^ 1);
        body(j, u);
        vmem_wait_all();
        __syncthreads();
      }
    }
  }
}

template <int L, bool kFirstIssued = false, class Issue, class Put, class Body>
__device__ __forceinline__ void run_pairs(int nb, Issue&& issue, Put&& put, Body&& body) {
  run_groups<L, 2, kFirstIssued>(nb, issue, put, body);
}

// Stores a wave's 32 output rows of D >= 64 elements held in the MFMA accumulator layout (lane:
// row c32, elements d = 32 dc + 8 ii + 4 g .. +3 as 8-byte pieces from piece(dc, ii)) through the
// wave's own idle LDS tile (at least 32 * D elements), so that each global store writes 16 bytes and
// CPR lanes cover a whole row (half the store instructions of the direct 8-byte stores, each
// covering whole rows instead of a 16-byte piece of 32 rows). Row r of the wave starts at
// row0 + r * row_stride (elements; wave-uniform) and exists for r < nrows; the wave reads back only
// what it wrote (LDS operations of one wave complete in order), so no barrier is needed.
template <int D, class PieceFn>
__device__ __forceinline__ void store_rows_via_lds(uint16_t* tile, int lane, uint16_t* row0, int64_t row_stride,
                                                   int nrows, PieceFn piece) {
  static_assert(D >= 64 && D % 64 == 0, "the chunk swizzle needs at least 8 chunks per row");
  constexpr int CPR = D / 8;     // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;  // rows per store instruction
  const int c32 = lane & 31, g = lane >> 5;
  // Chunk ch of row r sits at chunk ch ^ (r & 7): the 32 lanes writing one chunk column spread over
  // the banks.
#pragma unroll
  for (int dc = 0; dc < D / 32; ++dc) {
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int off = c32 * D + ((4 * dc + ii) ^ (c32 & 7)) * 8 + 4 * g;
      *reinterpret_cast<SPS_LDS u32x2_t*>((SPS_LDS uint16_t*)(tile + off)) = piece(dc, ii);
    }
  }
#pragma unroll
  for (int k = 0; k < kBlock / RPI; ++k) {
    const int r = k * RPI + lane / CPR, ch = lane % CPR;
    const u32x4_t x = lds_read_b128(tile + r * D + (ch ^ (r & 7)) * 8);
    if (r < nrows) *reinterpret_cast<u32x4_t*>(row0 + r * row_stride + ch * 8) = x;
  }
}

// Whether rows of a [B, H, N, D] 16-bit tensor with strides st (elements) starting at p are all
// 16-byte aligned.
__device__ __forceinline__ bool rows16_ok(const void* p, const Strides3& st) {
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0 && ((st.b | st.h | st.n) & 7) == 0;
}

// gfx950's 3-input IEEE maximum (v_maximum3_f32: NaN-propagating, so unlike fmaxf it needs no
// quieting of the MFMA results first).
__device__ __forceinline__ float max3f(float a, float b, float c) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

}  // namespace sps
