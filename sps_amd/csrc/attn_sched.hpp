// Visibility predicate, interval form, block classification and tile order for the
// document-masked causal (full) and SPS sliding-window attention families.
//
// Positions q, k index the attention sequence. For the SPS families the sequence is the
// interleaved input/<predict> sequence: token t owns positions 2t (input) and 2t+1 (predict).
// The "persistent" key parity P is exempt from the sliding window: P = 0 for sps_sliding_attention
// (reference: triton_sps_flash_attention.py:97), P = 1 for reverse_sps_sliding_attention
// (triton_reverse_sps_flash_attention.py:123). Keys of the other parity are "temporary" and are
// visible only within `window` tokens (triton_sps_flash_attention.py:89-95). The diagonal is always
// visible (:106-107); the optional persistent-key window limits persistent keys to
// q_tok - k_tok <= pkw (:102-104). The causal mask (k <= q, :109-111) and the document mask
// (docs[q] == docs[k], :81-87) apply to all families; the full family
// (triton_full_flash_attention.py:95-104) has no window.
//
// Interval form. Keys are split into streams: the natural stream (full family: every position) or,
// for the SPS families, the persistent stream (positions 2t + P) and the temporary stream
// (positions 2t + 1 - P), indexed by token t. When a row's document ids are non-decreasing, equal
// ids form one contiguous run, and the keys a query q sees in a stream are ONE interval of stream
// indices, fixed by the start s of q's run: persistent [ceil((s-P)/2), (q-P)>>1] (cut to
// [tq - pkw, ...] by a persistent-key window, or to the diagonal alone when pkw < 0), temporary
// [max(ceil((s-1+P)/2), tq - w), (q-1+P)>>1], natural [s, q]. Symmetrically the queries that see a
// key k form the interval [k, qhi(k)] with qhi bounded by the end of k's run and the window. A
// prepass (attn_prep.hip) writes each position's run start and end. Rows whose ids are not
// non-decreasing are scheduled as one run and every pair is also checked for equal ids.
//
// Blocks: the kernels consume 32 consecutive indices of one stream per MFMA block. A wave
// classifies a block from four per-wave numbers (min/max of its lanes' interval ends): SKIP (no
// lane sees any row), FULL (every lane sees every row) or PARTIAL (per-element interval test).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sps {

enum Family : int { FAMILY_FULL = 0, FAMILY_SPS = 1, FAMILY_REVERSE_SPS = 2 };
enum Stream : int { STREAM_NATURAL = 0, STREAM_PERSISTENT = 1, STREAM_TEMPORARY = 2 };
enum TileClass : int { TILE_SKIP = 0, TILE_FULL = 1, TILE_PARTIAL = 2 };

constexpr int kBlock = 32;              // stream rows per MFMA block
constexpr int kWaves = 4;               // waves per workgroup
constexpr int kTile = kBlock * kWaves;  // queries (or keys of one stream) per workgroup
constexpr int kEmptyLo = 0x3fffffff;    // interval marking "nothing visible"
constexpr int kEmptyHi = -0x3fffffff;

struct MaskSpec {
  int family;  // Family
  int P;       // persistent parity for the SPS families
  int N;       // sequence length (positions)
  int window;  // temporary-key window in tokens, clamped to [-1, N]
  int has_pkw;
  int pkw;  // persistent-key window in tokens, clamped to [-1, N]
  int has_docs;
};

struct Interval {
  int lo, hi;  // inclusive; empty when lo > hi
};

__host__ __device__ __forceinline__ int imin(int x, int y) { return x < y ? x : y; }
__host__ __device__ __forceinline__ int imax(int x, int y) { return x > y ? x : y; }

// Division by a divisor fixed at launch (the grid's batch rows, heads, row x head slots), for
// dividends below 2^31: q = (mulhi(x, mul) + x) >> shift with shift = ceil(log2 d) and
// mul = floor(2^32 (2^shift - d) / d) + 1 (Granlund & Montgomery, "Division by invariant integers
// using multiplication", 1994: the round-up method; the sum stays below 2^32 since mulhi(x, mul) <= x).
// The kernels divide wave-uniform values, so this is a few scalar instructions, where a division
// by a runtime divisor is a VALU sequence of ~20 instructions.
struct FastDiv {
  uint32_t d, mul, shift;
};

inline FastDiv make_fast_div(uint32_t d) {
  if (d == 0) return FastDiv{0, 0, 0};  // no grid to map
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  return FastDiv{d, (uint32_t)((((1ull << 32) * ((1ull << l) - d)) / d) + 1), l};
}

__host__ __device__ __forceinline__ uint32_t fast_div(uint32_t x, const FastDiv& f) {
  return ((uint32_t)(((uint64_t)x * f.mul) >> 32) + x) >> f.shift;
}

__host__ __device__ __forceinline__ int stream_parity(const MaskSpec& m, int stream) {
  return stream == STREAM_PERSISTENT ? m.P : 1 - m.P;
}

// Position of index t of a stream.
__host__ __device__ __forceinline__ int stream_pos(const MaskSpec& m, int stream, int t) {
  return stream == STREAM_NATURAL ? t : 2 * t + stream_parity(m, stream);
}

// Number of indices of a stream.
__host__ __device__ __forceinline__ int stream_len(int family, int N, int stream, int P) {
  if (family == FAMILY_FULL) return N;
  const int par = stream == STREAM_PERSISTENT ? P : 1 - P;
  return N > par ? (N - par + 1) >> 1 : 0;
}

// Keys of stream 0 (natural or persistent) and stream 1 (temporary) visible to query q whose
// document run starts at position s.
__host__ __device__ __forceinline__ void query_intervals(const MaskSpec& m, int q, int s, Interval& r0, Interval& r1) {
  if (m.family == FAMILY_FULL) {
    r0.lo = s;
    r0.hi = q;
    r1.lo = kEmptyLo;
    r1.hi = kEmptyHi;
    return;
  }
  const int P = m.P, tq = q >> 1;
  r0.lo = (s - P + 1) >> 1;
  r0.hi = (q - P) >> 1;
  if (m.has_pkw) {
    if (m.pkw >= 0) {
      r0.lo = imax(r0.lo, tq - m.pkw);
    } else if ((q & 1) == P) {
      r0.lo = tq;  // only the persistent diagonal
      r0.hi = tq;
    } else {
      r0.lo = kEmptyLo;
      r0.hi = kEmptyHi;
    }
  }
  r1.lo = imax((s + P) >> 1, tq - m.window);
  r1.hi = (q - 1 + P) >> 1;
  if (r0.lo > r0.hi) r0 = Interval{kEmptyLo, kEmptyHi};
  if (r1.lo > r1.hi) r1 = Interval{kEmptyLo, kEmptyHi};
}

// Last query position that sees key k (position) of `stream`, whose document run ends at e.
// The first such query is k itself.
__host__ __device__ __forceinline__ int key_last_query(const MaskSpec& m, int stream, int k, int e) {
  if (m.family == FAMILY_FULL) return e;
  const int tk = k >> 1;
  if (stream == STREAM_PERSISTENT) {
    if (!m.has_pkw) return e;
    return m.pkw >= 0 ? imin(e, 2 * (tk + m.pkw) + 1) : k;
  }
  return imin(e, 2 * (tk + m.window) + 1);
}

// Union, per stream, of the intervals of query tile qt's queries (kTile consecutive positions),
// from its first and last kTileEnds queries only: both interval bounds never decrease with the
// position (run starts, the diagonal and the window bounds all are non-decreasing), so the union
// runs from the first non-empty query's lo to the last non-empty query's hi, and among any two
// consecutive positions at least one has a non-empty interval of a stream unless no position of
// the tile does (tests/native/tile_plan_check.hip compares this with the union over every query).
// start(q) is q's run start.
constexpr int kTileEnds = 4;

// Row j (< 2 kTileEnds) of query tile qt's first and last kTileEnds positions, or -1 past a short
// tile's end.
__host__ __device__ __forceinline__ int q_tile_row(const MaskSpec& m, int qt, int j) {
  const int qa = qt * kTile, qz = imin(qa + kTile, m.N) - 1;
  const int q = j < kTileEnds ? qa + j : qz - (j - kTileEnds);
  return (q < qa || q > qz) ? -1 : q;
}

template <class StartFn>
__host__ __device__ __forceinline__ void q_tile_union(const MaskSpec& m, int qt, StartFn start, Interval& u0,
                                                      Interval& u1) {
  u0 = u1 = Interval{kEmptyLo, kEmptyHi};
  for (int j = 0; j < 2 * kTileEnds; ++j) {
    const int q = q_tile_row(m, qt, j);
    if (q < 0) continue;
    Interval i0, i1;
    query_intervals(m, q, start(q), i0, i1);  // an empty interval is {kEmptyLo, kEmptyHi}
    u0.lo = imin(u0.lo, i0.lo);
    u0.hi = imax(u0.hi, i0.hi);
    u1.lo = imin(u1.lo, i1.lo);
    u1.hi = imax(u1.hi, i1.hi);
  }
}

// Union of the query intervals [k, key_last_query(k)] of key tile kt's keys: every key of a stream
// has a non-empty interval or none has, and the last query never decreases with the key, so the
// tile's first and last keys give it. end(k) is the end of k's run.
template <class EndFn>
__host__ __device__ __forceinline__ Interval k_tile_union(const MaskSpec& m, int kt, EndFn end);

// Per-wave summary of the lanes' intervals: union bounds (for SKIP) and intersection bounds (FULL).
struct WaveSpan {
  int min_lo, max_hi;  // union [min_lo, max_hi] over lanes with a non-empty interval
  int max_lo, min_hi;  // every lane's interval contains [max_lo, min_hi] (lanes with nothing break it)
};

// Reduction of x over the 64 lanes (all active) with an associative, commutative op; the result is
// wave-uniform. Inside each row of 16 lanes by DPP moves (VALU, no LDS round trip): quad swaps, then
// the half-row and row mirrors leave every lane of a row holding the row's result; the four rows
// are then combined from one lane each.
template <class Op>
__device__ __forceinline__ int wave_reduce(int x, Op op) {
  x = op(x, __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));   // quad_perm [1, 0, 3, 2]
  x = op(x, __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));   // quad_perm [2, 3, 0, 1]
  x = op(x, __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, false));  // row_half_mirror
  x = op(x, __builtin_amdgcn_mov_dpp(x, 0x140, 0xF, 0xF, false));  // row_mirror
  const int r0 = __builtin_amdgcn_readlane(x, 0), r1 = __builtin_amdgcn_readlane(x, 16);
  const int r2 = __builtin_amdgcn_readlane(x, 32), r3 = __builtin_amdgcn_readlane(x, 48);
  return op(op(r0, r1), op(r2, r3));
}

__device__ __forceinline__ WaveSpan wave_span(const Interval& r) {
  const bool empty = r.lo > r.hi;
  WaveSpan w;  // the reductions are wave-uniform: keep them in scalar registers
  w.min_lo = __builtin_amdgcn_readfirstlane(wave_reduce(empty ? kEmptyLo : r.lo, [](int x, int y) { return imin(x, y); }));
  w.max_hi = __builtin_amdgcn_readfirstlane(wave_reduce(empty ? kEmptyHi : r.hi, [](int x, int y) { return imax(x, y); }));
  w.max_lo = __builtin_amdgcn_readfirstlane(wave_reduce(empty ? kEmptyLo : r.lo, [](int x, int y) { return imax(x, y); }));
  w.min_hi = __builtin_amdgcn_readfirstlane(wave_reduce(empty ? kEmptyHi : r.hi, [](int x, int y) { return imin(x, y); }));
  return w;
}

// The same spans for intervals that never decrease along the lanes 0-31 (lanes 32-63 repeat them):
// the union runs from the first non-empty lane's lo to the last non-empty lane's hi, and the common
// part, when no lane is empty, from lane 31's lo to lane 0's hi; four lane reads instead of four
// reductions. The kernels' lanes hold consecutive queries (keys) of one stream, and both bounds of
// their intervals are non-decreasing in the position (run starts and ends, the diagonal and the
// window bounds all are).
__device__ __forceinline__ WaveSpan wave_span_monotone(const Interval& r) {
  const uint64_t ne = __builtin_amdgcn_ballot_w64(r.lo <= r.hi) & 0xffffffffull;
  if (ne == 0) return WaveSpan{kEmptyLo, kEmptyHi, kEmptyLo, kEmptyHi};
  const int first = __builtin_ctzll(ne), last = 63 - __builtin_clzll(ne);
  const bool all = ne == 0xffffffffull;
  WaveSpan w;
  w.min_lo = __builtin_amdgcn_readlane(r.lo, first);
  w.max_hi = __builtin_amdgcn_readlane(r.hi, last);
  w.max_lo = all ? __builtin_amdgcn_readlane(r.lo, 31) : kEmptyLo;
  w.min_hi = all ? __builtin_amdgcn_readlane(r.hi, 0) : kEmptyHi;
  return w;
}

// Class of the block of 32 indices [t0, t0 + 31] for a wave. `exact_docs` is false when the row's
// ids are not a sequence of runs (then every visible-by-interval pair still needs an id check).
__host__ __device__ __forceinline__ int classify_block(const WaveSpan& w, int t0, bool exact_docs) {
  if (t0 > w.max_hi || t0 + kBlock - 1 < w.min_lo) return TILE_SKIP;
  if (exact_docs && t0 >= w.max_lo && t0 + kBlock - 1 <= w.min_hi) return TILE_FULL;
  return TILE_PARTIAL;
}

// Row of a 32x32 MFMA accumulator held in element i by a lane of half g (= lane / 32).
__device__ __forceinline__ int acc_row(int i, int g) { return 8 * (i >> 2) + 4 * g + (i & 3); }

// ---------------------------------------------------------------------------------------------
// Workgroup tiles and their order. Query-stationary kernels (forward, dQ) own kTile consecutive
// positions; the key-stationary kernel (dK/dV) owns kTile consecutive indices of one stream
// (SPS families: persistent-stream tiles, then temporary-stream tiles). Within a row, tiles are
// launched heaviest first: from the prepass's sorted order when documents are given, else by the
// closed form (later query tiles see more keys; earlier key tiles are seen by more queries).
// ---------------------------------------------------------------------------------------------
__host__ __device__ __forceinline__ int q_tiles(int N) { return (N + kTile - 1) / kTile; }

__host__ __device__ __forceinline__ int k_tiles_stream(int family, int N, int stream, int P) {
  return (stream_len(family, N, stream, P) + kTile - 1) / kTile;
}

__host__ __device__ __forceinline__ int k_tiles(int family, int N, int P) {
  if (family == FAMILY_FULL) return k_tiles_stream(family, N, STREAM_NATURAL, P);
  return k_tiles_stream(family, N, STREAM_PERSISTENT, P) + k_tiles_stream(family, N, STREAM_TEMPORARY, P);
}

// Stream and first stream index of key tile kt.
__host__ __device__ __forceinline__ void k_tile_run(const MaskSpec& m, int kt, int& stream, int& first) {
  if (m.family == FAMILY_FULL) {
    stream = STREAM_NATURAL;
    first = kt * kTile;
    return;
  }
  const int np = k_tiles_stream(m.family, m.N, STREAM_PERSISTENT, m.P);
  stream = kt < np ? STREAM_PERSISTENT : STREAM_TEMPORARY;
  first = (kt < np ? kt : kt - np) * kTile;
}

// Position of row j (< 2 kTileEnds) of key tile kt's first and last kTileEnds keys, or -1 past a
// short tile's end; `stream` is the tile's key stream.
__host__ __device__ __forceinline__ int k_tile_row(const MaskSpec& m, int kt, int j, int& stream) {
  int first;
  k_tile_run(m, kt, stream, first);
  const int len = stream_len(m.family, m.N, stream, m.P);
  const int ta = first, tz = imin(first + kTile, len) - 1;
  const int t = j < kTileEnds ? ta + j : tz - (j - kTileEnds);
  return (t < ta || t > tz) ? -1 : stream_pos(m, stream, t);
}

// (Definition of k_tile_union, declared above.)
template <class EndFn>
__host__ __device__ __forceinline__ Interval k_tile_union(const MaskSpec& m, int kt, EndFn end) {
  Interval u{kEmptyLo, kEmptyHi};
  for (int j = 0; j < 2 * kTileEnds; ++j) {
    int stream;
    const int kp = k_tile_row(m, kt, j, stream);
    if (kp < 0) continue;
    const int last = key_last_query(m, stream, kp, end(kp));
    if (last >= kp) {
      u.lo = imin(u.lo, kp);
      u.hi = imax(u.hi, last);
    }
  }
  return u;
}

}  // namespace sps
