// Visibility predicate, block-sparse tile schedule and tile classification for the
// document-masked causal (full) and SPS sliding-window attention families.
//
// Positions q, k index the attention sequence. For the SPS families the sequence is the
// interleaved input/<predict> sequence: token t owns positions 2t (input) and 2t+1 (predict).
// The "persistent" key parity P is exempt from the sliding window: P = 0 for sps_sliding_attention
// (reference: triton_sps_flash_attention.py:97), P = 1 for reverse_sps_sliding_attention
// (triton_reverse_sps_flash_attention.py:123). Keys of the other parity are "temporary" and are
// visible only within `window` tokens (triton_sps_flash_attention.py:89-95). The diagonal is always
// visible (triton_sps_flash_attention.py:106-107); the optional persistent-key window limits
// persistent keys to q_tok - k_tok <= pkw (triton_sps_flash_attention.py:102-104). The causal
// mask (k <= q, :109-111) and the document mask (docs[q] == docs[k], :81-87) apply to all
// families; the full family (triton_full_flash_attention.py:95-104) has no window.
//
// Keys are consumed in blocks of 32. For the SPS families a block is 32 consecutive keys of ONE
// parity stream (stride-2 rows), so window sparsity is exploited at tile granularity: a query
// block reads persistent-key blocks from its document start to its diagonal and only the
// ceil((w + 16)/32) + 1 temporary-key blocks that intersect its window.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sps {

enum Family : int { FAMILY_FULL = 0, FAMILY_SPS = 1, FAMILY_REVERSE_SPS = 2 };
enum Stream : int { STREAM_NATURAL = 0, STREAM_PERSISTENT = 1, STREAM_TEMPORARY = 2 };
enum TileClass : int { TILE_SKIP = 0, TILE_FULL = 1, TILE_PARTIAL = 2 };

constexpr int kGranule = 32;   // positions per document-range granule
constexpr int kBlock = 32;     // keys (or queries) per MFMA block
constexpr int kWaves = 4;      // waves per workgroup
constexpr int kTile = kBlock * kWaves;  // positions (or stream keys) per workgroup tile

struct MaskSpec {
  int family;   // Family
  int P;        // persistent parity for the SPS families
  int N;        // sequence length (positions)
  int window;   // temporary-key window in tokens
  int has_pkw;  // persistent-key window enabled
  int pkw;      // persistent-key window in tokens
  int has_docs;
};

// A run of `count` keys of one stream. For STREAM_NATURAL `first` is a position; for the SPS
// streams it is a token index and key r sits at position 2*(first + r) + parity.
struct KeyRun {
  int stream;
  int first;
  int count;
};

struct DocRange {
  int64_t lo, hi;
};

__device__ __forceinline__ int stream_parity(const MaskSpec& m, int stream) {
  return stream == STREAM_PERSISTENT ? m.P : 1 - m.P;
}

__device__ __forceinline__ int key_pos(const MaskSpec& m, const KeyRun& kr, int r) {
  if (kr.stream == STREAM_NATURAL) return kr.first + r;
  return 2 * (kr.first + r) + stream_parity(m, kr.stream);
}

// Exact visibility of key position k for query position q (the bit-exact mask contract).
__device__ __forceinline__ bool visible(const MaskSpec& m, int q, int k, int64_t dq, int64_t dk) {
  if (q >= m.N || k > q) return false;
  if (m.has_docs && dq != dk) return false;
  if (m.family == FAMILY_FULL) return true;
  const int tq = q >> 1, tk = k >> 1;
  if ((k & 1) == m.P) {
    if (!m.has_pkw) return true;
    return (tq - tk <= m.pkw) || (q == k);
  }
  return tq - tk <= m.window;
}

// Row of a 32x32 MFMA accumulator held in element i by a lane of half g (= lane/32).
__device__ __forceinline__ int acc_row(int i, int g) { return 8 * (i >> 2) + 4 * g + (i & 3); }

// Merged document range of the positions [lo, hi] (hi inclusive) from per-granule min/max.
__device__ __forceinline__ DocRange doc_range(const int64_t* gmin, const int64_t* gmax, int lo,
                                              int hi) {
  DocRange r = {INT64_MAX, INT64_MIN};
  for (int gi = lo / kGranule; gi <= hi / kGranule; ++gi) {
    r.lo = gmin[gi] < r.lo ? gmin[gi] : r.lo;
    r.hi = gmax[gi] > r.hi ? gmax[gi] : r.hi;
  }
  return r;
}

// Positions covered by a key run (for the document-range lookup), clamped to [0, N).
__device__ __forceinline__ void run_span(const MaskSpec& m, const KeyRun& kr, int& lo, int& hi) {
  if (kr.stream == STREAM_NATURAL) {
    lo = kr.first;
    hi = kr.first + kr.count - 1;
  } else {
    lo = 2 * kr.first;
    hi = 2 * (kr.first + kr.count) - 1;
  }
  hi = hi < m.N - 1 ? hi : m.N - 1;
}

// Classifies the pairs (queries [qlo, qhi], keys of `kr`): SKIP if no pair can be visible,
// FULL if every pair is visible, PARTIAL otherwise. SKIP and FULL are sound (never wrong);
// PARTIAL tiles evaluate `visible` per element, so the classification only affects speed.
__device__ __forceinline__ int classify(const MaskSpec& m, int qlo, int qhi, const KeyRun& kr,
                                       DocRange qd, DocRange kd) {
  const int klo = key_pos(m, kr, 0);
  const int khi = key_pos(m, kr, kr.count - 1);
  if (qlo >= m.N || klo >= m.N || klo > qhi) return TILE_SKIP;
  if (m.has_docs && (kd.hi < qd.lo || qd.hi < kd.lo)) return TILE_SKIP;
  bool full = khi <= qlo && qlo + kBlock - 1 < m.N;
  if (m.family != FAMILY_FULL) {
    const int tq_lo = qlo >> 1, tq_hi = qhi >> 1;
    const int tk_lo = kr.first, tk_hi = kr.first + kr.count - 1;
    if (kr.stream == STREAM_TEMPORARY) {
      if (tq_lo - tk_hi > m.window) return TILE_SKIP;
      if (tq_hi - tk_lo > m.window) full = false;
    } else if (m.has_pkw) {
      const int reach = m.pkw > 0 ? m.pkw : 0;  // the diagonal (distance 0) is always visible
      if (tq_lo - tk_hi > reach) return TILE_SKIP;
      if (tq_hi - tk_lo > m.pkw) full = false;
    }
  }
  if (m.has_docs && !(qd.lo == qd.hi && kd.lo == kd.hi && qd.lo == kd.lo)) full = false;
  return full ? TILE_FULL : TILE_PARTIAL;
}

// ---------------------------------------------------------------------------------------------
// Query-stationary schedule (forward and dQ): the workgroup owns queries [qa, qa + kTile) and
// walks key blocks of 32. Stream 0 is the natural stream (full family) or the persistent stream;
// stream 1 is the temporary stream (SPS families only).
// ---------------------------------------------------------------------------------------------
struct QSchedule {
  int n0, b0;  // stream-0 blocks [b0, b0 + n0)
  int n1, b1;  // temporary blocks [b1, b1 + n1)
  int stream0;
};

__device__ __forceinline__ QSchedule make_qschedule(const MaskSpec& m, int qa) {
  QSchedule s = {0, 0, 0, 0, STREAM_NATURAL};
  const int qhi = (qa + kTile - 1 < m.N - 1) ? qa + kTile - 1 : m.N - 1;
  if (m.family == FAMILY_FULL) {
    s.n0 = qhi / kBlock + 1;
    return s;
  }
  s.stream0 = STREAM_PERSISTENT;
  const int tq_lo = qa >> 1;
  // Persistent keys 2t+P <= qhi.
  const int tp_max = (qhi - m.P) >> 1;
  int tp_min = 0;
  if (m.has_pkw) {
    const int reach = m.pkw > 0 ? m.pkw : 0;
    tp_min = tq_lo - reach > 0 ? tq_lo - reach : 0;
  }
  if (tp_max >= tp_min) {
    s.b0 = tp_min / kBlock;
    s.n0 = tp_max / kBlock - s.b0 + 1;
  }
  // Temporary keys 2t+(1-P) <= qhi and t >= tq_lo - window.
  const int tt_max = (qhi - (1 - m.P)) >> 1;
  if (m.window >= 0) {
    const int tt_min = tq_lo - m.window > 0 ? tq_lo - m.window : 0;
    if (tt_max >= tt_min) {
      s.b1 = tt_min / kBlock;
      s.n1 = tt_max / kBlock - s.b1 + 1;
    }
  }
  return s;
}

__device__ __forceinline__ KeyRun qschedule_block(const QSchedule& s, int i) {
  KeyRun kr;
  kr.count = kBlock;
  if (i < s.n0) {
    kr.stream = s.stream0;
    kr.first = (s.b0 + i) * kBlock;
  } else {
    kr.stream = STREAM_TEMPORARY;
    kr.first = (s.b1 + i - s.n0) * kBlock;
  }
  return kr;
}

// ---------------------------------------------------------------------------------------------
// Key-stationary schedule (dK/dV): the workgroup owns kTile keys of one stream and walks query
// chunks of 32 positions [chunk*32, chunk*32 + 32).
// ---------------------------------------------------------------------------------------------
struct KSchedule {
  int c0, nc;  // query chunks [c0, c0 + nc)
};

__device__ __forceinline__ KSchedule make_kschedule(const MaskSpec& m, const KeyRun& kr) {
  KSchedule s = {0, 0};
  const int klo = key_pos(m, kr, 0);
  if (klo >= m.N) return s;
  int qlo = klo;  // causal: queries at or after the first key
  int qhi = m.N - 1;
  if (kr.stream == STREAM_TEMPORARY) {
    if (m.window < 0) return s;
    const int t_hi = kr.first + kr.count - 1 + m.window;  // last query token within the window
    const int p_hi = 2 * t_hi + 1;
    qhi = p_hi < qhi ? p_hi : qhi;
  } else if (kr.stream == STREAM_PERSISTENT && m.has_pkw) {
    const int reach = m.pkw > 0 ? m.pkw : 0;
    const int p_hi = 2 * (kr.first + kr.count - 1 + reach) + 1;
    qhi = p_hi < qhi ? p_hi : qhi;
  }
  if (qhi < qlo) return s;
  s.c0 = qlo / kBlock;
  s.nc = qhi / kBlock - s.c0 + 1;
  return s;
}

// Number of key-stationary workgroup tiles per (batch, head) and the run owned by tile `t`.
// SPS families: persistent-stream tiles first (they carry the most work), then temporary.
__host__ __device__ __forceinline__ int ktiles_per_head(int family, int N) {
  if (family == FAMILY_FULL) return (N + kTile - 1) / kTile;
  const int T = N / 2;
  return 2 * ((T + kTile - 1) / kTile);
}

__device__ __forceinline__ KeyRun ktile_run(int family, int N, int t) {
  KeyRun kr;
  kr.count = kTile;
  if (family == FAMILY_FULL) {
    kr.stream = STREAM_NATURAL;
    kr.first = t * kTile;
    return kr;
  }
  const int per = ((N / 2) + kTile - 1) / kTile;
  kr.stream = t < per ? STREAM_PERSISTENT : STREAM_TEMPORARY;
  kr.first = (t < per ? t : t - per) * kTile;
  return kr;
}

// Workgroup order: dispatch hands blocks to the 8 XCDs round-robin; give each XCD a contiguous
// range of logical tiles so that one (batch, head)'s K/V stays in one XCD's L2.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  constexpr int kXcd = 8;
  const int per = nblocks / kXcd;
  if (bid >= per * kXcd) return bid;
  return (bid % kXcd) * per + bid / kXcd;
}

}  // namespace sps
