// Host check that the kernels' lane intervals never decrease along a wave's 32 lanes, so that the
// four-lane-read span (wave_span_monotone) equals the span over every lane: for random rows (document
// ids in runs, including ids reused out of order), every family, persistent parity, window and
// persistent-key window, for every 32-query group (query-stationary, both key streams) and every
// 32-key group of each key stream (key-stationary). Prints "groups <n> bad <m>"; non-zero exit on
// any mismatch.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "../../sps_amd/csrc/attn_sched.hpp"

using namespace sps;

// Span over all lanes (the reduction's semantics: empty lanes push max_lo up and min_hi down).
static WaveSpan span_all(const Interval* r) {
  WaveSpan w{INT32_MAX, INT32_MIN, INT32_MIN, INT32_MAX};
  for (int l = 0; l < 32; ++l) {
    const bool e = r[l].lo > r[l].hi;
    w.min_lo = imin(w.min_lo, e ? kEmptyLo : r[l].lo);
    w.max_hi = imax(w.max_hi, e ? kEmptyHi : r[l].hi);
    w.max_lo = imax(w.max_lo, e ? kEmptyLo : r[l].lo);
    w.min_hi = imin(w.min_hi, e ? kEmptyHi : r[l].hi);
  }
  return w;
}

// The four-lane-read form, on the host.
static WaveSpan span_monotone(const Interval* r) {
  unsigned ne = 0;
  for (int l = 0; l < 32; ++l) ne |= (unsigned)(r[l].lo <= r[l].hi) << l;
  if (!ne) return WaveSpan{kEmptyLo, kEmptyHi, kEmptyLo, kEmptyHi};
  const int first = __builtin_ctz(ne), last = 31 - __builtin_clz(ne);
  const bool all = ne == 0xffffffffu;
  return WaveSpan{r[first].lo, r[last].hi, all ? r[31].lo : kEmptyLo, all ? r[0].hi : kEmptyHi};
}

static bool same(const WaveSpan& a, const WaveSpan& b) {
  return a.min_lo == b.min_lo && a.max_hi == b.max_hi && a.max_lo == b.max_lo && a.min_hi == b.min_hi;
}

int main(int argc, char** argv) {
  const int iters = argc > 1 ? atoi(argv[1]) : 300;
  std::mt19937 rng(7);
  auto r = [&](int n) { return (int)(rng() % (unsigned)n); };
  long groups = 0, bad = 0;
  for (int it = 0; it < iters; ++it) {
    MaskSpec m;
    m.family = r(3);
    m.P = m.family == FAMILY_REVERSE_SPS ? 1 : 0;
    m.N = 1 + r(700);
    if (m.family != FAMILY_FULL) m.N = 2 * ((m.N + 1) / 2);
    m.window = r(4) == 0 ? -1 : r(80);
    m.has_pkw = m.family != FAMILY_FULL && r(3) == 0;
    m.pkw = r(3) == 0 ? -1 : r(60);
    m.has_docs = 1;
    // Document ids in runs (a token's two positions share its id), sometimes reused out of order.
    std::vector<int> ids(m.N), run_start(m.N), run_end(m.N);
    int id = 0;
    for (int p = 0; p < m.N; ++p) {
      if ((m.family == FAMILY_FULL || p % 2 == 0) && p > 0 && r(40) == 0) id = r(5) == 0 ? r(4) : id + 1;
      ids[p] = id;
    }
    for (int p = 0; p < m.N; ++p) run_start[p] = (p > 0 && ids[p] == ids[p - 1]) ? run_start[p - 1] : p;
    for (int p = m.N - 1; p >= 0; --p) run_end[p] = (p + 1 < m.N && ids[p] == ids[p + 1]) ? run_end[p + 1] : p;
    // Query-stationary groups.
    for (int q0 = 0; q0 < m.N; q0 += 32) {
      Interval r0[32], r1[32];
      for (int l = 0; l < 32; ++l) {
        const int q = q0 + l;
        if (q < m.N) {
          query_intervals(m, q, run_start[q], r0[l], r1[l]);
        } else {
          r0[l] = r1[l] = Interval{kEmptyLo, kEmptyHi};
        }
      }
      groups += 2;
      if (!same(span_all(r0), span_monotone(r0)) || !same(span_all(r1), span_monotone(r1))) {
        if (bad < 5) printf("query group mismatch: it %d q0 %d\n", it, q0);
        ++bad;
      }
    }
    // Key-stationary groups of each stream.
    const int streams[2] = {m.family == FAMILY_FULL ? (int)STREAM_NATURAL : (int)STREAM_PERSISTENT, STREAM_TEMPORARY};
    for (int si = 0; si < (m.family == FAMILY_FULL ? 1 : 2); ++si) {
      const int stream = streams[si], len = stream_len(m.family, m.N, stream, m.P);
      for (int t0 = 0; t0 < len; t0 += 32) {
        Interval rk[32];
        for (int l = 0; l < 32; ++l) {
          const int t = t0 + l;
          rk[l] = Interval{kEmptyLo, kEmptyHi};
          if (t < len) {
            const int kp = stream_pos(m, stream, t);
            const int last = key_last_query(m, stream, kp, run_end[kp]);
            if (last >= kp) rk[l] = Interval{kp, last};
          }
        }
        ++groups;
        if (!same(span_all(rk), span_monotone(rk))) {
          if (bad < 5) printf("key group mismatch: it %d stream %d t0 %d\n", it, stream, t0);
          ++bad;
        }
      }
    }
  }
  printf("groups %ld bad %ld\n", groups, bad);
  return bad != 0;
}
