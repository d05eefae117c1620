// Host check of the row-layout prepass's tile plans: the closed-form unions q_tile_union and
// k_tile_union (from a tile's first and last few rows) against the union over every query (key)
// of the tile, for random rows (document ids in runs, including rows whose ids decrease, which the
// prepass records as one run), every family, persistent parity, window and persistent-key window.
// Prints "tiles <n> bad <m>"; non-zero exit on any mismatch.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "../../sps_amd/csrc/attn_sched.hpp"

using namespace sps;

static bool same(const Interval& a, const Interval& b) {
  const bool ea = a.lo > a.hi, eb = b.lo > b.hi;
  return ea == eb && (ea || (a.lo == b.lo && a.hi == b.hi));
}

int main(int argc, char** argv) {
  const int iters = argc > 1 ? atoi(argv[1]) : 2000;
  std::mt19937 rng(11);
  auto r = [&](int n) { return (int)(rng() % (unsigned)n); };
  long tiles = 0, bad = 0;
  for (int it = 0; it < iters; ++it) {
    MaskSpec m;
    m.family = r(3);
    m.P = m.family == FAMILY_REVERSE_SPS ? 1 : 0;
    m.N = 1 + r(1200);
    if (m.family != FAMILY_FULL) m.N = 2 * ((m.N + 1) / 2);
    const int wr = r(6);
    m.window = wr == 0 ? -1 : wr == 1 ? 0 : wr == 2 ? m.N : r(80);
    m.has_pkw = m.family != FAMILY_FULL && r(3) == 0;
    m.pkw = r(3) == 0 ? -1 : r(4) == 0 ? 0 : r(60);
    m.has_docs = 1;
    // Document ids in runs (a token's two positions share its id); short documents are common and
    // some rows reuse ids out of order.
    std::vector<int> ids(m.N), start(m.N), end(m.N);
    const int rate = 1 + r(60);
    int id = 0;
    for (int p = 0; p < m.N; ++p) {
      if ((m.family == FAMILY_FULL || p % 2 == 0) && p > 0 && r(rate) == 0) id = r(8) == 0 ? r(4) : id + 1;
      ids[p] = id;
    }
    bool mono = true;
    for (int p = 1; p < m.N; ++p) mono &= ids[p] >= ids[p - 1];
    for (int p = 0; p < m.N; ++p) start[p] = !mono ? 0 : (p > 0 && ids[p] == ids[p - 1]) ? start[p - 1] : p;
    for (int p = m.N - 1; p >= 0; --p) end[p] = !mono ? m.N - 1 : (p + 1 < m.N && ids[p] == ids[p + 1]) ? end[p + 1] : p;
    auto st = [&](int q) { return start[q]; };
    auto en = [&](int k) { return end[k]; };
    // Query tiles.
    for (int qt = 0; qt < q_tiles(m.N); ++qt) {
      Interval a0{kEmptyLo, kEmptyHi}, a1{kEmptyLo, kEmptyHi};
      for (int q = qt * kTile; q < imin((qt + 1) * kTile, m.N); ++q) {
        Interval i0, i1;
        query_intervals(m, q, start[q], i0, i1);
        if (i0.lo <= i0.hi) a0 = Interval{imin(a0.lo, i0.lo), imax(a0.hi, i0.hi)};
        if (i1.lo <= i1.hi) a1 = Interval{imin(a1.lo, i1.lo), imax(a1.hi, i1.hi)};
      }
      Interval u0, u1;
      q_tile_union(m, qt, st, u0, u1);
      ++tiles;
      if (!same(a0, u0) || !same(a1, u1)) {
        if (bad < 5)
          printf("query tile mismatch: it %d family %d N %d w %d pkw %d/%d tile %d: [%d,%d] [%d,%d] vs [%d,%d] [%d,%d]\n",
                 it, m.family, m.N, m.window, m.has_pkw, m.pkw, qt, a0.lo, a0.hi, a1.lo, a1.hi, u0.lo, u0.hi, u1.lo,
                 u1.hi);
        ++bad;
      }
    }
    // Key tiles.
    for (int kt = 0; kt < k_tiles(m.family, m.N, m.P); ++kt) {
      int stream, first;
      k_tile_run(m, kt, stream, first);
      const int len = stream_len(m.family, m.N, stream, m.P);
      Interval a{kEmptyLo, kEmptyHi};
      for (int t = first; t < imin(first + kTile, len); ++t) {
        const int kp = stream_pos(m, stream, t);
        const int last = key_last_query(m, stream, kp, end[kp]);
        if (last >= kp) a = Interval{imin(a.lo, kp), imax(a.hi, last)};
      }
      const Interval u = k_tile_union(m, kt, en);
      ++tiles;
      if (!same(a, u)) {
        if (bad < 5)
          printf("key tile mismatch: it %d family %d N %d w %d pkw %d/%d tile %d: [%d,%d] vs [%d,%d]\n", it, m.family,
                 m.N, m.window, m.has_pkw, m.pkw, kt, a.lo, a.hi, u.lo, u.hi);
        ++bad;
      }
    }
  }
  printf("tiles %ld bad %ld\n", tiles, bad);
  return bad != 0;
}
