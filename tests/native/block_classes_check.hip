// Host check of the closed-form block classes (add_block_classes / mask_class) against the per-block
// predicate classify_block on random wave spans and plans, including empty spans and spans without
// a common part. Prints "cases <n> bad <m>" and exits non-zero on any mismatch.
#include <cstdio>
#include <cstdlib>
#include <random>

#include "../../sps_amd/csrc/attn_tiles.hpp"

using namespace sps;

int main(int argc, char** argv) {
  const int iters = argc > 1 ? atoi(argv[1]) : 200000;
  std::mt19937 rng(1);
  auto r = [&](int n) { return (int)(rng() % (unsigned)n); };
  long bad = 0, cases = 0;
  for (int it = 0; it < iters; ++it) {
    // Span of two lane intervals in a row of up to R positions (or no visible index at all).
    auto span = [&](int R) {
      if (r(10) == 0) return WaveSpan{kEmptyLo, kEmptyHi, kEmptyLo, kEmptyHi};
      int a = r(R), b = r(R), c = r(R), d = r(R);
      if (a > b) std::swap(a, b);
      if (c > d) std::swap(c, d);
      WaveSpan w{a < c ? a : c, b > d ? b : d, a > c ? a : c, b < d ? b : d};
      if (r(4) == 0) w.max_lo = kEmptyLo, w.min_hi = kEmptyHi;  // a lane sees nothing
      return w;
    };
    const int R = 1 + r(6000);
    const WaveSpan w0 = span(R), w1 = span(R);
    const int n0 = r(80), n1 = r(80), b0 = r(200), b1 = r(200);
    const bool exact = r(3) != 0;
    BlockMask bm = {0ull, 0ull, 0ull, 0ull};
    add_block_classes(bm, w0, exact, 0, n0, b0);
    add_block_classes(bm, w1, exact, n0, n1, b1);
    for (int i = 0; i < 128; ++i) {
      const int want = i >= n0 + n1 ? TILE_SKIP
                                     : classify_block(i < n0 ? w0 : w1, kBlock * (i < n0 ? b0 + i : b1 + i - n0), exact);
      ++cases;
      if (mask_class(bm, i) != want) {
        if (bad < 5) printf("mismatch: iteration %d block %d\n", it, i);
        ++bad;
      }
    }
  }
  printf("cases %ld bad %ld\n", cases, bad);
  return bad != 0;
}
