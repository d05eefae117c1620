// Host check of fast_div (division by a launch-time divisor) and of the workgroup -> (row, head)
// slot rotation built on it: exhaustive over small divisors and dividends, random dividends below
// 2^31 for every divisor up to 1 << 16 and random larger ones, and the rotation against
// (j + rank H) mod B H. Prints "cases <n> bad <m>"; non-zero exit on any mismatch.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>

#include "../../sps_amd/csrc/attn_sched.hpp"

using namespace sps;

int main(int argc, char** argv) {
  const int iters = argc > 1 ? atoi(argv[1]) : 2000;
  std::mt19937_64 rng(5);
  long cases = 0, bad = 0;
  auto check = [&](uint32_t x, uint32_t d, const FastDiv& f) {
    ++cases;
    if (fast_div(x, f) != x / d) {
      if (bad < 10) printf("fast_div(%u, %u) = %u, want %u\n", x, d, fast_div(x, f), x / d);
      ++bad;
    }
  };
  for (uint32_t d = 1; d <= 1024; ++d) {
    const FastDiv f = make_fast_div(d);
    for (uint32_t x = 0; x < 4 * 1024 + 7; ++x) check(x, d, f);
    for (int k = 0; k < 64; ++k) check((uint32_t)(rng() & 0x7fffffffu), d, f);
    check(0x7fffffffu, d, f);
    check(0x7ffffffeu, d, f);
  }
  for (uint32_t d = 1025; d <= (1u << 16); ++d) {
    const FastDiv f = make_fast_div(d);
    for (int k = 0; k < 16; ++k) check((uint32_t)(rng() & 0x7fffffffu), d, f);
    check(0x7fffffffu, d, f);
    check(d * 3 - 1, d, f);
    check(d * 3, d, f);
  }
  for (int it = 0; it < iters; ++it) {
    const uint32_t d = 1 + (uint32_t)(rng() % 0x7fffffffu);
    const FastDiv f = make_fast_div(d);
    for (int k = 0; k < 16; ++k) check((uint32_t)(rng() & 0x7fffffffu), d, f);
    check(0x7fffffffu, d, f);
  }
  // The slot rotation of workgroup_slot (attn_tiles.hpp), in host form.
  for (int it = 0; it < iters; ++it) {
    const int B = 1 + (int)(rng() % 64), H = 1 + (int)(rng() % 64), BH = B * H;
    const FastDiv fbh = make_fast_div(BH), fb = make_fast_div(B), fh = make_fast_div(H);
    for (int k = 0; k < 64; ++k) {
      const uint32_t id = (uint32_t)(rng() % (uint64_t)(BH * 200));
      const int rank = (int)fast_div(id, fbh), j = (int)id - rank * BH;
      int bh = j + (rank - (int)fast_div((uint32_t)rank, fb) * B) * H;
      if (bh >= BH) bh -= BH;
      const int b = (int)fast_div((uint32_t)bh, fh), h = bh - b * H;
      const int want = (int)(((int64_t)(id % BH) + (int64_t)(id / BH) * H) % BH);
      ++cases;
      if (rank != (int)(id / BH) || bh != want || b != want / H || h != want % H) {
        if (bad < 10) printf("slot: B %d H %d id %u -> rank %d bh %d, want %d\n", B, H, id, rank, bh, want);
        ++bad;
      }
    }
  }
  printf("cases %ld bad %ld\n", cases, bad);
  return bad ? 1 : 0;
}
