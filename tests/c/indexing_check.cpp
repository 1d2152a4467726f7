// The kernels' index arithmetic (pega-omni_amd/csrc/indexing.h) on the host.
// Page division against the division and remainder operators: every page
// size 1..4096 over every t < 2^16 and around multiples of the page near
// 2^31, then larger pages on edge values and a seeded sample of t < 2^31.
// Decode split rotation: for 1..64 splits and 512 S units, every unit's
// workgroup slots map to its split indices one to one, and over whole periods
// every XCD (workgroup index mod 8) gets the same number of each split index.
// Run by tests/test_c_abi.py (make indexing).
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <initializer_list>

#include "indexing.h"

static long long g_checked = 0;

static void check(const omni::PageDiv& d, int t) {
  const int q = omni::page_index(d, t);
  const int64_t slot = omni::page_slot(d, 7, t);
  ++g_checked;
  if (q != t / d.page || slot != (int64_t)7 * d.page + t % d.page) {
    std::printf("FAIL page=%d t=%d: index %d (want %d) slot %lld\n", d.page, t, q, t / d.page, (long long)slot);
    std::exit(1);
  }
}

static void edges(const omni::PageDiv& d) {
  const int64_t top = INT32_MAX;
  for (int64_t k : {top / d.page, top / d.page - 1, top / d.page - 2, (int64_t)1 << 16, (int64_t)1000003})
    for (int64_t dt = -2; dt <= 2; ++dt) {
      const int64_t t = k * d.page + dt;
      if (t >= 0 && t <= top) check(d, (int)t);
    }
  check(d, (int)top);
  check(d, (int)top - 1);
}

int main() {
  for (int page = 1; page <= 4096; ++page) {
    const omni::PageDiv d = omni::make_page_div(page);
    if ((d.magic == 0) != ((page & (page - 1)) == 0)) {
      std::printf("FAIL page=%d: magic %u\n", page, d.magic);
      return 1;
    }
    for (int t = 0; t < (1 << 16); ++t) check(d, t);
    edges(d);
  }
  uint64_t x = 0x9E3779B97F4A7C15ull;
  auto next = [&]() {
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    return x;
  };
  for (int page : {4097, 6000, 65535, 65536, 65537, 1000000, 1 << 20, 12345678, INT32_MAX / 3, INT32_MAX}) {
    const omni::PageDiv d = omni::make_page_div(page);
    edges(d);
    for (int i = 0; i < 200000; ++i) check(d, (int)(next() & INT32_MAX));
  }
  for (int i = 0; i < 2000000; ++i) {
    const int page = 1 + (int)(next() % 100000);
    check(omni::make_page_div(page), (int)(next() & INT32_MAX));
  }
  std::printf("page division: %lld checks passed\n", g_checked);
  long long rot = 0;
  for (int S = 1; S <= 64; ++S) {
    const int units = 512 * S;  // whole periods of P S units (P divides 8)
    static int per_xcd[8][64];
    for (auto& row : per_xcd)
      for (int& v : row) v = 0;
    for (int u = 0; u < units; ++u) {
      unsigned long long seen = 0;
      for (int slot = 0; slot < S; ++slot) {
        const int split = omni::rotated_split(slot, u, S);
        if (split < 0 || split >= S || (seen >> split & 1)) {
          std::printf("FAIL rotation S=%d u=%d slot=%d -> %d\n", S, u, slot, split);
          return 1;
        }
        seen |= 1ull << split;
        ++per_xcd[((long long)u * S + slot) % 8][split];
        ++rot;
      }
    }
    for (int x = 0; x < 8; ++x)
        for (int k = 0; k < S; ++k)
          if (per_xcd[x][k] != per_xcd[0][0]) {
            std::printf("FAIL balance S=%d xcd=%d split=%d: %d vs %d\n", S, x, k, per_xcd[x][k], per_xcd[0][0]);
            return 1;
          }
  }
  std::printf("split rotation: %lld checks passed\n", rot);
  return 0;
}
