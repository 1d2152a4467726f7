// Index arithmetic shared by the kernels, the host code that fills their
// arguments, and the host checks in tests/c/indexing_check.cpp.
//
// Page division: the page-table slot rule pages[t / page] * page + t % page (crates/omni-qwen3/kernels/qwen3.cu:
// 210-214, crates/omni-personaplex/kernels/lm.cu:189-192), which accepts any
// positive page.
//
// Kernels divide with a multiply (the round-up method of Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994):
// with shift = ceil(log2 page) and magic = floor(2^32 (2^shift - page) / page)
// + 1, t / page = (umulhi(t, magic) + t) >> shift for every 0 <= t < 2^31
// (the sum stays below 2^32 because umulhi(t, magic) < t). A power of two has
// magic 0, so its division is the plain shift.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define OMNI_HD __host__ __device__
#else
#define OMNI_HD
#endif

namespace omni {

struct PageDiv {
  int32_t page;    // > 0
  uint32_t magic;  // 0 for a power of two
  int32_t shift;   // ceil(log2 page)
};

inline PageDiv make_page_div(int page) {
  PageDiv d{page, 0u, 0};
  while ((1LL << d.shift) < (long long)page) ++d.shift;
  if ((1LL << d.shift) != (long long)page)
    d.magic = (uint32_t)((((uint64_t)1 << 32) * (((uint64_t)1 << d.shift) - (uint64_t)page)) / (uint64_t)page + 1);
  return d;
}

inline OMNI_HD bool page_pow2(const PageDiv& d) { return d.magic == 0u; }

// t / page for 0 <= t < 2^31.
inline OMNI_HD int page_index(const PageDiv& d, int t) {
  const uint32_t hi = (uint32_t)(((uint64_t)(uint32_t)t * d.magic) >> 32);
  return (int)((hi + (uint32_t)t) >> d.shift);
}

// Physical slot of token t whose page (page_index(d, t)) has id pid.
inline OMNI_HD int64_t page_slot(const PageDiv& d, int pid, int t) {
  return (int64_t)pid * d.page + (t - page_index(d, t) * d.page);
}

// Split index of workgroup slot `slot` (0 .. S - 1) of decode unit u, S >= 1.
// Workgroup i runs on XCD i % 8, and a unit's S slots are consecutive
// workgroups, so slot x of unit u lands on XCD (x + S u) % 8, a phase with
// period P = 8 / gcd(S, 8) in u. Slot x alone would pin each split index to a
// few XCDs (S = 2 or 4: the short rows' absent last splits leave half the XCDs
// idle while the other half read every first split). Rotating the slot by
// u / P pairs every phase with every split index over P S consecutive units,
// so each XCD gets an even share of each split index. For each u the map is a
// permutation of 0 .. S - 1, so every split of a unit runs exactly once.
inline OMNI_HD int rotated_split(int slot, int u, int S) {
  const int tz = __builtin_ctz((unsigned)S);
  const int P = 8 >> (tz < 3 ? tz : 3);
  return (slot + u / P) % S;
}

}  // namespace omni

#undef OMNI_HD
