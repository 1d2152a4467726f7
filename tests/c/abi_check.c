/*
 * A compiled C consumer of include/omni_attn.h: built with gcc -std=c11 -Wall
 * -Wextra -Werror against the header and linked to libomni_attn.so, the way
 * the engines' FFI crate binds it (the typed launch ABI the reference's kern
 * manifest checks, crates/omni-kern/src/lib.rs:261-302). It runs host-only
 * entry points and the validation that every run call does before it
 * launches, so it needs no GPU, and asserts the documented return codes.
 *
 * Exit status 0 and "abi_check: N checks passed" on success; the first failed
 * check prints its line and exits 1.
 */
#include <stddef.h>
#include <stdint.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "omni_attn.h"

static int g_checks = 0;

#define CHECK(cond)                                                                    \
  do {                                                                                 \
    ++g_checks;                                                                        \
    if (!(cond)) {                                                                     \
      fprintf(stderr, "abi_check: %s:%d: failed: %s (last error: \"%s\")\n", __FILE__, \
              __LINE__, #cond, omni_attn_last_error());                                \
      exit(1);                                                                         \
    }                                                                                  \
  } while (0)

/* The plan structs are part of the ABI: the Rust #[repr(C)] mirrors depend on
 * these sizes and offsets. */
_Static_assert(sizeof(omni_attn_decode_plan) == 40, "decode plan size");
_Static_assert(offsetof(omni_attn_decode_plan, group_heads) == 28, "decode plan group_heads");
_Static_assert(offsetof(omni_attn_decode_plan, workspace_bytes) == 32, "decode plan workspace_bytes");
_Static_assert(sizeof(omni_attn_prefill_plan) == 40, "prefill plan size");
_Static_assert(offsetof(omni_attn_prefill_plan, work_bytes) == 24, "prefill plan work_bytes");
_Static_assert(offsetof(omni_attn_prefill_plan, workgroups) == 32, "prefill plan workgroups");
_Static_assert(offsetof(omni_attn_prefill_plan, exact_p) == 36, "prefill plan exact_p");

/* A non-null address no call below dereferences: every call that receives it
 * fails validation before touching device memory. */
static void* const kFake = (void*)(uintptr_t)256;

static void check_decode_plan(void) {
  omni_attn_decode_plan p;
  CHECK(omni_attn_decode_plan_init(128, 32, 32, 16, 3000, 0, &p) == OMNI_ATTN_OK);
  CHECK(p.rows == 128 && p.hq == 32 && p.hk == 32 && p.page == 16 && p.max_len == 3000);
  CHECK(p.chunk % 128 == 0 && p.splits == (3000 + p.chunk - 1) / p.chunk);
  CHECK(p.workspace_bytes == (p.splits > 1 ? 128LL * 32 * p.splits * 129 * 4 : 0));
  CHECK(p.group_heads == 0);
  CHECK(omni_attn_decode_plan_init(4, 16, 8, 16, 1000, 256, &p) == OMNI_ATTN_OK && p.chunk == 256 && p.splits == 4);
  /* the FP8 plan: split size for the FP8 kernel, otherwise the same plan */
  CHECK(omni_attn_decode_plan_init_fp8(128, 32, 16, 3000, 0, &p) == OMNI_ATTN_OK && p.chunk == 768 && p.splits == 4 &&
        p.hq == 32 && p.hk == 32 && p.workspace_bytes == 128LL * 32 * 4 * 129 * 4);
  CHECK(omni_attn_decode_plan_init_fp8(4, 0, 16, 100, 0, &p) == OMNI_ATTN_EINVAL);
  /* documented rejections */
  CHECK(omni_attn_decode_plan_init(4, 16, 6, 16, 100, 0, &p) == OMNI_ATTN_EINVAL);        /* hq % hk */
  CHECK(omni_attn_decode_plan_init(4, 16, 2, 16, 100, 0, &p) == OMNI_ATTN_EUNSUPPORTED);  /* G = 8 */
  CHECK(omni_attn_decode_plan_init(4, 16, 8, 0, 100, 0, &p) == OMNI_ATTN_EINVAL);         /* page */
  CHECK(omni_attn_decode_plan_init(4, 16, 8, 12, 100, 0, &p) == OMNI_ATTN_OK && p.page == 12); /* any page > 0 */
  CHECK(omni_attn_decode_plan_init(4, 16, 8, 16, 0, 0, &p) == OMNI_ATTN_EINVAL);          /* max_len */
  CHECK(omni_attn_decode_plan_init(4, 16, 8, 16, 100, 100, &p) == OMNI_ATTN_EINVAL);      /* chunk */
  CHECK(omni_attn_decode_plan_init(70000, 16, 8, 16, 100, 0, &p) == OMNI_ATTN_EINVAL);    /* rows */
  CHECK(omni_attn_decode_plan_init(4, 16, 8, 16, 100, 0, NULL) == OMNI_ATTN_EINVAL);
  CHECK(strlen(omni_attn_last_error()) > 0);
}

static void check_decode_run_validation(void) {
  omni_attn_decode_plan p;
  CHECK(omni_attn_decode_plan_init(4, 16, 8, 16, 1000, 128, &p) == OMNI_ATTN_OK && p.splits == 8);
  /* split plan without a workspace */
  CHECK(omni_qwen3_attend(kFake, kFake, kFake, NULL, 0, kFake, kFake, 16, kFake, 16, 8, 0.1f, &p, NULL, NULL) ==
        OMNI_ATTN_EWORKSPACE);
  /* plan made for another shape */
  CHECK(omni_qwen3_attend(kFake, kFake, kFake, NULL, 0, kFake, kFake, 16, kFake, 16, 4, 0.1f, &p, kFake, NULL) ==
        OMNI_ATTN_EINVAL);
  /* null device pointers, ragged without seq, null plan, bad scale */
  CHECK(omni_qwen3_attend(NULL, kFake, kFake, NULL, 0, kFake, kFake, 16, kFake, 16, 8, 0.1f, &p, kFake, NULL) ==
        OMNI_ATTN_EINVAL);
  CHECK(omni_qwen3_attend(kFake, kFake, kFake, NULL, 1, kFake, kFake, 16, kFake, 16, 8, 0.1f, &p, kFake, NULL) ==
        OMNI_ATTN_EINVAL);
  CHECK(omni_qwen3_attend(kFake, kFake, kFake, NULL, 0, kFake, kFake, 16, kFake, 16, 8, 0.1f, NULL, kFake, NULL) ==
        OMNI_ATTN_EINVAL);
  CHECK(omni_qwen3_attend(kFake, kFake, kFake, NULL, 0, kFake, kFake, 16, kFake, 16, 8, 1.0f / 0.0f, &p, kFake,
                          NULL) == OMNI_ATTN_EINVAL);
  CHECK(omni_attn_decode_run_lastlen(NULL, kFake, kFake, NULL, 0, kFake, kFake, 16, kFake, 16, 8, 0.1f, &p, kFake,
                                     NULL) == OMNI_ATTN_EINVAL);
  /* lm_attend needs a positive ring */
  omni_attn_decode_plan m;
  CHECK(omni_attn_decode_plan_init(4, 8, 8, 16, 1000, 128, &m) == OMNI_ATTN_OK);
  CHECK(omni_lm_attend(kFake, kFake, kFake, NULL, 0, kFake, kFake, 16, kFake, 8, 0.1f, 0, &m, kFake, NULL) ==
        OMNI_ATTN_EINVAL);
  CHECK(omni_lm_attend_fp8(kFake, kFake, kFake, NULL, 0, kFake, kFake, 16, kFake, 8, 0.1f, -1, &m, kFake, NULL) ==
        OMNI_ATTN_EINVAL);
  m.group_heads = 3; /* not 1, 2, 4 or 8 */
  CHECK(omni_lm_attend_fp8(kFake, kFake, kFake, NULL, 0, kFake, kFake, 16, kFake, 8, 0.1f, 1000, &m, kFake, NULL) ==
        OMNI_ATTN_EINVAL);
  /* dense: base + per beyond the span, plan too short */
  omni_attn_decode_plan d;
  CHECK(omni_attn_decode_plan_init(4, 16, 8, 1, 16, 0, &d) == OMNI_ATTN_OK);
  CHECK(omni_qwen3_attend_dense(kFake, kFake, 1, 16, 16, kFake, 16, 8, 0.1f, &d, kFake, NULL) == OMNI_ATTN_EINVAL);
  CHECK(omni_qwen3_attend_dense(kFake, kFake, 4, 14, 32, kFake, 16, 8, 0.1f, &d, kFake, NULL) == OMNI_ATTN_EINVAL);
  /* the allocation-free call: a plan above its static scratch is rejected */
  omni_attn_decode_plan big;
  CHECK(omni_attn_decode_plan_init(4096, 32, 32, 16, 65536, 128, &big) == OMNI_ATTN_OK);
  CHECK(big.workspace_bytes > OMNI_ATTN_NOALLOC_SCRATCH_BYTES);
  CHECK(omni_qwen3_attend_noalloc(kFake, kFake, kFake, NULL, 0, kFake, kFake, 16, kFake, 32, 32, 0.1f, &big, NULL) ==
        OMNI_ATTN_EWORKSPACE);
  CHECK(omni_qwen3_attend_noalloc(kFake, kFake, kFake, NULL, 0, kFake, kFake, 16, kFake, 32, 32, 0.1f, NULL, NULL) ==
        OMNI_ATTN_EINVAL);
  /* a zero-row plan is a no-op */
  omni_attn_decode_plan z;
  CHECK(omni_attn_decode_plan_init(0, 16, 8, 16, 100, 0, &z) == OMNI_ATTN_OK);
  CHECK(omni_qwen3_attend(NULL, NULL, NULL, NULL, 0, NULL, NULL, 16, NULL, 16, 8, 0.1f, &z, NULL, NULL) ==
        OMNI_ATTN_OK);
}

static void check_table(void) {
  /* two sequences of 3 and 2 pages (page 16) in a pool of 8 pages */
  const int32_t indptr[3] = {0, 3, 5};
  const int32_t pages[5] = {7, 2, 5, 0, 6};
  const int32_t pos[2] = {47, 20};
  CHECK(omni_attn_check_table(indptr, 2, pages, 8, pos, NULL, 0, 2, 16, 0) == OMNI_ATTN_OK);
  const int32_t pos_long[2] = {48, 20}; /* 49 tokens need 4 pages */
  CHECK(omni_attn_check_table(indptr, 2, pages, 8, pos_long, NULL, 0, 2, 16, 0) == OMNI_ATTN_ETABLE);
  CHECK(omni_attn_check_table(indptr, 2, pages, 8, pos_long, NULL, 0, 2, 16, 40) == OMNI_ATTN_OK); /* ring cap */
  const int32_t bad_pages[5] = {7, 2, 8, 0, 6};
  CHECK(omni_attn_check_table(indptr, 2, bad_pages, 8, pos, NULL, 0, 2, 16, 0) == OMNI_ATTN_ETABLE);
  const int32_t bad_indptr[3] = {0, 3, 2};
  CHECK(omni_attn_check_table(bad_indptr, 2, pages, 8, NULL, NULL, 0, 0, 16, 0) == OMNI_ATTN_ETABLE);
  const int32_t bad_start[3] = {1, 3, 5};
  CHECK(omni_attn_check_table(bad_start, 2, pages, 8, NULL, NULL, 0, 0, 16, 0) == OMNI_ATTN_ETABLE);
  const int32_t seq[3] = {0, 1, 2}; /* row 2 names a missing sequence */
  const int32_t pos3[3] = {1, 2, 3};
  CHECK(omni_attn_check_table(indptr, 2, pages, 8, pos3, seq, 1, 3, 16, 0) == OMNI_ATTN_ETABLE);
  CHECK(omni_attn_check_table(indptr, 2, pages, 8, pos3, seq, 1, 2, 16, 0) == OMNI_ATTN_OK);
  CHECK(omni_attn_check_table(NULL, 2, pages, 8, pos, NULL, 0, 2, 16, 0) == OMNI_ATTN_EINVAL);
}

static void check_prefill_plan(void) {
  /* two sequences: 300 rows at positions 10.., 5 rows at 0.. (G = 4: 64 positions per tile) */
  enum { kRows = 305 };
  int32_t seq[kRows], pos[kRows];
  for (int n = 0; n < 300; ++n) seq[n] = 0, pos[n] = 10 + n;
  for (int n = 300; n < kRows; ++n) seq[n] = 1, pos[n] = n - 300;
  omni_attn_prefill_plan p;
  /* too small a work list: EWORKSPACE with the size set */
  int32_t tiny[4];
  CHECK(omni_attn_prefill_plan_init(kRows, 32, 8, 16, seq, pos, tiny, 4, &p) == OMNI_ATTN_EWORKSPACE);
  const int tiles = (300 + 63) / 64 + 1;
  CHECK(p.tiles == tiles && p.work_bytes == (int64_t)(16 + 4 * tiles * 8) * 4);
  int32_t* work = (int32_t*)malloc((size_t)p.work_bytes);
  CHECK(work != NULL);
  CHECK(omni_attn_prefill_plan_init(kRows, 32, 8, 16, seq, pos, work, p.work_bytes / 4, &p) == OMNI_ATTN_OK);
  CHECK(p.exact_p == 0); /* P rounded to bf16 unless the caller sets exact_p = 1 */
  CHECK(p.rows == kRows && p.hq == 32 && p.hk == 8 && p.tile_rows == 256);
  /* header: XCD ranges cover every item once, in order, widths differ by <= 1 */
  const int items = tiles * 8;
  CHECK(work[0] == 0 && work[8] == items);
  int widest = 0, narrowest = items;
  for (int x = 0; x < 8; ++x) {
    const int w = work[x + 1] - work[x];
    CHECK(w >= 0);
    if (w > widest) widest = w;
    if (w < narrowest) narrowest = w;
  }
  CHECK(widest - narrowest <= 1 && p.workgroups == 8 * widest);
  /* every (tile, kv head) appears once and every row is covered once per head */
  int covered[8][kRows];
  memset(covered, 0, sizeof covered);
  for (int k = 0; k < items; ++k) {
    const int32_t* it = work + 16 + 4 * k;
    CHECK(it[0] == 0 || it[0] == 1);
    CHECK(it[2] >= 1 && it[2] <= 64 && it[3] >= 0 && it[3] < 8);
    for (int r = it[1]; r < it[1] + it[2]; ++r) {
      CHECK(seq[r] == it[0]);
      ++covered[it[3]][r];
    }
  }
  for (int h = 0; h < 8; ++h)
    for (int r = 0; r < kRows; ++r) CHECK(covered[h][r] == 1);
  free(work);
  /* rejections */
  CHECK(omni_attn_prefill_plan_init(4, 48, 3, 16, seq, pos, NULL, 0, &p) == OMNI_ATTN_EUNSUPPORTED); /* G = 16 */
  CHECK(omni_attn_prefill_plan_init(4, 32, 8, 0, seq, pos, NULL, 0, &p) == OMNI_ATTN_EINVAL); /* page */
  CHECK(omni_attn_prefill_plan_init(4, 32, 8, 16, NULL, pos, NULL, 0, &p) == OMNI_ATTN_EINVAL);
  const int32_t neg[2] = {-1, 0}, s2[2] = {0, 0};
  CHECK(omni_attn_prefill_plan_init(2, 32, 8, 16, s2, neg, NULL, 0, &p) == OMNI_ATTN_ETABLE);
  CHECK(omni_attn_prefill_run(NULL, kFake, kFake, kFake, kFake, kFake, kFake, kFake, 0.1f, kFake, NULL) ==
        OMNI_ATTN_EINVAL);
}

static void check_dit_validation(void) {
  int32_t* kvl = (int32_t*)kFake;
  CHECK(omni_hidream_attend(kFake, kFake, kFake, kFake, -1, kvl, 48 * 128, 0, 0.1f, 32, 8, NULL) == OMNI_ATTN_EINVAL);
  CHECK(omni_hidream_attend(kFake, kFake, kFake, kFake, 0, kvl, 48 * 128, 0, 0.1f, 32, 8, NULL) == OMNI_ATTN_OK);
  CHECK(omni_hidream_attend(kFake, NULL, kFake, kFake, 16, kvl, 48 * 128, 0, 0.1f, 32, 8, NULL) == OMNI_ATTN_EINVAL);
  CHECK(omni_hidream_attend(kFake, kFake, kFake, kFake, 16, kvl, 48 * 128, 0, 0.1f, 32, 6, NULL) == OMNI_ATTN_EINVAL);
  CHECK(omni_hidream_attend(kFake, kFake, kFake, kFake, 16, kvl, 48 * 128, 0, 0.1f, 48, 3, NULL) ==
        OMNI_ATTN_EUNSUPPORTED);
  CHECK(omni_hidream_attend(kFake, kFake, kFake, kFake, 16, kvl, 100, 0, 0.1f, 32, 8, NULL) == OMNI_ATTN_EINVAL);
  CHECK(omni_hidream_attend_batched(kFake, kFake, kFake, kFake, 16, kvl, 48 * 128, 0, 0.1f, 32, 8, -1, 0, 0, 0,
                                    NULL) == OMNI_ATTN_EINVAL);
  CHECK(omni_hidream_attend_ws(kFake, kFake, kFake, kFake, 16, kvl, 48 * 128, 0, 0.1f, 32, 8, 1, 0, 0, 0,
                               (void*)(uintptr_t)264, 1 << 20, NULL) == OMNI_ATTN_EINVAL); /* misaligned */
}

static void check_rows(void) {
  omni_attn_rows* r = omni_attn_rows_new(16, 0);
  CHECK(r != NULL);
  const int32_t lease_a[3] = {9, 4, 1}, lease_b[1] = {6};
  CHECK(omni_attn_rows_push(r, lease_a, 3, 30, 5, 0) == OMNI_ATTN_OK); /* positions 30..34 */
  CHECK(omni_attn_rows_push(r, lease_b, 1, 3, 1, 1) == OMNI_ATTN_OK);
  int rows = 0, seqs = 0, npages = 0;
  CHECK(omni_attn_rows_count(r, &rows, &seqs, &npages) == OMNI_ATTN_OK);
  CHECK(rows == 6 && seqs == 2 && npages == 4);
  const int32_t* pos = omni_attn_rows_get(r, OMNI_ATTN_ROWS_POS);
  const int32_t* slot = omni_attn_rows_get(r, OMNI_ATTN_ROWS_SLOT);
  const int32_t* seq = omni_attn_rows_get(r, OMNI_ATTN_ROWS_SEQ);
  const int32_t* indptr = omni_attn_rows_get(r, OMNI_ATTN_ROWS_INDPTR);
  const int32_t* pages = omni_attn_rows_get(r, OMNI_ATTN_ROWS_PAGES);
  CHECK(pos && slot && seq && indptr && pages);
  CHECK(pos[0] == 30 && pos[4] == 34 && pos[5] == 3);
  CHECK(slot[0] == 4 * 16 + 14 && slot[1] == 4 * 16 + 15 && slot[2] == 1 * 16 + 0 && slot[4] == 1 * 16 + 2);
  CHECK(slot[5] == 6 * 16 + 3);
  CHECK(seq[4] == 0 && seq[5] == 1);
  CHECK(indptr[0] == 0 && indptr[1] == 3 && indptr[2] == 4 && pages[3] == 6);
  CHECK(omni_attn_rows_get(r, 99) == NULL);
  /* a position past the lease */
  CHECK(omni_attn_rows_push(r, lease_b, 1, 15, 2, 2) == OMNI_ATTN_ETABLE);
  omni_attn_rows_clear(r);
  CHECK(omni_attn_rows_count(r, &rows, &seqs, &npages) == OMNI_ATTN_OK && rows == 0 && seqs == 0 && npages == 0);
  omni_attn_rows_free(r);
  /* the ring: position p uses the lease's slot of p % ring */
  omni_attn_rows* g = omni_attn_rows_new(16, 40);
  CHECK(g != NULL);
  CHECK(omni_attn_rows_push(g, lease_a, 3, 45, 1, 0) == OMNI_ATTN_OK);
  CHECK(omni_attn_rows_get(g, OMNI_ATTN_ROWS_SLOT)[0] == 9 * 16 + 5);
  omni_attn_rows_free(g);
  CHECK(omni_attn_rows_new(0, 0) == NULL);
  /* any positive page: slot of position p is lease[p / page] * page + p % page */
  omni_attn_rows* t12 = omni_attn_rows_new(12, 0);
  CHECK(t12 != NULL);
  CHECK(omni_attn_rows_push(t12, lease_a, 3, 25, 1, 0) == OMNI_ATTN_OK);
  CHECK(omni_attn_rows_get(t12, OMNI_ATTN_ROWS_SLOT)[0] == lease_a[2] * 12 + 1);
  omni_attn_rows_free(t12);
  CHECK(omni_attn_rows_new(16, -1) == NULL);
}

static void check_hidream_rows(void) {
  enum { kCausal = 5, kGr = 3, kGc = 4, kRows = 1 + kGr * kGc };
  int32_t tp[3 * kCausal], ts[kCausal], gp[3 * kRows], gs[kRows], kv = 0;
  CHECK(omni_hidream_rows(kCausal, kGr, kGc, 4096, tp, ts, gp, gs, &kv) == OMNI_ATTN_OK);
  CHECK(kv == kCausal + kRows);
  CHECK(tp[3 * 4] == 4 && tp[3 * 4 + 2] == 4 && ts[4] == 4);
  CHECK(gp[0] == kCausal && gp[1] == kCausal && gs[0] == kCausal);
  /* patch (i, j) = (2, 3) is generation row 1 + 2 * 4 + 3 */
  CHECK(gp[3 * 12] == 4096 && gp[3 * 12 + 1] == 4096 + 2 && gp[3 * 12 + 2] == 4096 + 3 && gs[12] == kCausal + 12);
  CHECK(omni_hidream_rows(0, kGr, kGc, 4096, NULL, NULL, NULL, NULL, NULL) == OMNI_ATTN_EINVAL);
  CHECK(omni_hidream_rows(kCausal, kGr, kGc, -1, NULL, NULL, NULL, NULL, NULL) == OMNI_ATTN_EINVAL);
}

static void check_head64_validation(void) {
  CHECK(omni_mimi_attend(kFake, kFake, kFake, kFake, kFake, 4, 0, 8, 0.1f, 100, 4096, NULL) == OMNI_ATTN_EINVAL);
  CHECK(omni_codec_attention(kFake, kFake, kFake, kFake, kFake, 4, 100, 16, 1e4f, NULL) == OMNI_ATTN_EINVAL);
  CHECK(omni_lm_dep_kv_attend(kFake, kFake, 8, kFake, 4, 16, 0.1f, NULL) == OMNI_ATTN_EINVAL);
  CHECK(omni_lm_rope(kFake, kFake, kFake, (void*)(uintptr_t)260, 4, 8, -0.1f, NULL) == OMNI_ATTN_EINVAL);
  CHECK(omni_qwen3_rope(kFake, kFake, kFake, kFake, kFake, kFake, 4, 16, 8, -1.0f, 1e6f, NULL) == OMNI_ATTN_EINVAL);
  CHECK(omni_qwen3_rope_dense(kFake, kFake, kFake, kFake, 4, 4, 14, 16, 16, 8, 1e-6f, 1e6f, NULL) ==
        OMNI_ATTN_EINVAL);
  CHECK(omni_hidream_qk_rope(kFake, 48 * 128, kFake, kFake, kFake, kFake, kFake, kFake, 4, 32, 8, 22, 1e-6f, 5e6f,
                             NULL) == OMNI_ATTN_EINVAL);
  CHECK(omni_attn_gather_kv(kFake, 8, kFake, kFake, 0, kFake, kFake, kFake, 2, kFake, NULL) == OMNI_ATTN_EINVAL);
  CHECK(omni_mimi_rope_kv(kFake, kFake, kFake, kFake, 4, 0, 8, -0.28f, 250, 64000, NULL) == OMNI_ATTN_EINVAL);
  CHECK(omni_mimi_rope_kv(kFake, kFake, kFake, kFake, 0, 2, 8, -0.28f, 250, 64000, NULL) == OMNI_ATTN_OK);
  CHECK(omni_lm_copy_kv(kFake, kFake, kFake, 3, 8440, NULL) == OMNI_ATTN_EINVAL);
  CHECK(omni_lm_copy_kv(NULL, NULL, NULL, 0, 8448, NULL) == OMNI_ATTN_OK);
  {
    omni_attn_decode_plan p;
    CHECK(omni_attn_decode_plan_init(4, 16, 8, 16, 600, 256, &p) == OMNI_ATTN_OK);
    /* bad eps; null slots; a head-group plan; a plan made for other heads */
    CHECK(omni_qwen3_rope_attend(kFake, kFake, kFake, kFake, kFake, kFake, kFake, kFake, 16, kFake, 16, 8, -1.0f,
                                 1e6f, 0.1f, &p, kFake, NULL) == OMNI_ATTN_EINVAL);
    CHECK(omni_qwen3_rope_attend(kFake, kFake, kFake, kFake, NULL, kFake, kFake, kFake, 16, kFake, 16, 8, 1e-6f,
                                 1e6f, 0.1f, &p, kFake, NULL) == OMNI_ATTN_EINVAL);
    p.group_heads = 2;
    CHECK(omni_qwen3_rope_attend(kFake, kFake, kFake, kFake, kFake, kFake, kFake, kFake, 16, kFake, 16, 8, 1e-6f,
                                 1e6f, 0.1f, &p, kFake, NULL) == OMNI_ATTN_EINVAL);
    p.group_heads = 0;
    CHECK(omni_qwen3_rope_attend(kFake, kFake, kFake, kFake, kFake, kFake, kFake, kFake, 16, kFake, 32, 8, 1e-6f,
                                 1e6f, 0.1f, &p, kFake, NULL) == OMNI_ATTN_EINVAL);
    CHECK(omni_attn_decode_plan_init(0, 16, 8, 16, 600, 256, &p) == OMNI_ATTN_OK);
    CHECK(omni_qwen3_rope_attend(NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, 16, NULL, 16, 8, 1e-6f, 1e6f, 0.1f,
                                 &p, NULL, NULL) == OMNI_ATTN_OK);
  }
  {
    omni_attn_decode_plan p;
    CHECK(omni_attn_decode_plan_init(4, 8, 8, 16, 600, 256, &p) == OMNI_ATTN_OK);
    /* context; null slots; coef; a plan for other heads */
    CHECK(omni_lm_rope_attend_fp8(kFake, kFake, kFake, kFake, kFake, kFake, 16, kFake, 8, -0.1f, 0.1f, 0, &p, kFake,
                                  NULL) == OMNI_ATTN_EINVAL);
    CHECK(omni_lm_rope_attend_fp8(kFake, kFake, NULL, kFake, kFake, kFake, 16, kFake, 8, -0.1f, 0.1f, 600, &p, kFake,
                                  NULL) == OMNI_ATTN_EINVAL);
    CHECK(omni_lm_rope_attend_fp8(kFake, kFake, kFake, kFake, kFake, kFake, 16, kFake, 8, NAN, 0.1f, 600, &p, kFake,
                                  NULL) == OMNI_ATTN_EINVAL);
    CHECK(omni_lm_rope_attend_fp8(kFake, kFake, kFake, kFake, kFake, kFake, 16, kFake, 16, -0.1f, 0.1f, 600, &p, kFake,
                                  NULL) == OMNI_ATTN_EINVAL);
  }
}

int main(void) {
  CHECK(omni_attn_version() >= 100);
  CHECK(omni_attn_last_error() != NULL);
  check_decode_plan();
  check_decode_run_validation();
  check_table();
  check_prefill_plan();
  check_dit_validation();
  check_rows();
  check_hidream_rows();
  check_head64_validation();
  printf("abi_check: %d checks passed\n", g_checks);
  return 0;
}
