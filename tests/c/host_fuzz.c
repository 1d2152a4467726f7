/*
 * Seeded random and malformed inputs for the host-side planners and
 * validators of the C ABI (omni_attn_prefill_plan_init, omni_attn_check_table,
 * omni_attn_decode_plan_init, omni_attn_rows_*, omni_hidream_rows), built with
 * AddressSanitizer and UBSan (tests/c/Makefile, `make sanitize`). Every array
 * is allocated at exactly the size the call is told, so a read or write past
 * it is reported. Each accepted prefill plan is checked to cover every row
 * once per kv head. Exit 0 prints "host_fuzz: N cases".
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "omni_attn.h"

static uint64_t g_state = 0x243F6A8885A308D3ull;

static uint32_t rnd(void) {
  g_state = g_state * 6364136223846793005ull + 1442695040888963407ull;
  return (uint32_t)(g_state >> 33);
}

static int range(int lo, int hi) { return lo + (int)(rnd() % (uint32_t)(hi - lo + 1)); }

static void fail(const char* what, int iter) {
  fprintf(stderr, "host_fuzz: %s (case %d, last error \"%s\")\n", what, iter, omni_attn_last_error());
  exit(1);
}

/* Ragged rows: runs of consecutive positions, sometimes broken (a jump, a
 * repeated sequence, a negative position). */
static void fuzz_prefill(int iter) {
  const int rows = range(0, 700);
  const int G = 1 << range(0, 4);  /* 16 is rejected */
  const int hk = 1 << range(0, 3);
  const int page = range(0, 5) == 0 ? range(1, 40) : 1 << range(0, 6);
  int32_t* seq = (int32_t*)malloc(sizeof(int32_t) * (size_t)(rows ? rows : 1));
  int32_t* pos = (int32_t*)malloc(sizeof(int32_t) * (size_t)(rows ? rows : 1));
  int s = 0, p = range(0, 3000);
  int malformed = 0;
  for (int n = 0; n < rows; ++n) {
    if (range(0, 60) == 0) s = range(0, 9), p = range(0, 3000);
    if (range(0, 400) == 0) p = -range(1, 5), malformed = 1;
    seq[n] = s;
    pos[n] = p++;
  }
  omni_attn_prefill_plan plan;
  int rc = omni_attn_prefill_plan_init(rows, G * hk, hk, page, seq, pos, NULL, 0, &plan);
  const int shape_ok = G <= 8;
  if (!shape_ok) {
    if (rc != OMNI_ATTN_EUNSUPPORTED) fail("bad shape accepted", iter);
  } else if (malformed) {
    if (rc != OMNI_ATTN_ETABLE) fail("negative position accepted", iter);
  } else if (rc != OMNI_ATTN_EWORKSPACE) {
    fail("sizing call did not report the work list size", iter);
  }
  if (shape_ok && !malformed) {
    const int64_t cap = plan.work_bytes / 4;
    int32_t* work = (int32_t*)malloc((size_t)plan.work_bytes);
    rc = omni_attn_prefill_plan_init(rows, G * hk, hk, page, seq, pos, work, cap, &plan);
    if (rc != OMNI_ATTN_OK) fail("plan with the reported size failed", iter);
    const int items = plan.tiles * hk;
    if (work[8] != items) fail("header end", iter);
    int* hits = (int*)calloc((size_t)(rows ? rows : 1) * (size_t)hk, sizeof(int));
    for (int k = 0; k < items; ++k) {
      const int32_t* it = work + 16 + 4 * k;
      if (it[1] < 0 || it[2] < 1 || it[1] + it[2] > rows || it[3] < 0 || it[3] >= hk) fail("item range", iter);
      if (it[2] > 256 / G) fail("item larger than a tile", iter);
      for (int r = it[1]; r < it[1] + it[2]; ++r) {
        if (seq[r] != it[0]) fail("item spans two sequences", iter);
        if (r > it[1] && pos[r] != pos[r - 1] + 1) fail("item spans a position jump", iter);
        ++hits[(size_t)r * hk + it[3]];
      }
    }
    for (int i = 0; i < rows * hk; ++i)
      if (hits[i] != 1) fail("row not covered exactly once", iter);
    /* one int32 short of the list */
    if (cap > 0 && omni_attn_prefill_plan_init(rows, G * hk, hk, page, seq, pos, work, cap - 1, &plan) !=
                       OMNI_ATTN_EWORKSPACE)
      fail("short work list accepted", iter);
    free(hits);
    free(work);
  }
  free(seq);
  free(pos);
}

static void fuzz_table(int iter) {
  const int nseqs = range(0, 20), num_pages = range(1, 200), page = 1 << range(0, 5);
  int32_t* indptr = (int32_t*)malloc(sizeof(int32_t) * (size_t)(nseqs + 1));
  indptr[0] = range(0, 30) == 0 ? 1 : 0;
  for (int s = 0; s < nseqs; ++s) indptr[s + 1] = indptr[s] + (range(0, 40) == 0 ? -1 : range(0, 6));
  const int total = indptr[nseqs] > 0 ? indptr[nseqs] : 0;
  int32_t* pages = (int32_t*)malloc(sizeof(int32_t) * (size_t)(total ? total : 1));
  for (int i = 0; i < total; ++i) pages[i] = range(0, 100) == 0 ? num_pages : range(0, num_pages - 1);
  const int rows = range(0, 30), ragged = range(0, 1);
  int32_t* pos = (int32_t*)malloc(sizeof(int32_t) * (size_t)(rows ? rows : 1));
  int32_t* seq = (int32_t*)malloc(sizeof(int32_t) * (size_t)(rows ? rows : 1));
  for (int n = 0; n < rows; ++n) {
    pos[n] = range(-1, 6 * page);
    seq[n] = range(-1, nseqs);
  }
  const int mono = indptr[0] == 0;
  int monotone = mono;
  for (int s = 0; s < nseqs; ++s) monotone &= indptr[s + 1] >= indptr[s];
  /* a non-monotone indptr must be rejected before pages are read */
  const int rc = omni_attn_check_table(indptr, nseqs, monotone ? pages : NULL, num_pages, pos, seq, ragged,
                                       ragged || rows <= nseqs ? rows : nseqs, page, range(0, 1) ? 0 : 40);
  if (!monotone && rc != OMNI_ATTN_ETABLE) fail("bad indptr accepted", iter);
  if (rc != OMNI_ATTN_OK && rc != OMNI_ATTN_ETABLE) fail("unexpected code", iter);
  free(indptr);
  free(pages);
  free(pos);
  free(seq);
}

static void fuzz_rows(int iter) {
  const int page = range(0, 3) == 0 ? range(1, 40) : 1 << range(0, 5), ring = range(0, 1) ? 0 : range(1, 300);
  omni_attn_rows* r = omni_attn_rows_new(page, ring);
  if (!r) fail("rows_new", iter);
  int expect_rows = 0;
  for (int k = 0; k < range(0, 8); ++k) {
    const int npages = range(0, 12);
    int32_t* ids = (int32_t*)malloc(sizeof(int32_t) * (size_t)(npages ? npages : 1));
    for (int i = 0; i < npages; ++i) ids[i] = range(0, 50) == 0 ? -1 : range(0, 1000);
    const int first = range(0, 400), count = range(0, 40);
    const int rc = omni_attn_rows_push(r, npages ? ids : NULL, npages, first, count, k);
    if (rc == OMNI_ATTN_OK) expect_rows += count;
    else if (rc != OMNI_ATTN_ETABLE && rc != OMNI_ATTN_EINVAL) fail("rows_push code", iter);
    free(ids);
  }
  int rows = -1;
  omni_attn_rows_count(r, &rows, NULL, NULL);
  if (rows != expect_rows) fail("row count", iter);
  const int32_t* slot = omni_attn_rows_get(r, OMNI_ATTN_ROWS_SLOT);
  for (int n = 0; n < rows; ++n)
    if (slot[n] < 0) fail("negative slot", iter);
  omni_attn_rows_free(r);
}

static void fuzz_small(int iter) {
  omni_attn_decode_plan p;
  const int rc = omni_attn_decode_plan_init(range(-2, 70000), range(-1, 64), range(-1, 33), range(-1, 70),
                                            range(-5, 70000), range(-1, 3) * 128 + range(0, 1), &p);
  if (rc != OMNI_ATTN_OK && rc != OMNI_ATTN_EINVAL && rc != OMNI_ATTN_EUNSUPPORTED) fail("decode_plan code", iter);
  if (rc == OMNI_ATTN_OK && (p.splits < 1 || p.chunk % 128 != 0 || p.workspace_bytes < 0)) fail("decode plan", iter);
  const int causal = range(0, 40), gr = range(0, 20), gc = range(0, 20), rows = 1 + gr * gc;
  int32_t* tp = (int32_t*)malloc(sizeof(int32_t) * 3 * (size_t)(causal ? causal : 1));
  int32_t* ts = (int32_t*)malloc(sizeof(int32_t) * (size_t)(causal ? causal : 1));
  int32_t* gp = (int32_t*)malloc(sizeof(int32_t) * 3 * (size_t)rows);
  int32_t* gs = (int32_t*)malloc(sizeof(int32_t) * (size_t)rows);
  int32_t kv = 0;
  const int hr = omni_hidream_rows(causal, gr, gc, range(-1, 8192), tp, ts, gp, gs, &kv);
  if (hr == OMNI_ATTN_OK && kv != causal + rows) fail("hidream_rows kv", iter);
  free(tp);
  free(ts);
  free(gp);
  free(gs);
}

int main(void) {
  const int n = 3000;
  for (int i = 0; i < n; ++i) {
    fuzz_prefill(i);
    fuzz_table(i);
    fuzz_rows(i);
    fuzz_small(i);
  }
  printf("host_fuzz: %d cases\n", 4 * n);
  return 0;
}
