// The C ABI (include/omni_attn.h): host-side planning and validation, and the
// entry points the engines bind. Every function returns a status code; the
// text of the last failure is kept per thread for omni_attn_last_error().
#include "../../include/omni_attn.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <vector>

#include "kernels.h"

static_assert(OMNI_ATTN_NOALLOC_SCRATCH_BYTES == omni::kNoAllocScratchBytes, "static scratch size");

namespace {

thread_local char g_err[256] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = 0;
  return OMNI_ATTN_OK;
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// Split size for a decode bucket: the largest chunk (<= 1024 keys) that
// still gives the launch >= 4096 split workgroups at full length (16 per CU
// on 256 CUs), down to 256. Measured on MI355X over seven bucket shapes: a
// 128-session MHA tick (4096 row x head pairs) runs best at 1024, buckets of
// 128-512 pairs best at 256-384 (the 64-row GQA talker: 59.5 us at 256
// against 64.0 at 512), and 128-key splits were slower in every shape.
int pick_chunk(int rows, int hk, int max_len) {
  int chunk = 1024;
  while (chunk > 256) {
    const long long units = (long long)rows * hk * (((long long)max_len + chunk - 1) / chunk);
    if (units >= 4096) break;
    chunk /= 2;
  }
  return chunk;
}

// Split size for lm_attend over FP8 slots (decode_split_fp8, up to 8 heads per
// workgroup): the largest of 1024 / 768 / 512 / 384 keys that still gives
// >= 2048 workgroups of 8 heads at full length, else 256. Measured on MI355X
// (PersonaPlex rows, lengths U[100, 3000], 32 heads, us per call): 32 rows
// 99.7 / 87.9 / 84.9 / 79.7 / 79.7 at 1024 / 768 / 512 / 384 / 256; 64 rows
// 143.7 / 135.5 / 130.1 / 130.9 / 136.2; 128 rows 294.2 / 275.6 / 276.7 /
// 272.5 / 293.3; 256 rows 540.8 / 547.3 / 539.6 / 551.1 / 583.6. The bf16
// rule above (1024 for all but the 32-row bucket) is 0-10% slower here.
int pick_chunk_fp8(int rows, int heads, int max_len) {
  for (int chunk : {1024, 768, 512, 384}) {
    const long long wgs = (long long)rows * ((heads + 7) / 8) * (((long long)max_len + chunk - 1) / chunk);
    if (wgs >= 2048) return chunk;
  }
  return 256;
}

int decode_common(const void* qkv, const void* kv, const int32_t* pos, const int32_t* seq, int ragged,
                  const int32_t* indptr, const int32_t* pages, int page, void* out, int hq, int hk, float scale,
                  int context, int len_mode, const omni_attn_decode_plan* plan, void* workspace, void* stream,
                  int fp8 = 0, int dense_per = 0, int dense_base = 0, int dense_span = 0,
                  const omni::DecodeArgs* rope = nullptr) {
  if (!plan) return fail(OMNI_ATTN_EINVAL, "decode: null plan");
  if (plan->hq != hq || plan->hk != hk || plan->page != page)
    return fail(OMNI_ATTN_EINVAL, "decode: plan was made for hq=%d hk=%d page=%d, called with hq=%d hk=%d page=%d",
                plan->hq, plan->hk, plan->page, hq, hk, page);
  // The kernels size their grid and the split partials from the plan, so a
  // plan edited or built by hand must still be the one decode_plan_init
  // would have made for its (rows, max_len, chunk).
  if (plan->rows < 0 || plan->rows > 65535 || plan->max_len <= 0 || plan->chunk <= 0 || plan->chunk % 128 != 0 ||
      plan->splits != ((int64_t)plan->max_len + plan->chunk - 1) / plan->chunk ||
      (plan->splits > 1 &&
       plan->workspace_bytes < (int64_t)plan->rows * hq * plan->splits * (OMNI_ATTN_HEAD_DIM + 1) * (int64_t)sizeof(float)))
    return fail(OMNI_ATTN_EINVAL, "decode: plan is not self-consistent (rows=%d max_len=%d chunk=%d splits=%d workspace=%lld)",
                plan->rows, plan->max_len, plan->chunk, plan->splits, (long long)plan->workspace_bytes);
  if (plan->rows == 0) return ok();
  const bool dense = len_mode == 2;
  if (!qkv || !kv || !out || (!dense && (!pos || !indptr || !pages || (ragged && !seq))))
    return fail(OMNI_ATTN_EINVAL, "decode: null device pointer");
  if (((reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(out)) & 15) != 0 ||
      (reinterpret_cast<uintptr_t>(kv) & (fp8 ? 7 : 15)) != 0)
    return fail(OMNI_ATTN_EINVAL, "decode: qkv and out must be 16-byte aligned, kv %d-byte aligned", fp8 ? 8 : 16);
  if (plan->splits > 1 && (!workspace || plan->workspace_bytes <= 0))
    return fail(OMNI_ATTN_EWORKSPACE, "decode: plan needs %lld workspace bytes", (long long)plan->workspace_bytes);
  if (!std::isfinite(scale)) return fail(OMNI_ATTN_EINVAL, "decode: non-finite scale");
  const int gh = plan->group_heads;
  if (fp8 && gh != 0 && (gh < 0 || (gh & (gh - 1)) != 0 || gh > 8 || hk % gh != 0))
    return fail(OMNI_ATTN_EINVAL, "decode: plan group_heads=%d is not 1, 2, 4 or 8 dividing heads=%d", gh, hk);
  if (!fp8 && gh != 0 &&
      (len_mode == 2 || (gh != 1 && gh != 2 && gh != 4) || hk % gh != 0 || (hq / hk == 4 && gh == 4)))
    return fail(OMNI_ATTN_EINVAL,
                "decode: plan group_heads=%d: paged bf16 slots take 1, 2 or 4 dividing hk=%d (1 or 2 when hq = 4 hk)", gh,
                hk);
  omni::DecodeArgs a{};
  a.qkv = static_cast<const omni::bf16_t*>(qkv);
  a.q_stride = (int64_t)(hq + 2 * hk) * OMNI_ATTN_HEAD_DIM;
  a.kv = static_cast<const omni::bf16_t*>(kv);
  a.pos = pos;
  a.seq = seq;
  a.indptr = indptr;
  a.pages = pages;
  a.out = static_cast<omni::bf16_t*>(out);
  const int64_t o_floats = (int64_t)plan->rows * hq * plan->splits * OMNI_ATTN_HEAD_DIM;
  a.ws_o = static_cast<float*>(workspace);
  a.ws_lse = a.ws_o ? a.ws_o + o_floats : nullptr;
  a.hq = hq;
  a.hk = hk;
  a.ragged = ragged ? 1 : 0;
  a.pd = omni::make_page_div(page);
  a.context = context > 0 ? context : INT_MAX;
  a.len_mode = len_mode;
  a.chunk = plan->chunk;
  a.splits = plan->splits;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.fp8 = fp8;
  a.slot_bytes = 2LL * hk * OMNI_ATTN_HEAD_DIM + 2LL * hk * 4;
  a.group_heads = plan->group_heads;
  a.dense_per = dense_per;
  a.dense_base = dense_base;
  a.dense_span = dense_span;
  if (rope) {
    a.rope = 1;
    a.q_norm = rope->q_norm;
    a.k_norm = rope->k_norm;
    a.slots = rope->slots;
    a.kv_w = rope->kv_w;
    a.eps = rope->eps;
    a.theta = rope->theta;
    a.coef = rope->coef;
  }
  const int rc = omni::launch_decode(a, plan->rows, as_stream(stream));
  if (rc == -2)
    return fail(OMNI_ATTN_EUNSUPPORTED, "decode: hq/hk=%d and group_heads=%d not served, or the grid passes 2^31 "
                "workgroups", hq / hk, plan->group_heads);
  if (rc != 0) return fail(OMNI_ATTN_ELAUNCH, "decode: launch failed: %s", hipGetErrorString(omni::g_launch_status));
  return ok();
}

}  // namespace

extern "C" {

int omni_attn_version(void) { return 100; }

const char* omni_attn_last_error(void) { return g_err; }

static int decode_plan_fill(int rows, int hq, int hk, int page, int max_len, int chunk_hint, bool fp8,
                            omni_attn_decode_plan* plan) {
  if (!plan) return fail(OMNI_ATTN_EINVAL, "decode_plan: null plan");
  std::memset(plan, 0, sizeof *plan);
  if (rows < 0 || rows > 65535) return fail(OMNI_ATTN_EINVAL, "decode_plan: rows=%d outside [0, 65535]", rows);
  if (hk <= 0 || hq <= 0 || hq % hk != 0)
    return fail(OMNI_ATTN_EINVAL, "decode_plan: hq=%d is not a multiple of hk=%d", hq, hk);
  const int G = hq / hk;
  if (G != 1 && G != 2 && G != 4) return fail(OMNI_ATTN_EUNSUPPORTED, "decode_plan: hq/hk=%d not in {1,2,4}", G);
  if (page <= 0) return fail(OMNI_ATTN_EINVAL, "decode_plan: page=%d", page);
  if (max_len <= 0) return fail(OMNI_ATTN_EINVAL, "decode_plan: max_len=%d", max_len);
  int chunk = chunk_hint > 0 ? chunk_hint : fp8 ? pick_chunk_fp8(rows, hk, max_len) : pick_chunk(rows, hk, max_len);
  if (chunk % 128 != 0) return fail(OMNI_ATTN_EINVAL, "decode_plan: chunk=%d is not a multiple of 128", chunk);
  plan->rows = rows;
  plan->hq = hq;
  plan->hk = hk;
  plan->page = page;
  plan->max_len = max_len;
  plan->chunk = chunk;
  plan->splits = (int32_t)(((int64_t)max_len + chunk - 1) / chunk);
  plan->workspace_bytes =
      plan->splits > 1 ? (int64_t)rows * hq * plan->splits * (OMNI_ATTN_HEAD_DIM + 1) * (int64_t)sizeof(float) : 0;
  return ok();
}

int omni_attn_decode_plan_init(int rows, int hq, int hk, int page, int max_len, int chunk_hint,
                               omni_attn_decode_plan* plan) {
  return decode_plan_fill(rows, hq, hk, page, max_len, chunk_hint, false, plan);
}

int omni_attn_decode_plan_init_fp8(int rows, int heads, int page, int max_len, int chunk_hint,
                                   omni_attn_decode_plan* plan) {
  return decode_plan_fill(rows, heads, heads, page, max_len, chunk_hint, true, plan);
}

int omni_qwen3_attend(const void* qkv, const void* kv, const int32_t* pos, const int32_t* seq, int ragged,
                      const int32_t* indptr, const int32_t* pages, int page, void* out, int hq, int hk, float scale,
                      const omni_attn_decode_plan* plan, void* workspace, void* stream) {
  return decode_common(qkv, kv, pos, seq, ragged, indptr, pages, page, out, hq, hk, scale, 0, 0, plan, workspace,
                       stream);
}

int omni_qwen3_attend_noalloc(const void* qkv, const void* kv, const int32_t* pos, const int32_t* seq, int ragged,
                              const int32_t* indptr, const int32_t* pages, int page, void* out, int hq, int hk,
                              float scale, const omni_attn_decode_plan* plan, void* stream) {
  if (!plan) return fail(OMNI_ATTN_EINVAL, "qwen3_attend_noalloc: null plan");
  if (plan->workspace_bytes > omni::kNoAllocScratchBytes)
    return fail(OMNI_ATTN_EWORKSPACE,
                "qwen3_attend_noalloc: the plan needs %lld workspace bytes, above the %lld-byte static scratch "
                "(fewer rows per call, or omni_qwen3_attend with a workspace)",
                (long long)plan->workspace_bytes, (long long)omni::kNoAllocScratchBytes);
  float* ws = nullptr;
  if (plan->splits > 1 && plan->rows > 0 && omni::noalloc_scratch(&ws) != 0)
    return fail(OMNI_ATTN_ELAUNCH, "qwen3_attend_noalloc: no device address for the static scratch: %s",
                hipGetErrorString(omni::g_launch_status));
  return decode_common(qkv, kv, pos, seq, ragged, indptr, pages, page, out, hq, hk, scale, 0, 0, plan, ws, stream);
}

int omni_lm_attend(const void* qkv, const void* kv, const int32_t* pos, const int32_t* seq, int ragged,
                   const int32_t* indptr, const int32_t* pages, int page, void* out, int heads, float scale,
                   int context, const omni_attn_decode_plan* plan, void* workspace, void* stream) {
  if (context <= 0) return fail(OMNI_ATTN_EINVAL, "lm_attend: context=%d", context);
  return decode_common(qkv, kv, pos, seq, ragged, indptr, pages, page, out, heads, heads, scale, context, 0, plan,
                       workspace, stream);
}

int omni_lm_attend_fp8(const void* qkv, const void* kv, const int32_t* pos, const int32_t* seq, int ragged,
                       const int32_t* indptr, const int32_t* pages, int page, void* out, int heads, float scale,
                       int context, const omni_attn_decode_plan* plan, void* workspace, void* stream) {
  if (context <= 0) return fail(OMNI_ATTN_EINVAL, "lm_attend_fp8: context=%d", context);
  return decode_common(qkv, kv, pos, seq, ragged, indptr, pages, page, out, heads, heads, scale, context, 0, plan,
                       workspace, stream, 1);
}

int omni_attn_decode_run_lastlen(const void* qkv, const void* kv, const int32_t* last_page_len, const int32_t* seq,
                                 int ragged, const int32_t* indptr, const int32_t* pages, int page, void* out, int hq,
                                 int hk, float scale, const omni_attn_decode_plan* plan, void* workspace,
                                 void* stream) {
  return decode_common(qkv, kv, last_page_len, seq, ragged, indptr, pages, page, out, hq, hk, scale, 0, 1, plan,
                       workspace, stream);
}

int omni_attn_check_table(const int32_t* indptr_h, int nseqs, const int32_t* pages_h, int num_pages,
                          const int32_t* pos_h, const int32_t* seq_h, int ragged, int rows, int page, int context) {
  if (!indptr_h || nseqs < 0 || num_pages < 0 || rows < 0 || page <= 0)
    return fail(OMNI_ATTN_EINVAL, "check_table: bad arguments");
  if (indptr_h[0] != 0) return fail(OMNI_ATTN_ETABLE, "check_table: indptr[0]=%d, expected 0", indptr_h[0]);
  for (int s = 0; s < nseqs; ++s)
    if (indptr_h[s + 1] < indptr_h[s])
      return fail(OMNI_ATTN_ETABLE, "check_table: indptr not monotone at %d (%d > %d)", s, indptr_h[s],
                  indptr_h[s + 1]);
  if (pages_h) {
    for (int i = 0; i < indptr_h[nseqs]; ++i)
      if (pages_h[i] < 0 || pages_h[i] >= num_pages)
        return fail(OMNI_ATTN_ETABLE, "check_table: page id %d at %d outside [0, %d)", pages_h[i], i, num_pages);
  }
  if (pos_h) {
    for (int n = 0; n < rows; ++n) {
      const int s = ragged ? (seq_h ? seq_h[n] : -1) : n;
      if (s < 0 || s >= nseqs) return fail(OMNI_ATTN_ETABLE, "check_table: row %d names sequence %d", n, s);
      if (pos_h[n] < 0) return fail(OMNI_ATTN_ETABLE, "check_table: row %d at negative position %d", n, pos_h[n]);
      long long len = (long long)pos_h[n] + 1;
      if (context > 0 && len > context) len = context;
      const long long have = (long long)(indptr_h[s + 1] - indptr_h[s]) * page;
      if (len > have)
        return fail(OMNI_ATTN_ETABLE, "check_table: row %d needs %lld tokens, sequence %d has pages for %lld", n, len,
                    s, have);
    }
  }
  return ok();
}

int omni_attn_gather_kv(const void* kv, int hk, const int32_t* indptr, const int32_t* pages, int page,
                        const int32_t* seq_ids, const int32_t* lens, const int32_t* out_indptr, int nseq, void* out,
                        void* stream) {
  if (nseq < 0 || hk <= 0) return fail(OMNI_ATTN_EINVAL, "gather_kv: nseq=%d hk=%d", nseq, hk);
  if (nseq == 0) return ok();
  if (!kv || !indptr || !pages || !seq_ids || !lens || !out_indptr || !out)
    return fail(OMNI_ATTN_EINVAL, "gather_kv: null device pointer");
  if (page <= 0) return fail(OMNI_ATTN_EINVAL, "gather_kv: page=%d", page);
  if (omni::launch_gather_kv(kv, hk, indptr, pages, omni::make_page_div(page), seq_ids, lens, out_indptr, nseq, out,
                             as_stream(stream)) != 0)
    return fail(OMNI_ATTN_ELAUNCH, "gather_kv: launch failed: %s", hipGetErrorString(omni::g_launch_status));
  return ok();
}


int omni_attn_prefill_plan_init(int rows, int hq, int hk, int page, const int32_t* seq_h, const int32_t* pos_h,
                                int32_t* work_h, int64_t work_cap, omni_attn_prefill_plan* plan) {
  if (!plan) return fail(OMNI_ATTN_EINVAL, "prefill_plan: null plan");
  std::memset(plan, 0, sizeof *plan);
  if (rows < 0) return fail(OMNI_ATTN_EINVAL, "prefill_plan: rows=%d", rows);
  if (hk <= 0 || hq <= 0 || hq % hk != 0)
    return fail(OMNI_ATTN_EINVAL, "prefill_plan: hq=%d is not a multiple of hk=%d", hq, hk);
  const int G = hq / hk;
  if (G != 1 && G != 2 && G != 4 && G != 8)
    return fail(OMNI_ATTN_EUNSUPPORTED, "prefill_plan: hq/hk=%d not in {1,2,4,8}", G);
  if (page <= 0) return fail(OMNI_ATTN_EINVAL, "prefill_plan: page=%d", page);
  if (rows > 0 && (!seq_h || !pos_h)) return fail(OMNI_ATTN_EINVAL, "prefill_plan: null host arrays");
  const int per_tile = omni::kTiledRows / G;  // query positions per tile
  plan->rows = rows;
  plan->hq = hq;
  plan->hk = hk;
  plan->page = page;
  plan->tile_rows = omni::kTiledRows;
  // Runs of rows of one sequence at consecutive positions, cut into tiles:
  // (sequence, first row, rows, keys the last row sees).
  std::vector<std::array<int32_t, 4>> tl;
  for (int n = 0; n < rows;) {
    int e = n + 1;
    if (pos_h[n] < 0 || pos_h[n] == INT_MAX)
      return fail(OMNI_ATTN_ETABLE, "prefill_plan: row %d at position %d outside [0, INT_MAX)", n, pos_h[n]);
    if (seq_h[n] < 0) return fail(OMNI_ATTN_ETABLE, "prefill_plan: row %d names sequence %d", n, seq_h[n]);
    while (e < rows && seq_h[e] == seq_h[n] && (int64_t)pos_h[e] == (int64_t)pos_h[e - 1] + 1 && pos_h[e] != INT_MAX)
      ++e;
    for (int f = n; f < e; f += per_tile) {
      const int nq = (e - f) < per_tile ? (e - f) : per_tile;
      tl.push_back({seq_h[n], f, nq, pos_h[f + nq - 1] + 1});
    }
    n = e;
  }
  const int64_t tiles = (int64_t)tl.size();
  const int64_t items = tiles * hk;
  if (items > (INT_MAX - omni::kPrefillWorkHeader) / 4) return fail(OMNI_ATTN_EUNSUPPORTED, "prefill_plan: too many tiles");
  plan->tiles = (int32_t)tiles;
  const int64_t need = omni::kPrefillWorkHeader + 4 * items;
  plan->work_bytes = need * (int64_t)sizeof(int32_t);
  plan->workgroups = 0;
  plan->exact_p = 0;
  if (!work_h || need > work_cap)
    return fail(OMNI_ATTN_EWORKSPACE, "prefill_plan: work list needs %lld int32", (long long)need);
  // Item order: tiles by the keys they see, most first (a tile's time grows
  // with its key tiles, whatever its row count), each followed by its hk kv
  // heads. Workgroup i runs on XCD i % 8 and item k goes to XCD k % 8, so each
  // XCD's workgroups run longest first and the grid ends on short tiles; and
  // as hk is a power of two, an XCD always sees the same kv heads (h = x mod
  // hk for hk <= 8, h = x mod 8 beyond), so its L2 holds their K/V.
  std::stable_sort(tl.begin(), tl.end(), [](const auto& x, const auto& y) {
    if (x[3] != y[3]) return x[3] > y[3];
    if (x[0] != y[0]) return x[0] < y[0];
    return x[1] < y[1];
  });
  int32_t* hdr = work_h;
  for (int k = 0; k < omni::kPrefillWorkHeader; ++k) hdr[k] = 0;
  int32_t* body = work_h + omni::kPrefillWorkHeader;
  int64_t at = 0;
  for (int x = 0; x < omni::kXcds; ++x) {
    hdr[x] = (int32_t)at;
    for (int64_t k = x; k < items; k += omni::kXcds, ++at) {
      const auto& t = tl[k / hk];
      int32_t* it = body + 4 * at;
      it[0] = t[0];
      it[1] = t[1];
      it[2] = t[2];
      it[3] = (int32_t)(k % hk);
    }
  }
  hdr[omni::kXcds] = (int32_t)items;
  int32_t widest = 0;
  for (int x = 0; x < omni::kXcds; ++x) widest = std::max(widest, hdr[x + 1] - hdr[x]);
  plan->workgroups = widest * omni::kXcds;
  return ok();
}

int omni_attn_prefill_run(const omni_attn_prefill_plan* plan, const void* qkv, const void* kv, const int32_t* pos,
                          const int32_t* seq, const int32_t* indptr, const int32_t* pages, void* out, float scale,
                          const int32_t* work, void* stream) {
  if (!plan) return fail(OMNI_ATTN_EINVAL, "prefill_run: null plan");
  // The kernel's grid and item ranges come from the plan and the work list:
  // a plan whose fields disagree with each other would skip items silently.
  const int G = plan->hk > 0 && plan->hq > 0 && plan->hq % plan->hk == 0 ? plan->hq / plan->hk : 0;
  const int64_t items = (int64_t)plan->tiles * (plan->hk > 0 ? plan->hk : 0);
  if (plan->tiles < 0 || (G != 1 && G != 2 && G != 4 && G != 8) || plan->page <= 0 ||
      plan->tile_rows != omni::kTiledRows || plan->workgroups != (items + omni::kXcds - 1) / omni::kXcds * omni::kXcds ||
      plan->work_bytes != (omni::kPrefillWorkHeader + 4 * items) * (int64_t)sizeof(int32_t) ||
      (plan->exact_p != 0 && plan->exact_p != 1))
    return fail(OMNI_ATTN_EINVAL,
                "prefill_run: plan is not one prefill_plan_init made (tiles=%d hq=%d hk=%d page=%d tile_rows=%d "
                "workgroups=%d exact_p=%d)",
                plan->tiles, plan->hq, plan->hk, plan->page, plan->tile_rows, plan->workgroups, plan->exact_p);
  if (plan->tiles == 0) return ok();
  if (!qkv || !kv || !pos || !seq || !indptr || !pages || !out || !work)
    return fail(OMNI_ATTN_EINVAL, "prefill_run: null device pointer");
  if (((reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(kv) | reinterpret_cast<uintptr_t>(out)) & 15) != 0)
    return fail(OMNI_ATTN_EINVAL, "prefill_run: qkv, kv and out must be 16-byte aligned");
  omni::TiledArgs a{};
  a.q = static_cast<const omni::bf16_t*>(qkv);
  a.q_stride = (int64_t)(plan->hq + 2 * plan->hk) * OMNI_ATTN_HEAD_DIM;
  a.kv = static_cast<const omni::bf16_t*>(kv);
  a.pos = pos;
  a.seq = seq;
  a.indptr = indptr;
  a.pages = pages;
  a.work = work;
  a.pd = omni::make_page_div(plan->page);
  a.causal = 1;
  a.out = static_cast<omni::bf16_t*>(out);
  a.hq = plan->hq;
  a.hk = plan->hk;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.exact_p = plan->exact_p;
  const int rc = omni::launch_prefill(a, plan->workgroups, as_stream(stream));
  if (rc == -2) return fail(OMNI_ATTN_EUNSUPPORTED, "prefill_run: shape not implemented");
  if (rc != 0) return fail(OMNI_ATTN_ELAUNCH, "prefill_run: launch failed: %s", hipGetErrorString(omni::g_launch_status));
  return ok();
}

namespace {

// The DiT kernels move q, K, V and out rows in 16-byte pieces: every base and
// every batch stride (elements) must keep 16-byte alignment.
int dit_alignment(const void* q, const void* k, const void* v, const void* out, int batch, int64_t q_bstride,
                  int64_t kv_bstride, int64_t out_bstride) {
  const uintptr_t bits = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                         reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(out);
  if ((bits & 15) != 0) return fail(OMNI_ATTN_EINVAL, "hidream_attend: q, k, v and out must be 16-byte aligned");
  if (batch > 1 && (q_bstride < 0 || kv_bstride < 0 || out_bstride < 0 || q_bstride % 8 != 0 ||
                    kv_bstride % 8 != 0 || out_bstride % 8 != 0))
    return fail(OMNI_ATTN_EINVAL, "hidream_attend: batch strides %lld / %lld / %lld are not multiples of 8 elements",
                (long long)q_bstride, (long long)kv_bstride, (long long)out_bstride);
  return 0;
}

// Workgroups of the tiled kernel resident at once on the current device (one per CU).
int resident_tiled_groups() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return cus;
}

}  // namespace

}  // extern "C"

namespace {

// Validation and argument packing shared by the DiT entry points. Returns
// OMNI_ATTN_OK with `a` filled and `*empty` set when there is nothing to do.
int dit_prepare(const void* q, const void* k, const void* v, void* out, int q_len, const int32_t* kv_len_at,
                int q_stride, int causal, float scale_log2, int hq, int hk, int batch, int64_t q_bstride,
                int64_t kv_bstride, int64_t out_bstride, omni::TiledArgs* a, bool* empty) {
  *empty = false;
  if (q_len < 0 || batch < 0) return fail(OMNI_ATTN_EINVAL, "hidream_attend: q_len=%d batch=%d", q_len, batch);
  if (q_len == 0 || batch == 0) {
    *empty = true;
    return ok();
  }
  if (!q || !k || !v || !out || !kv_len_at) return fail(OMNI_ATTN_EINVAL, "hidream_attend: null device pointer");
  if (hk <= 0 || hq <= 0 || hq % hk != 0)
    return fail(OMNI_ATTN_EINVAL, "hidream_attend: hq=%d is not a multiple of hk=%d", hq, hk);
  const int G = hq / hk;
  if (G != 1 && G != 2 && G != 4 && G != 8)
    return fail(OMNI_ATTN_EUNSUPPORTED, "hidream_attend: hq/hk=%d not in {1,2,4,8}", G);
  if (q_stride < hq * OMNI_ATTN_HEAD_DIM || q_stride % 8 != 0)
    return fail(OMNI_ATTN_EINVAL, "hidream_attend: q_stride=%d", q_stride);
  if (batch > 65535) return fail(OMNI_ATTN_EUNSUPPORTED, "hidream_attend: batch=%d", batch);
  if (int rc = dit_alignment(q, k, v, out, batch, q_bstride, kv_bstride, out_bstride)) return rc;
  *a = omni::TiledArgs{};
  a->q = static_cast<const omni::bf16_t*>(q);
  a->q_stride = q_stride;
  a->k = static_cast<const omni::bf16_t*>(k);
  a->v = static_cast<const omni::bf16_t*>(v);
  a->kv_len_at = kv_len_at;
  a->q_len = q_len;
  a->causal = causal ? 1 : 0;
  a->q_bstride = q_bstride;
  a->kv_bstride = kv_bstride;
  a->out_bstride = out_bstride;
  a->out = static_cast<omni::bf16_t*>(out);
  a->hq = hq;
  a->hk = hk;
  a->scale_log2 = scale_log2;
  return ok();
}

int dit_launch(const omni::TiledArgs& a, int batch, void* stream) {
  const int rc = omni::launch_dit(a, batch, as_stream(stream));
  if (rc == -2) return fail(OMNI_ATTN_EUNSUPPORTED, "hidream_attend: shape not implemented");
  if (rc != 0)
    return fail(OMNI_ATTN_ELAUNCH, "hidream_attend: launch failed: %s", hipGetErrorString(omni::g_launch_status));
  return ok();
}

}  // namespace

extern "C" {

int omni_hidream_attend_batched(const void* q, const void* k, const void* v, void* out, int q_len,
                                const int32_t* kv_len_at, int q_stride, int causal, float scale_log2, int hq, int hk,
                                int batch, int64_t q_bstride, int64_t kv_bstride, int64_t out_bstride, void* stream) {
  omni::TiledArgs a;
  bool empty = false;
  if (int rc = dit_prepare(q, k, v, out, q_len, kv_len_at, q_stride, causal, scale_log2, hq, hk, batch, q_bstride,
                           kv_bstride, out_bstride, &a, &empty))
    return rc;
  if (empty) return ok();
  a.halved = omni::dit_halves(a, batch, resident_tiled_groups());
  return dit_launch(a, batch, stream);
}

int64_t omni_hidream_workspace_bytes(void) { return (int64_t)resident_tiled_groups() * omni::kSegmentBytes; }

int omni_hidream_attend_ws(const void* q, const void* k, const void* v, void* out, int q_len, const int32_t* kv_len_at,
                           int q_stride, int causal, float scale_log2, int hq, int hk, int batch, int64_t q_bstride,
                           int64_t kv_bstride, int64_t out_bstride, void* workspace, int64_t workspace_bytes,
                           void* stream) {
  if (!workspace)
    return omni_hidream_attend_batched(q, k, v, out, q_len, kv_len_at, q_stride, causal, scale_log2, hq, hk, batch,
                                       q_bstride, kv_bstride, out_bstride, stream);
  omni::TiledArgs a;
  bool empty = false;
  if (int rc = dit_prepare(q, k, v, out, q_len, kv_len_at, q_stride, causal, scale_log2, hq, hk, batch, q_bstride,
                           kv_bstride, out_bstride, &a, &empty))
    return rc;
  if (empty) return ok();
  if ((reinterpret_cast<uintptr_t>(workspace) & 15) != 0)
    return fail(OMNI_ATTN_EINVAL, "hidream_attend: workspace must be 16-byte aligned");
  int items = 0;
  omni::dit_split(a, batch, resident_tiled_groups(), &items, &a.split_from, &a.split_k);
  const int64_t need = (int64_t)(items - a.split_from) * a.split_k * omni::kSegmentBytes;
  if (need > workspace_bytes)
    return fail(OMNI_ATTN_EWORKSPACE, "hidream_attend: the split needs %lld workspace bytes, got %lld",
                (long long)need, (long long)workspace_bytes);
  a.ws = static_cast<float*>(workspace);
  return dit_launch(a, batch, stream);
}

int omni_hidream_attend(const void* q, const void* k, const void* v, void* out, int q_len, const int32_t* kv_len_at,
                        int q_stride, int causal, float scale_log2, int hq, int hk, void* stream) {
  return omni_hidream_attend_batched(q, k, v, out, q_len, kv_len_at, q_stride, causal, scale_log2, hq, hk, 1, 0, 0, 0,
                                     stream);
}

}  // extern "C"

// ------------------------------------------------------------------ rotary + scatter

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int rope_common(omni::RopeArgs& a, int mode, const char* who, void* stream) {
  if (a.rows < 0) return fail(OMNI_ATTN_EINVAL, "%s: rows=%d", who, a.rows);
  if (a.hq <= 0 || a.hk <= 0) return fail(OMNI_ATTN_EINVAL, "%s: hq=%d hk=%d", who, a.hq, a.hk);
  if ((int64_t)a.hq + 2LL * a.hk > 65535 * 16LL) return fail(OMNI_ATTN_EUNSUPPORTED, "%s: too many heads", who);
  if (a.rows == 0) return ok();
  if (!a.qkv || !aligned16(a.qkv)) return fail(OMNI_ATTN_EINVAL, "%s: qkv must be a 16-byte aligned device pointer", who);
  if (a.ld % 8 != 0) return fail(OMNI_ATTN_EINVAL, "%s: row stride %lld is not a multiple of 8", who, (long long)a.ld);
  const int rc = omni::launch_rope(a, mode, as_stream(stream));
  if (rc == -2) return fail(OMNI_ATTN_EUNSUPPORTED, "%s: mode not implemented", who);
  if (rc != 0) return fail(OMNI_ATTN_ELAUNCH, "%s: launch failed: %s", who, hipGetErrorString(omni::g_launch_status));
  return ok();
}

int norm_rope_checks(const void* q_norm, const void* k_norm, float eps, float theta, const char* who) {
  if (!q_norm || !k_norm || !aligned16(q_norm) || !aligned16(k_norm))
    return fail(OMNI_ATTN_EINVAL, "%s: q_norm / k_norm must be 16-byte aligned device pointers", who);
  if (!std::isfinite(eps) || eps < 0.f || !std::isfinite(theta) || theta <= 0.f)
    return fail(OMNI_ATTN_EINVAL, "%s: eps=%g theta=%g", who, (double)eps, (double)theta);
  return 0;
}

}  // namespace

int omni_qwen3_rope(void* qkv, const void* q_norm, const void* k_norm, const int32_t* pos, const int32_t* slots,
                    void* kv, int rows, int hq, int hk, float eps, float theta, void* stream) {
  if (rows > 0) {
    if (int rc = norm_rope_checks(q_norm, k_norm, eps, theta, "qwen3_rope")) return rc;
    if (!pos || !slots || !kv || !aligned16(kv)) return fail(OMNI_ATTN_EINVAL, "qwen3_rope: null or misaligned pointer");
  }
  omni::RopeArgs a{};
  a.qkv = static_cast<omni::bf16_t*>(qkv);
  a.ld = (int64_t)(hq + 2 * hk) * OMNI_ATTN_HEAD_DIM;
  a.q_norm = static_cast<const omni::bf16_t*>(q_norm);
  a.k_norm = static_cast<const omni::bf16_t*>(k_norm);
  a.pos = pos;
  a.slots = slots;
  a.kv = static_cast<omni::bf16_t*>(kv);
  a.rows = rows;
  a.hq = hq;
  a.hk = hk;
  a.eps = eps;
  a.theta = theta;
  return rope_common(a, omni::kRopeQwen3, "qwen3_rope", stream);
}

int omni_qwen3_rope_dense(void* qkv, const void* q_norm, const void* k_norm, void* kv, int rows, int per, int base,
                          int span, int hq, int hk, float eps, float theta, void* stream) {
  if (rows > 0) {
    if (int rc = norm_rope_checks(q_norm, k_norm, eps, theta, "qwen3_rope_dense")) return rc;
    if (!kv || !aligned16(kv)) return fail(OMNI_ATTN_EINVAL, "qwen3_rope_dense: null or misaligned kv");
    if (per <= 0 || base < 0 || (int64_t)base + per > span)
      return fail(OMNI_ATTN_EINVAL, "qwen3_rope_dense: per=%d base=%d span=%d (need base + per <= span)", per, base,
                  span);
  }
  omni::RopeArgs a{};
  a.qkv = static_cast<omni::bf16_t*>(qkv);
  a.ld = (int64_t)(hq + 2 * hk) * OMNI_ATTN_HEAD_DIM;
  a.q_norm = static_cast<const omni::bf16_t*>(q_norm);
  a.k_norm = static_cast<const omni::bf16_t*>(k_norm);
  a.kv = static_cast<omni::bf16_t*>(kv);
  a.rows = rows;
  a.hq = hq;
  a.hk = hk;
  a.per = per;
  a.base = base;
  a.span = span;
  a.eps = eps;
  a.theta = theta;
  return rope_common(a, omni::kRopeQwen3Dense, "qwen3_rope_dense", stream);
}

int omni_lm_rope(void* qkv, const int32_t* pos, const int32_t* slots, void* kv, int rows, int heads, float coef,
                 void* stream) {
  if (rows > 0) {
    if (!pos || !slots || !kv || (reinterpret_cast<uintptr_t>(kv) & 7) != 0)
      return fail(OMNI_ATTN_EINVAL, "lm_rope: null pointer or kv not 8-byte aligned");
    if (!std::isfinite(coef)) return fail(OMNI_ATTN_EINVAL, "lm_rope: non-finite coef");
  }
  omni::RopeArgs a{};
  a.qkv = static_cast<omni::bf16_t*>(qkv);
  a.ld = 3LL * heads * OMNI_ATTN_HEAD_DIM;
  a.pos = pos;
  a.slots = slots;
  a.kv_bytes = kv;
  a.slot_bytes = 2LL * heads * OMNI_ATTN_HEAD_DIM + 2LL * heads * 4;
  a.rows = rows;
  a.hq = heads;
  a.hk = heads;
  a.coef = coef;
  return rope_common(a, omni::kRopeLm, "lm_rope", stream);
}

int omni_hidream_qk_rope(void* qkv, int ld, const void* q_norm, const void* k_norm, const int32_t* positions,
                         const int32_t* slots, void* k_cache, void* v_cache, int rows, int hq, int hk, int mrope_hw,
                         float eps, float theta, void* stream) {
  if (rows > 0) {
    if (int rc = norm_rope_checks(q_norm, k_norm, eps, theta, "hidream_qk_rope")) return rc;
    if (!positions || !slots || !k_cache || !v_cache || !aligned16(k_cache) || !aligned16(v_cache))
      return fail(OMNI_ATTN_EINVAL, "hidream_qk_rope: null or misaligned pointer");
    if ((int64_t)ld < (int64_t)(hq + 2 * hk) * OMNI_ATTN_HEAD_DIM)
      return fail(OMNI_ATTN_EINVAL, "hidream_qk_rope: ld=%d shorter than a [q | k | v] row", ld);
    if (mrope_hw < 0 || 3 * mrope_hw > OMNI_ATTN_HEAD_DIM / 2)
      return fail(OMNI_ATTN_EINVAL, "hidream_qk_rope: mrope_hw=%d outside [0, 21]", mrope_hw);
  }
  omni::RopeArgs a{};
  a.qkv = static_cast<omni::bf16_t*>(qkv);
  a.ld = ld;
  a.q_norm = static_cast<const omni::bf16_t*>(q_norm);
  a.k_norm = static_cast<const omni::bf16_t*>(k_norm);
  a.pos = positions;
  a.slots = slots;
  a.k_cache = static_cast<omni::bf16_t*>(k_cache);
  a.v_cache = static_cast<omni::bf16_t*>(v_cache);
  a.rows = rows;
  a.hq = hq;
  a.hk = hk;
  a.mrope_hw = mrope_hw;
  a.eps = eps;
  a.theta = theta;
  return rope_common(a, omni::kRopeHidream, "hidream_qk_rope", stream);
}

int omni_qwen3_rope_attend(const void* qkv, const void* q_norm, const void* k_norm, const int32_t* pos,
                           const int32_t* slots, void* kv, const int32_t* indptr, const int32_t* pages, int page,
                           void* out, int hq, int hk, float eps, float theta, float scale,
                           const omni_attn_decode_plan* plan, void* workspace, void* stream) {
  if (plan && plan->rows > 0) {
    if (int rc = norm_rope_checks(q_norm, k_norm, eps, theta, "qwen3_rope_attend")) return rc;
    if (!slots) return fail(OMNI_ATTN_EINVAL, "qwen3_rope_attend: null slots");
    if (plan->group_heads > 1)
      return fail(OMNI_ATTN_EINVAL, "qwen3_rope_attend: plan group_heads=%d (the fused kernel takes one K/V head per "
                  "workgroup: 0 or 1)", plan->group_heads);
  }
  omni::DecodeArgs r{};
  r.q_norm = static_cast<const omni::bf16_t*>(q_norm);
  r.k_norm = static_cast<const omni::bf16_t*>(k_norm);
  r.slots = slots;
  r.kv_w = static_cast<omni::bf16_t*>(kv);
  r.eps = eps;
  r.theta = theta;
  return decode_common(qkv, kv, pos, nullptr, 0, indptr, pages, page, out, hq, hk, scale, 0, 0, plan, workspace,
                       stream, 0, 0, 0, 0, &r);
}

int omni_lm_rope_attend_fp8(const void* qkv, const int32_t* pos, const int32_t* slots, void* kv, const int32_t* indptr,
                            const int32_t* pages, int page, void* out, int heads, float coef, float scale, int context,
                            const omni_attn_decode_plan* plan, void* workspace, void* stream) {
  if (context <= 0) return fail(OMNI_ATTN_EINVAL, "lm_rope_attend_fp8: context=%d", context);
  if (plan && plan->rows > 0) {
    if (!slots) return fail(OMNI_ATTN_EINVAL, "lm_rope_attend_fp8: null slots");
    if (!std::isfinite(coef)) return fail(OMNI_ATTN_EINVAL, "lm_rope_attend_fp8: non-finite coef");
  }
  omni::DecodeArgs r{};
  r.slots = slots;
  r.kv_w = static_cast<omni::bf16_t*>(kv);
  r.coef = coef;
  return decode_common(qkv, kv, pos, nullptr, 0, indptr, pages, page, out, heads, heads, scale, context, 0, plan,
                       workspace, stream, 1, 0, 0, 0, &r);
}

int omni_qwen3_attend_dense(const void* qkv, const void* kv, int per, int base, int span, void* out, int hq, int hk,
                            float scale, const omni_attn_decode_plan* plan, void* workspace, void* stream) {
  if (per <= 0 || base < 0 || (int64_t)base + per > span)
    return fail(OMNI_ATTN_EINVAL, "qwen3_attend_dense: per=%d base=%d span=%d (need base + per <= span)", per, base,
                span);
  if (plan && plan->max_len < base + per)
    return fail(OMNI_ATTN_EINVAL, "qwen3_attend_dense: plan max_len=%d below base + per=%d", plan->max_len, base + per);
  return decode_common(qkv, kv, nullptr, nullptr, 0, nullptr, nullptr, 1, out, hq, hk, scale, 0, 2, plan, workspace,
                       stream, 0, per, base, span);
}

// ------------------------------------------------------ head-64 ring attentions

namespace {

int short_common(omni::ShortArgs& a, int kind, const char* who, void* stream) {
  if (a.rows < 0 || a.heads <= 0) return fail(OMNI_ATTN_EINVAL, "%s: rows=%d heads=%d", who, a.rows, a.heads);
  if (a.heads > 65535) return fail(OMNI_ATTN_EUNSUPPORTED, "%s: heads=%d", who, a.heads);
  if (a.rows == 0) return ok();
  if (!a.qkv || !a.out || !aligned16(a.qkv) || !aligned16(a.out))
    return fail(OMNI_ATTN_EINVAL, "%s: qkv / out must be 16-byte aligned device pointers", who);
  const int rc = omni::launch_short(a, kind, as_stream(stream));
  if (rc != 0) return fail(OMNI_ATTN_ELAUNCH, "%s: launch failed: %s", who, hipGetErrorString(omni::g_launch_status));
  return ok();
}

}  // namespace

int omni_mimi_attend(const void* qkv, const int32_t* pos, const int32_t* lines, const void* state, void* out, int rows,
                     int T, int heads, float scale, int context, int64_t stride, void* stream) {
  if (rows > 0) {
    if (!pos || !lines || !state || !aligned16(state)) return fail(OMNI_ATTN_EINVAL, "mimi_attend: null pointer");
    if (T <= 0 || context <= 0 || stride % 16 != 0 || !std::isfinite(scale))
      return fail(OMNI_ATTN_EINVAL, "mimi_attend: T=%d context=%d stride=%lld", T, context, (long long)stride);
  }
  omni::ShortArgs a{};
  a.qkv = static_cast<const omni::bf16_t*>(qkv);
  a.pos = pos;
  a.lines = lines;
  a.state = const_cast<void*>(state);
  a.stride = stride;
  a.out = static_cast<omni::bf16_t*>(out);
  a.rows = rows;
  a.heads = heads;
  a.T = T;
  a.context = context;
  a.scale = scale;
  return short_common(a, omni::kShortMimi, "mimi_attend", stream);
}

int omni_mimi_rope_kv(void* qkv, const int32_t* pos, const int32_t* lines, void* state, int rows, int T, int heads,
                      float coef, int context, int64_t stride, void* stream) {
  if (rows < 0 || heads <= 0) return fail(OMNI_ATTN_EINVAL, "mimi_rope_kv: rows=%d heads=%d", rows, heads);
  if (rows == 0) return ok();
  if (!qkv || !pos || !lines || !state || !aligned16(qkv) || !aligned16(state))
    return fail(OMNI_ATTN_EINVAL, "mimi_rope_kv: qkv and state must be 16-byte aligned device pointers");
  if (T <= 0 || context <= 0 || stride % 16 != 0 || !std::isfinite(coef) || heads > 4096)
    return fail(OMNI_ATTN_EINVAL, "mimi_rope_kv: T=%d context=%d stride=%lld heads=%d", T, context, (long long)stride,
                heads);
  omni::ShortArgs a{};
  a.qkv_rw = static_cast<omni::bf16_t*>(qkv);
  a.pos = pos;
  a.lines = lines;
  a.state = state;
  a.stride = stride;
  a.rows = rows;
  a.heads = heads;
  a.T = T;
  a.context = context;
  a.coef = coef;
  if (omni::launch_short(a, omni::kShortMimiRope, as_stream(stream)) != 0)
    return fail(OMNI_ATTN_ELAUNCH, "mimi_rope_kv: launch failed: %s", hipGetErrorString(omni::g_launch_status));
  return ok();
}

int omni_lm_copy_kv(void* kv, const int32_t* src_slot, const int32_t* dst_slot, int tokens, int slot_bytes,
                    void* stream) {
  if (tokens < 0 || slot_bytes <= 0 || slot_bytes % 16 != 0)
    return fail(OMNI_ATTN_EINVAL, "lm_copy_kv: tokens=%d slot_bytes=%d (a positive multiple of 16)", tokens,
                slot_bytes);
  if (tokens == 0) return ok();
  if (!kv || !src_slot || !dst_slot || !aligned16(kv))
    return fail(OMNI_ATTN_EINVAL, "lm_copy_kv: kv must be a 16-byte aligned device pointer");
  if (omni::launch_copy_slots(kv, src_slot, dst_slot, tokens, slot_bytes, as_stream(stream)) != 0)
    return fail(OMNI_ATTN_ELAUNCH, "lm_copy_kv: launch failed: %s", hipGetErrorString(omni::g_launch_status));
  return ok();
}

int omni_codec_attention(const void* qkv, const int32_t* pos, const int32_t* lines, void* kv, void* out, int rows,
                         int64_t stride, int heads, float theta, void* stream) {
  if (rows > 0) {
    if (!pos || !lines || !kv || !aligned16(kv)) return fail(OMNI_ATTN_EINVAL, "codec_attention: null pointer");
    if (stride % 16 != 0 || !std::isfinite(theta) || theta <= 0.f)
      return fail(OMNI_ATTN_EINVAL, "codec_attention: stride=%lld theta=%g", (long long)stride, (double)theta);
  }
  omni::ShortArgs a{};
  a.qkv = static_cast<const omni::bf16_t*>(qkv);
  a.pos = pos;
  a.lines = lines;
  a.state = kv;
  a.stride = stride;
  a.out = static_cast<omni::bf16_t*>(out);
  a.rows = rows;
  a.heads = heads;
  a.theta = theta;
  return short_common(a, omni::kShortCodec, "codec_attention", stream);
}

int omni_lm_dep_kv_attend(const void* qkv, void* ws, int step, void* out, int rows, int heads, float scale,
                          void* stream) {
  if (rows > 0) {
    if (!ws || !aligned16(ws)) return fail(OMNI_ATTN_EINVAL, "lm_dep_kv_attend: null or misaligned ws");
    if (step < 0 || step >= 8 || !std::isfinite(scale))
      return fail(OMNI_ATTN_EINVAL, "lm_dep_kv_attend: step=%d outside [0, 8)", step);
  }
  omni::ShortArgs a{};
  a.qkv = static_cast<const omni::bf16_t*>(qkv);
  a.ws = static_cast<omni::bf16_t*>(ws);
  a.out = static_cast<omni::bf16_t*>(out);
  a.rows = rows;
  a.heads = heads;
  a.step = step;
  a.scale = scale;
  return short_common(a, omni::kShortDep, "lm_dep_kv_attend", stream);
}

// ----------------------------------------------------------- host row builder

struct omni_attn_rows {
  int page;
  int ring;  // > 0: slot of position p is the lease's slot of p % ring (PersonaPlex)
  std::vector<int32_t> pos, slot, seq, indptr, pages;
};

omni_attn_rows* omni_attn_rows_new(int page, int ring) {
  if (page <= 0 || ring < 0) {
    fail(OMNI_ATTN_EINVAL, "rows_new: page=%d ring=%d", page, ring);
    return nullptr;
  }
  omni_attn_rows* r = new (std::nothrow) omni_attn_rows();
  if (!r) {
    fail(OMNI_ATTN_EINVAL, "rows_new: out of memory");
    return nullptr;
  }
  r->page = page;
  r->ring = ring;
  ok();
  return r;
}

void omni_attn_rows_free(omni_attn_rows* r) { delete r; }

void omni_attn_rows_clear(omni_attn_rows* r) {
  if (!r) return;
  r->pos.clear();
  r->slot.clear();
  r->seq.clear();
  r->indptr.clear();
  r->pages.clear();
}

int omni_attn_rows_push(omni_attn_rows* r, const int32_t* page_ids, int npages, int first, int count, int seq) {
  if (!r || (npages > 0 && !page_ids) || npages < 0 || first < 0 || count < 0 || seq < 0)
    return fail(OMNI_ATTN_EINVAL, "rows_push: npages=%d first=%d count=%d seq=%d", npages, first, count, seq);
  for (int i = 0; i < npages; ++i)
    if (page_ids[i] < 0) return fail(OMNI_ATTN_ETABLE, "rows_push: page id %d at %d", page_ids[i], i);
  // Every row's slot must lie in the lease.
  const int64_t last = count > 0 ? (int64_t)first + count - 1 : -1;
  const int64_t reach = r->ring > 0 ? std::min<int64_t>(last, r->ring - 1) : last;
  if (last > INT32_MAX) return fail(OMNI_ATTN_EINVAL, "rows_push: position %lld past int32", (long long)last);
  if (count > 0 && reach / r->page >= npages)
    return fail(OMNI_ATTN_ETABLE, "rows_push: position %lld needs page %lld of a %d-page lease", (long long)last,
                (long long)(reach / r->page), npages);
  if (r->pos.size() + (size_t)count > (size_t)INT32_MAX || r->pages.size() + (size_t)npages > (size_t)INT32_MAX)
    return fail(OMNI_ATTN_EINVAL, "rows_push: too many rows or pages");
  for (int i = 0; i < npages; ++i)
    if ((int64_t)page_ids[i] * r->page + r->page - 1 > INT32_MAX)
      return fail(OMNI_ATTN_ETABLE, "rows_push: page id %d puts slots past int32", page_ids[i]);
  if (r->indptr.empty()) r->indptr.push_back(0);
  for (int i = 0; i < count; ++i) {
    const int64_t p = (int64_t)first + i;
    const int64_t q = r->ring > 0 ? p % r->ring : p;
    r->pos.push_back((int32_t)p);
    r->slot.push_back((int32_t)((int64_t)page_ids[q / r->page] * r->page + q % r->page));
    r->seq.push_back(seq);
  }
  r->pages.insert(r->pages.end(), page_ids, page_ids + npages);
  r->indptr.push_back((int32_t)r->pages.size());
  return ok();
}

int omni_attn_rows_count(const omni_attn_rows* r, int* rows, int* nseqs, int* npages) {
  if (!r) return fail(OMNI_ATTN_EINVAL, "rows_count: null builder");
  if (rows) *rows = (int)r->pos.size();
  if (nseqs) *nseqs = r->indptr.empty() ? 0 : (int)r->indptr.size() - 1;
  if (npages) *npages = (int)r->pages.size();
  return ok();
}

int omni_hidream_rows(int causal, int grid_rows, int grid_cols, int image_position, int32_t* text_pos,
                      int32_t* text_slots, int32_t* gen_pos, int32_t* gen_slots, int32_t* step_kv) {
  if (causal < 1 || grid_rows < 1 || grid_cols < 1)
    return fail(OMNI_ATTN_EINVAL, "hidream_rows: causal=%d grid=%dx%d", causal, grid_rows, grid_cols);
  const int64_t patches = (int64_t)grid_rows * grid_cols, rows = 1 + patches;
  if (causal + rows > INT_MAX || (int64_t)image_position + std::max(grid_rows, grid_cols) > INT_MAX ||
      image_position < 0)
    return fail(OMNI_ATTN_EINVAL, "hidream_rows: positions or slots overflow int32");
  for (int k = 0; k < causal; ++k) {
    if (text_pos) text_pos[3 * k] = text_pos[3 * k + 1] = text_pos[3 * k + 2] = k;
    if (text_slots) text_slots[k] = k;
  }
  if (gen_pos) {
    gen_pos[0] = gen_pos[1] = gen_pos[2] = causal;  // the timestep slot at the last text position
    int64_t n = 1;
    for (int i = 0; i < grid_rows; ++i)
      for (int j = 0; j < grid_cols; ++j, ++n) {
        gen_pos[3 * n] = image_position;
        gen_pos[3 * n + 1] = image_position + i;
        gen_pos[3 * n + 2] = image_position + j;
      }
  }
  if (gen_slots)
    for (int64_t n = 0; n < rows; ++n) gen_slots[n] = (int32_t)(causal + n);
  if (step_kv) *step_kv = (int32_t)(causal + rows);
  return ok();
}

const int32_t* omni_attn_rows_get(const omni_attn_rows* r, int which) {
  if (!r) return nullptr;
  switch (which) {
    case OMNI_ATTN_ROWS_POS: return r->pos.data();
    case OMNI_ATTN_ROWS_SLOT: return r->slot.data();
    case OMNI_ATTN_ROWS_SEQ: return r->seq.data();
    case OMNI_ATTN_ROWS_INDPTR: return r->indptr.data();
    case OMNI_ATTN_ROWS_PAGES: return r->pages.data();
    default: return nullptr;
  }
}
