/*
 * omni_attn — MI355X (gfx950) attention for the pega-omni engines, C ABI.
 *
 * Three kernels behind plan/run calls:
 *   - paged GQA / MHA decode (split-K, bandwidth-bound, no MFMA),
 *   - ragged causal chunked prefill over the same paged cache (bf16 MFMA),
 *   - HiDream-O1 DiT attention over dense K/V caches, causal or full (bf16 MFMA).
 *
 * Conventions for every entry point:
 *   - returns OMNI_ATTN_OK (0) or a negative OMNI_ATTN_E* code; nothing throws;
 *   - device pointers are plain `void*` / `int32_t*`; bf16 data is passed as
 *     `void*` (2-byte elements, head_dim 128);
 *   - `*_run` calls launch on `stream` (a hipStream_t, passed as void*), never
 *     allocate, never synchronise the host, and are safe to capture in a HIP
 *     graph: lengths are read from device arrays at run time;
 *   - `*_plan` calls are pure host code: they validate shapes and size the
 *     workspace; the caller owns and allocates the workspace. A run takes the
 *     plan its `*_plan_init` filled; a plan whose fields disagree with each
 *     other is refused (OMNI_ATTN_EINVAL) before anything is launched;
 *   - bf16 row buffers (qkv, q, k, v, kv, out) are 16-byte aligned (FP8 K/V
 *     slots 8-byte), and batch strides are multiples of 8 elements.
 *
 * Layouts are the reference's (paths in the pega-omni tree):
 *   qkv row n: [(hq + 2 hk)][128] bf16, q heads first (qwen3.cu:5-7, lm.cu:285);
 *   paged KV slot: [K heads | V heads][128] bf16 = 2 * hk * 256 bytes;
 *   token t of sequence s lives in slot pages[indptr[s] + t / page] * page + t % page
 *   (qwen3.cu:210-214); a row of sequence s at position pos sees tokens 0..pos;
 *   out row n: [hq][128] bf16.
 */
#ifndef OMNI_ATTN_H
#define OMNI_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OMNI_ATTN_OK 0
#define OMNI_ATTN_EINVAL (-1)       /* bad argument (null pointer, negative size) */
#define OMNI_ATTN_EUNSUPPORTED (-2) /* shape the kernels do not implement */
#define OMNI_ATTN_ELAUNCH (-3)      /* the HIP launch failed */
#define OMNI_ATTN_EWORKSPACE (-4)   /* workspace missing or too small */
#define OMNI_ATTN_ETABLE (-5)       /* page table / indptr failed host validation */

#define OMNI_ATTN_HEAD_DIM 128

/* ------------------------------------------------------------------ decode */

/* How a decode run partitions keys. Depends only on (rows, heads, page,
 * max_len), never on the lengths of one step, so one plan serves every replay
 * of a captured graph of the same batch bucket. */
typedef struct omni_attn_decode_plan {
  int32_t rows;     /* rows per launch (the batch bucket) */
  int32_t hq, hk;   /* query heads, K/V heads (hq % hk == 0, hq / hk in {1,2,4}, as the
                       reference's stack.rs:94-106 accepts) */
  int32_t page;     /* tokens per page, any positive size (16 in every engine) */
  int32_t max_len;  /* bound on keys any row sees; longer rows still run, slower */
  int32_t chunk;    /* keys per split (a multiple of 128) */
  int32_t splits;   /* ceil(max_len / chunk): workgroups per (row, kv head) */
  int32_t group_heads; /* MHA kernels (hq == hk): heads per workgroup dividing hk, 1/2/4/8
                          over FP8 slots, 1/2/4 over bf16 slots (paged rows); 0 (what
                          plan_init sets) picks from the shape */
  int64_t workspace_bytes; /* device scratch `*_run` needs (split partials) */
} omni_attn_decode_plan;

/* Fill `plan`. chunk_hint <= 0 picks the split size from the shape. */
int omni_attn_decode_plan_init(int rows, int hq, int hk, int page, int max_len, int chunk_hint,
                               omni_attn_decode_plan* plan);

/* The plan for lm_attend over its FP8 slots (omni_lm_attend_fp8 and
 * omni_lm_rope_attend_fp8; crates/omni-personaplex/kernels/lm.cu:273-290 has
 * no plan, its launch is fixed per bucket by crates/omni-personaplex/src/helium.rs:256-260):
 * the plan omni_attn_decode_plan_init makes with hq = hk = heads, except that
 * chunk_hint <= 0 picks the split size for the FP8 kernel's shape (up to 8
 * heads per workgroup): the largest of 1024 / 768 / 512 / 384 keys that still
 * gives 2048 workgroups of 8 heads, else 256. */
int omni_attn_decode_plan_init_fp8(int rows, int heads, int page, int max_len, int chunk_hint,
                                   omni_attn_decode_plan* plan);

/* Replaces `qwen3_attend` (crates/omni-qwen3/kernels/qwen3.cu:234-240): row n
 * of sequence s = ragged ? seq[n] : n attends to pos[n] + 1 keys. Arguments in
 * the reference's order, then the plan's rows, workspace and stream.
 * `seq` may be NULL when ragged == 0. */
int omni_qwen3_attend(const void* qkv, const void* kv, const int32_t* pos, const int32_t* seq, int ragged,
                      const int32_t* indptr, const int32_t* pages, int page, void* out, int hq, int hk, float scale,
                      const omni_attn_decode_plan* plan, void* workspace, void* stream);

/* omni_qwen3_attend without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, serving loops that forbid
 * hipMalloc); it has no counterpart in the reference. The split partials go to
 * a static 16 MiB device array the library holds on each GPU until the
 * process ends (OMNI_ATTN_NOALLOC_SCRATCH_BYTES); a plan whose
 * workspace_bytes exceeds it is rejected with OMNI_ATTN_EWORKSPACE. The call
 * allocates nothing. All calls on one GPU share the array: calls that overlap
 * on one GPU (concurrent streams) race. */
#define OMNI_ATTN_NOALLOC_SCRATCH_BYTES (16LL << 20)
int omni_qwen3_attend_noalloc(const void* qkv, const void* kv, const int32_t* pos, const int32_t* seq, int ragged,
                              const int32_t* indptr, const int32_t* pages, int page, void* out, int hq, int hk,
                              float scale, const omni_attn_decode_plan* plan, void* stream);

/* `lm_attend`'s semantics (crates/omni-personaplex/kernels/lm.cu:273-290) over
 * bf16 slots (the layout of attend.cuh's bf16 attend_row, attend.cuh:41-106):
 * MHA with `heads` query and K/V heads, qkv rows [3 heads][128], each row sees
 * min(pos[n] + 1, context) ring slots through its page table. */
int omni_lm_attend(const void* qkv, const void* kv, const int32_t* pos, const int32_t* seq, int ragged,
                   const int32_t* indptr, const int32_t* pages, int page, void* out, int heads, float scale,
                   int context, const omni_attn_decode_plan* plan, void* workspace, void* stream);

/* Replaces `lm_attend` itself (crates/omni-personaplex/kernels/lm.cu:273-290,
 * attend_row_fp8 at lm.cu:196-271), over its cache format: FP8 E4M3 slots of 2 * heads * 128 + 2 * heads * 4
 * bytes, [K heads x 128 B | V heads x 128 B | K scales f32 x heads | V scales
 * f32 x heads]; score = q . k * k_scale * scale, V weighted by p * v_scale.
 * Same arguments as omni_lm_attend; the plan is made with hq = hk = heads
 * (its group_heads may fix the heads per workgroup). */
int omni_lm_attend_fp8(const void* qkv, const void* kv, const int32_t* pos, const int32_t* seq, int ragged,
                       const int32_t* indptr, const int32_t* pages, int page, void* out, int heads, float scale,
                       int context, const omni_attn_decode_plan* plan, void* workspace, void* stream);

/* Same kernels with the FlashInfer-style length encoding the engines can also
 * produce: sequence s holds (indptr[s+1] - indptr[s] - 1) * page +
 * last_page_len[s] tokens, and row n (sequence ragged ? seq[n] : n) sees all
 * of them. qkv rows are [(hq + 2 hk)][128]. */
int omni_attn_decode_run_lastlen(const void* qkv, const void* kv, const int32_t* last_page_len, const int32_t* seq,
                                 int ragged, const int32_t* indptr, const int32_t* pages, int page, void* out, int hq,
                                 int hk, float scale, const omni_attn_decode_plan* plan, void* workspace,
                                 void* stream);

/* Replaces `qwen3_attend_dense` (crates/omni-qwen3/kernels/qwen3.cu:243-248),
 * the code predictor's attention over a dense workspace laid out as
 * omni_qwen3_rope_dense writes it: row n sees keys 0 .. base + n % per at slots
 * (n / per) * span + t of kv [slot][2 hk][128]. The plan is made with page = 1
 * and max_len >= base + per. */
int omni_qwen3_attend_dense(const void* qkv, const void* kv, int per, int base, int span, void* out, int hq, int hk,
                            float scale, const omni_attn_decode_plan* plan, void* workspace, void* stream);

/* ------------------------------------------------ head-64 ring attentions */

/* One workgroup of 64 per (row, head); rings are a few hundred keys at most.
 * Head dim 64; qkv rows [3 heads][64]; out rows [heads][64]. Per-session
 * state lives at state + lines[s] * stride bytes (16-byte aligned). */

/* Replaces `mimi_attend` (crates/omni-personaplex/kernels/mimi.cu:248-263):
 * row n of session s = n / T at position p = pos[s] * T + n % T sees
 * len = min(p + 1, context) ring slots (p - len + 1 + t) % context, slots
 * [2 heads][64] (K heads then V heads). */
int omni_mimi_attend(const void* qkv, const int32_t* pos, const int32_t* lines, const void* state, void* out, int rows,
                     int T, int heads, float scale, int context, int64_t stride, void* stream);

/* Replaces `mimi_rope_kv` (crates/omni-personaplex/kernels/mimi.cu:226-246), the
 * step before mimi_attend, same arguments (the reference's launch:
 * crates/omni-personaplex/src/mimi.rs:208-223): row n of session s = n / T at
 * p = pos[s] * T + n % T; its q heads are turned in place by the interleaved
 * rotary (pair (2i, 2i + 1) by p * exp(i * coef)), its k heads turned into ring
 * slot p % context (the slot's K heads) and its v heads copied there (the V
 * heads), each rotated value rounded to bf16. qkv rows [3 heads][64]. */
int omni_mimi_rope_kv(void* qkv, const int32_t* pos, const int32_t* lines, void* state, int rows, int T, int heads,
                      float coef, int context, int64_t stride, void* stream);

/* Replaces `codec_attention` (crates/omni-qwen3-tts/kernels/codec.cu:168-277):
 * for session r at p = pos[r], q and k turned by the half-split rotary
 * (pair i = dims i, i + 32, angle p * theta^(-2i/64)) and rounded to bf16; k
 * and v written to frame p % 72 of the session's ring K[72][heads * 64] then
 * V[72][heads * 64]; q attends to frames p - n + 1 .. p, n = min(p + 1, 72),
 * with scale 1/8. */
int omni_codec_attention(const void* qkv, const int32_t* pos, const int32_t* lines, void* kv, void* out, int rows,
                         int64_t stride, int heads, float theta, void* stream);

/* Replaces `lm_dep_kv_attend` (crates/omni-personaplex/kernels/lm.cu:314-366):
 * depformer step `step` (0..7) of session s writes its K and V into ws
 * [seqs][8][K | V][heads * 64] at that step and attends to steps 0 .. step. */
int omni_lm_dep_kv_attend(const void* qkv, void* ws, int step, void* out, int rows, int heads, float scale,
                          void* stream);

/* Replaces `lm_copy_kv` (crates/omni-personaplex/kernels/lm.cu:583-593; launched per
 * layer by crates/omni-personaplex/src/helium.rs:166-177 for prefix K/V reuse):
 * slot dst_slot[r] of one layer's cache takes the bytes of slot src_slot[r],
 * r < tokens; slot_bytes is a positive multiple of 16 (8448 for the FP8 cache).
 * A slot that is both a source and a destination of one call gives an
 * unspecified result, as in the reference. */
int omni_lm_copy_kv(void* kv, const int32_t* src_slot, const int32_t* dst_slot, int tokens, int slot_bytes,
                    void* stream);

/* ---------------------------------------------------------- page tables */

/* Host check of a page table before upload: indptr monotone from 0, every
 * page id in [0, num_pages), and every row's pos + 1 covered by its pages
 * (min(pos + 1, context) when context > 0). The manifest-domain checks of
 * crates/omni-qwen3-tts/src/model.rs:348-359, done once on the host. */
int omni_attn_check_table(const int32_t* indptr_h, int nseqs, const int32_t* pages_h, int num_pages,
                          const int32_t* pos_h, const int32_t* seq_h, int ragged, int rows, int page, int context);

/* Bit-exact gather of paged K/V to dense rows: for i < nseq and t < lens[i],
 * out[(out_indptr[i] + t)] = slot(seq_ids[i], t) of kv, 2 * hk * 128 bf16 each.
 * The paged addressing every kernel uses, exposed for verification. */
int omni_attn_gather_kv(const void* kv, int hk, const int32_t* indptr, const int32_t* pages, int page,
                        const int32_t* seq_ids, const int32_t* lens, const int32_t* out_indptr, int nseq, void* out,
                        void* stream);

/* ------------------------------------------------------- prefill (MFMA) */

/* Work list for a ragged causal prefill: rows of one sequence are contiguous
 * and at consecutive positions (how Rows::push_seq lays them out,
 * crates/omni-qwen3-tts/src/model.rs:278-289). */
typedef struct omni_attn_prefill_plan {
  int32_t rows, hq, hk, page;
  int32_t tiles;     /* query tiles (each runs once per kv head) */
  int32_t tile_rows; /* packed (position, head) rows per tile */
  int64_t work_bytes; /* bytes of the int32 work list the caller uploads */
  int32_t workgroups; /* grid of omni_attn_prefill_run */
  int32_t exact_p;    /* 0 (what plan_init sets): P rounded to bf16 for P.V, as the MFMA
                         flash kernels of the reference do (hidream.cu:317-324); 1: P carried
                         as two bf16 terms (hi + lo) through P.V, 16 significant bits, for
                         qwen3_attend(ragged = 1)'s f32 P (qwen3.cu:160-176) at about 1.4x
                         the time */
} omni_attn_prefill_plan;

/* Host: validate (seq_h, pos_h) for `rows` ragged rows and write the work list
 * into work_h (capacity work_cap int32): a header of 16 int32 whose entries
 * 0..8 bound the item ranges of the GPU's 8 XCDs, then 4 int32 per (tile, kv
 * head) item (sequence, first row, rows, kv head). Workgroup i runs item
 * header[i % 8] + i / 8. In workgroup order the tiles run by the keys they
 * see, most first, each with its hk kv heads, so every XCD ends on short
 * tiles and always sees the same kv heads (their K/V stays in its L2); the
 * XCD ranges differ by at most one item. Returns OMNI_ATTN_EWORKSPACE with plan->work_bytes set when
 * work_h is too small. */
int omni_attn_prefill_plan_init(int rows, int hq, int hk, int page, const int32_t* seq_h, const int32_t* pos_h,
                                int32_t* work_h, int64_t work_cap, omni_attn_prefill_plan* plan);

/* Ragged causal prefill with the semantics of qwen3_attend(ragged = 1): row n
 * sees keys 0..pos[n] of sequence seq[n] through the page table. `work` is
 * the device copy of the plan's work list. */
int omni_attn_prefill_run(const omni_attn_prefill_plan* plan, const void* qkv, const void* kv, const int32_t* pos,
                          const int32_t* seq, const int32_t* indptr, const int32_t* pages, void* out, float scale,
                          const int32_t* work, void* stream);

/* ---------------------------------------------------------- DiT (MFMA) */

/* Replaces `hidream_attend` (crates/omni-hidream-o1/kernels/hidream.cu:209-347).
 * q rows at q + n * q_stride + h * 128 (h < hq = G * hk), k and v [slots][hk][128],
 * out [q_len][hq][128]; row n sees the first *kv_len_at keys, with causal
 * only keys 0..n. A row that sees no key (*kv_len_at = 0) stores NaN, as the
 * reference's 1 / l does. The reference fixes G = 4 and hk = gridDim.y; here hq and hk
 * are arguments (G in {1,2,4,8}). When the last round of tiles would fill at
 * most half the GPU, its tiles run as two workgroups of half the rows each
 * (no workspace; each row is computed the same way). */
int omni_hidream_attend(const void* q, const void* k, const void* v, void* out, int q_len, const int32_t* kv_len_at,
                        int q_stride, int causal, float scale_log2, int hq, int hk, void* stream);

/* Batched form: `batch` independent problems (the CFG pair) at element strides
 * q_bstride, kv_bstride (k and v), out_bstride, sharing *kv_len_at. */
int omni_hidream_attend_batched(const void* q, const void* k, const void* v, void* out, int q_len,
                                const int32_t* kv_len_at, int q_stride, int causal, float scale_log2, int hq, int hk,
                                int batch, int64_t q_bstride, int64_t kv_bstride, int64_t out_bstride, void* stream);

/* ------------------------------------------ rotary embedding + K/V scatter */

/* The step before attention: rotary embedding of each new row's q (in place)
 * and k, and K and V written to the row's cache slot. One workgroup per (row,
 * 16 heads); `rows` is the launch size the reference gives as its grid. */

/* Replaces `qwen3_rope` (crates/omni-qwen3/kernels/qwen3.cu:64-103): per-head
 * RMSNorm of q and k (f32, x * rsqrt(mean(x^2) + eps) rounded to bf16, times
 * the bf16 weight), half-split rotary (pair i = elements i, i + 64, angle
 * pos * theta^(-2i/128)), q in place in qkv rows [(hq + 2 hk)][128], K and V
 * to slot `slots[n]` of the bf16 paged cache [slot][2 hk][128]. */
int omni_qwen3_rope(void* qkv, const void* q_norm, const void* k_norm, const int32_t* pos, const int32_t* slots,
                    void* kv, int rows, int hq, int hk, float eps, float theta, void* stream);

/* omni_qwen3_rope followed by omni_qwen3_attend on decode rows (ragged = 0:
 * row n is sequence n and attends to pos[n] + 1 keys), in one launch; it has
 * no counterpart in the reference, which runs the two as separate launches
 * (crates/omni-qwen3/src/stack.rs:222-240). The output and the K and V
 * written to slot slots[n] are bit-identical to the two calls'. Differences:
 * q is rotated in registers only (qkv is not written), and key pos[n] of row
 * n is taken from the rotated row, so slots[n] must be the slot the page
 * table gives key pos[n] (what the engines' Rows builder produces), and no
 * other row of the call may read slots[n]. The plan is a decode plan
 * (group_heads 0 or 1: the fused kernel runs one K/V head per workgroup, so
 * for MHA it matches omni_qwen3_attend with group_heads = 1 bit for bit). */
int omni_qwen3_rope_attend(const void* qkv, const void* q_norm, const void* k_norm, const int32_t* pos,
                           const int32_t* slots, void* kv, const int32_t* indptr, const int32_t* pages, int page,
                           void* out, int hq, int hk, float eps, float theta, float scale,
                           const omni_attn_decode_plan* plan, void* workspace, void* stream);

/* Replaces `qwen3_rope_dense` (qwen3.cu:105-111): `per` consecutive rows per
 * sequence at positions base, base + 1, ..., slot seq * span + pos of a dense
 * workspace (base + per <= span). */
int omni_qwen3_rope_dense(void* qkv, const void* q_norm, const void* k_norm, void* kv, int rows, int per, int base,
                          int span, int hq, int hk, float eps, float theta, void* stream);

/* Replaces `lm_rope` (crates/omni-personaplex/kernels/lm.cu:125-182):
 * interleaved rotary (pair i = elements 2i, 2i + 1, angle pos * exp(i * coef))
 * of q in place and of k, then K and V quantized to FP8 E4M3 (round to
 * nearest even) with per-(slot, head) scale max(amax / 448, 1e-12) into the
 * slot layout omni_lm_attend_fp8 reads. kv must be 8-byte aligned. */
int omni_lm_rope(void* qkv, const int32_t* pos, const int32_t* slots, void* kv, int rows, int heads, float coef,
                 void* stream);

/* omni_lm_rope followed by omni_lm_attend_fp8 on decode rows (ragged = 0: row n
 * is sequence n and attends to min(pos[n] + 1, context) ring slots), in one
 * launch; it has no counterpart in the reference, which runs the two as
 * separate launches (crates/omni-personaplex/src/helium.rs:242-275). The
 * output and the FP8 bytes and scales written to slot slots[n] are
 * bit-identical to the two calls'. Differences: q is rotated in registers only
 * (qkv is not written), and ring index pos[n] % context of row n is taken from
 * the rotated, quantized row, so slots[n] must be the slot the page table gives
 * that ring index (what the engines' Rows builder produces), and no other row
 * of the call may read slots[n]. The plan is the FP8 decode plan (hq = hk =
 * heads; its group_heads may fix the heads per workgroup). */
int omni_lm_rope_attend_fp8(const void* qkv, const int32_t* pos, const int32_t* slots, void* kv, const int32_t* indptr,
                            const int32_t* pages, int page, void* out, int heads, float coef, float scale, int context,
                            const omni_attn_decode_plan* plan, void* workspace, void* stream);

/* Replaces `hidream_qk_rope` (crates/omni-hidream-o1/kernels/hidream.cu:55-106):
 * RMSNorm as qwen3_rope, then Qwen3-VL's interleaved M-RoPE: row n has
 * positions (t, h, w) at positions[3n..3n+2]; pair i turns by the h position
 * when i % 3 == 1 and by w when i % 3 == 2, while i < 3 * mrope_hw, else by t.
 * q in place (rows of `ld` elements), K and V to slot `slots[n]` of the
 * separate caches [slots][hk][128]. */
int omni_hidream_qk_rope(void* qkv, int ld, const void* q_norm, const void* k_norm, const int32_t* positions,
                         const int32_t* slots, void* k_cache, void* v_cache, int rows, int hq, int hk, int mrope_hw,
                         float eps, float theta, void* stream);

/* The batched call with a workspace: the last fraction of a round of tiles
 * (tiles % resident workgroups) is split by keys into chunks that fill the
 * round, and a combine kernel merges the chunks (log-sum-exp). Same results
 * to rounding; workspace NULL runs as omni_hidream_attend_batched.
 * workspace_bytes must be at least omni_hidream_workspace_bytes() (16-byte
 * aligned); the split depends only on the shape and the device, never on
 * *kv_len_at. */
int omni_hidream_attend_ws(const void* q, const void* k, const void* v, void* out, int q_len, const int32_t* kv_len_at,
                           int q_stride, int causal, float scale_log2, int hq, int hk, int batch, int64_t q_bstride,
                           int64_t kv_bstride, int64_t out_bstride, void* workspace, int64_t workspace_bytes,
                           void* stream);

/* Workspace bytes omni_hidream_attend_ws needs at most on the current device. */
int64_t omni_hidream_workspace_bytes(void);

/* ------------------------------------------------------- host row builder */

/* The engines' `Rows` (crates/omni-qwen3-tts/src/model.rs:266-303,
 * crates/omni-personaplex/src/model.rs:472-499) in native host code: a step's
 * rows are pushed one sequence at a time with that sequence's lease (its page
 * ids) and a range of positions; the builder yields pos, slot, seq, indptr and
 * pages exactly as Rows::push_seq / Rows::push do. slot of position p is
 * page_ids[q / page] * page + q % page with q = p, or q = p % ring when ring > 0
 * (PersonaPlex's CONTEXT). Host memory only; the arrays are the inputs of the
 * omni_*_rope and omni_*_attend entry points once uploaded. */
typedef struct omni_attn_rows omni_attn_rows;

#define OMNI_ATTN_ROWS_POS 0
#define OMNI_ATTN_ROWS_SLOT 1
#define OMNI_ATTN_ROWS_SEQ 2
#define OMNI_ATTN_ROWS_INDPTR 3
#define OMNI_ATTN_ROWS_PAGES 4

/* NULL on a bad argument (omni_attn_last_error says which). */
omni_attn_rows* omni_attn_rows_new(int page, int ring);
void omni_attn_rows_free(omni_attn_rows* rows);
void omni_attn_rows_clear(omni_attn_rows* rows);
/* Rows first .. first + count - 1 of sequence `seq` with lease pages
 * page_ids[0 .. npages); OMNI_ATTN_ETABLE if a row's slot is not in the lease. */
int omni_attn_rows_push(omni_attn_rows* rows, const int32_t* page_ids, int npages, int first, int count, int seq);
int omni_attn_rows_count(const omni_attn_rows* rows, int* nrows, int* nseqs, int* npages);
/* One of the arrays (OMNI_ATTN_ROWS_*), valid until the next push / clear / free. */
const int32_t* omni_attn_rows_get(const omni_attn_rows* rows, int which);

/* Host: HiDream-O1's row arrays for hidream_qk_rope and hidream_attend
 * (crates/omni-hidream-o1/src/model.rs:123-160, prompt.rs:71-80). The prompt's
 * `causal` text rows: text_pos[k] = (k, k, k), text_slots[k] = k. The
 * generation rows, rows = 1 + grid_rows * grid_cols of them: the timestep slot
 * at text position `causal`, then the patches in raster order at
 * (image_position, image_position + i, image_position + j); gen_slots =
 * causal .. causal + rows - 1, and *step_kv = causal + rows keys. Positions
 * are [n][3] int32. Any output may be null. HiDream-O1's image_position is
 * 4096 (crates/omni-hidream-o1/src/config.rs:16). */
int omni_hidream_rows(int causal, int grid_rows, int grid_cols, int image_position, int32_t* text_pos,
                      int32_t* text_slots, int32_t* gen_pos, int32_t* gen_slots, int32_t* step_kv);

/* ------------------------------------------------------------- library */

/* Library version (major * 10000 + minor * 100 + patch). */
int omni_attn_version(void);

/* Text of the last error raised on this thread by any entry point ("" if none). */
const char* omni_attn_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* OMNI_ATTN_H */
