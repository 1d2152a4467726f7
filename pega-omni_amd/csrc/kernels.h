// Launch interface between the C ABI (capi.cpp) and the HIP kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "indexing.h"

namespace omni {

typedef uint16_t bf16_t;

// The HIP status of this thread's last launch, kept for error messages.
inline thread_local hipError_t g_launch_status = hipSuccess;
inline int check_launch() {
  g_launch_status = hipGetLastError();
  return g_launch_status == hipSuccess ? 0 : -3;
}

// Everything a decode launch reads; passed by value as the kernel argument.
struct DecodeArgs {
  const bf16_t* qkv;
  int64_t q_stride;  // elements between consecutive qkv rows
  const bf16_t* kv;
  const int32_t* pos;  // len_mode 0: per-row positions; 1: per-sequence last page lengths
  const int32_t* seq;
  const int32_t* indptr;
  const int32_t* pages;
  bf16_t* out;
  float* ws_o;   // [rows][hq][splits][128] split outputs (normalised)
  float* ws_lse; // [rows][hq][splits] split log2-sum-exp
  int hq, hk;
  int ragged;
  PageDiv pd;   // page size and its divisor
  int context;  // cap on keys per row
  int len_mode;
  int chunk, splits;
  float scale_log2;  // softmax scale times log2(e)
  int fp8;           // 1: kv slots are FP8 E4M3 with f32 scales (lm_attend's cache)
  int64_t slot_bytes;  // bytes per FP8 slot: 2 hk 128 + 2 hk 4
  int group_heads;     // K/V heads per workgroup of the head-group kernels (0 = pick from the shape)
  int dense_per, dense_base, dense_span;  // dense rows (len_mode 2): slot (n / per) * span + t
  // Fused rotary (rope != 0, decode rows only): q and the row's own key are
  // rotated in the kernel (Qwen3: normalised first; FP8 ring: K and V
  // quantized), and the split holding the row's new key writes it into slot
  // slots[n] of kv_w (the cache kv points to) and takes it from registers.
  int rope;
  const bf16_t* q_norm;
  const bf16_t* k_norm;
  const int32_t* slots;
  bf16_t* kv_w;
  float eps, theta;
  float coef;  // FP8 ring (lm_rope): pair i turns by p * exp(i * coef)
};

int launch_decode(const DecodeArgs& a, int rows, hipStream_t stream);

// The allocation-free decode entry point's split-partial workspace: a
// file-scope device array of this many bytes per GPU.
constexpr int64_t kNoAllocScratchBytes = 16LL << 20;
constexpr int kMaxDevices = 64;
// Device address of that array on the current device (looked up once per
// device); 0 on success, -1 if the lookup fails.
int noalloc_scratch(float** ptr);

// Copy of whole cache slots (prefix K/V reuse): slot dst[r] takes slot src[r].
int launch_copy_slots(void* kv, const int32_t* src, const int32_t* dst, int tokens, int slot_bytes,
                      hipStream_t stream);

int launch_gather_kv(const void* kv, int hk, const int32_t* indptr, const int32_t* pages, PageDiv pd,
                     const int32_t* seq_ids, const int32_t* lens, const int32_t* out_indptr, int nseq, void* out,
                     hipStream_t stream);

// Tiled MFMA attention (prefill and DiT).
struct TiledArgs {
  const bf16_t* q;
  int64_t q_stride;  // elements between query rows
  // paged source (mode 0): kv slots [2 hk][128]
  const bf16_t* kv;
  const int32_t* pos;
  const int32_t* seq;
  const int32_t* indptr;
  const int32_t* pages;
  const int32_t* work;  // 4 int32 per tile: seq, first row, rows, unused
  PageDiv pd;
  // dense source (mode 1): k, v [slots][hk][128]
  const bf16_t* k;
  const bf16_t* v;
  const int32_t* kv_len_at;
  int q_len;
  int causal;
  int64_t q_bstride, kv_bstride, out_bstride;
  bf16_t* out;
  int hq, hk;
  float scale_log2;
  // Tail split (dense, uniform key ranges): items >= split_from run as
  // split_k key chunks each, writing f32 partials to ws (one segment per
  // chunk: O[128 rows][128] then (m, l)[128 rows]); 0 chunks = no split.
  int split_from, split_k;
  float* ws;
  // Row halves (dense, no split): the last `halved` items run as two
  // workgroups of kTiledRows / 2 packed rows each; 0 = none.
  int halved;
  // Prefill with P carried as two bf16 terms (hi + lo) through P.V.
  int exact_p;
};

// Packed (position, head) query rows per MFMA tile: one 8-wave workgroup, one per CU.
constexpr int kTiledRows = 256;
// Bytes of one partial segment of the tail split: O (f32) and (m, l) per packed row.
constexpr int64_t kSegmentBytes = (int64_t)kTiledRows * (128 + 2) * 4;

// Prefill work list: a header of kPrefillWorkHeader int32 (entries 0..8: the
// item ranges of the 8 XCDs, range x = [h[x], h[x + 1])) then 4 int32 per
// (tile, kv head) item: sequence, first row, rows, kv head.
constexpr int kPrefillWorkHeader = 16;
constexpr int kXcds = 8;
int launch_prefill(const TiledArgs& a, int workgroups, hipStream_t stream);

// Rotary embedding + K/V scatter (the step before attention).
struct RopeArgs {
  bf16_t* qkv;
  int64_t ld;  // elements between qkv rows
  const bf16_t* q_norm;
  const bf16_t* k_norm;
  const int32_t* pos;    // [rows], or [rows][3] (t, h, w) for M-RoPE
  const int32_t* slots;  // [rows] cache slot of each row
  bf16_t* kv;            // bf16 slots [2 hk][128]
  void* kv_bytes;        // FP8 slots of slot_bytes
  int64_t slot_bytes;
  bf16_t* k_cache;  // M-RoPE: separate caches [slots][hk][128]
  bf16_t* v_cache;
  int rows, hq, hk;
  int per, base, span;  // dense rows: seq n / per at position base + n % per, slot seq * span + pos
  int mrope_hw;
  float eps, theta, coef;
};
// Head-64 ring attentions (Mimi, Qwen3-TTS codec, depformer).
struct ShortArgs {
  const bf16_t* qkv;
  const int32_t* pos;
  const int32_t* lines;  // session -> line of the per-session state
  void* state;           // Mimi / codec rings: state + lines[s] * stride bytes
  int64_t stride;
  bf16_t* ws;            // depformer workspace [seqs][8][K | V][heads * 64]
  bf16_t* out;
  bf16_t* qkv_rw;        // Mimi rotary: the qkv rows, q turned in place
  int rows, heads, T, context, step;
  float scale, theta;
  float coef;            // Mimi rotary: pair i turns by p * exp(i * coef)
};
constexpr int kShortMimi = 0, kShortCodec = 1, kShortDep = 2, kShortMimiRope = 3;
int launch_short(const ShortArgs& a, int kind, hipStream_t stream);

constexpr int kRopeQwen3 = 0, kRopeQwen3Dense = 1, kRopeHidream = 2, kRopeLm = 3;
int launch_rope(const RopeArgs& a, int mode, hipStream_t stream);
int launch_dit(const TiledArgs& a, int batch, hipStream_t stream);
// Items and the tail split launch_dit would use for a call (split_k = 0: none).
void dit_split(const TiledArgs& a, int batch, int resident, int* items, int* split_from, int* split_k);
// Items launch_dit should run as row halves when no split is used (0: none).
int dit_halves(const TiledArgs& a, int batch, int resident);

}  // namespace omni
