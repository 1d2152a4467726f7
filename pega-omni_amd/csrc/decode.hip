// Paged GQA / MHA decode attention for gfx950: split-K over keys, bandwidth
// bound, no MFMA (one query token per row is a GEMV per K/V head).
//
// Semantics are those of qwen3_attend (crates/omni-qwen3/kernels/qwen3.cu:
// 123-240) and lm_attend over bf16 slots (crates/omni-personaplex/kernels/
// lm.cu:273-290): row n of sequence s = ragged ? seq[n] : n sees the first
// min(pos[n] + 1, context) tokens of s, token t in slot
// pages[indptr[s] + t / page] * page + t % page, slot = [K heads | V heads][128].
//
// Work: one workgroup of four waves per (split, kv head, row). A split is
// `chunk` consecutive keys; wave w takes 32-key tiles w, w + 4, ... of it.
// Within a wave, lane (r, c) = (lane / 16, lane % 16) owns the 16-byte chunk c
// (8 of 128 dims) of keys 4 i + r of the tile, i = 0..7: each row of 16 lanes
// reads one key's 256-byte K (and V) head row with one coalesced 16-byte load
// per lane, so every load instruction moves four whole 256-byte rows.
// Scores: per-lane partial dot products of the G query heads sharing the K/V
// head, summed over the 16 lanes of a DPP row. Softmax: base 2 with the scale
// folded into q, online per tile, the running max shared by the whole wave.
// V: each lane accumulates p * v for its 8 dims and G heads; rows merge at the
// end, waves merge in LDS, splits merge in `decode_combine` (log-sum-exp).
// (Merging in the last-arriving split workgroup needs a device-scope release
// fence per workgroup, which writes back the L2 on gfx950 and costs far more
// than the separate combine launch.)
#include <mutex>

#include "common.h"
#include "kernels.h"
#include "rotary.h"

namespace omni {

constexpr int kDecodeWaves = 4;
constexpr int kDecodeThreads = kDecodeWaves * 64;
constexpr int kTileKeys = 32;

__device__ __forceinline__ int decode_len(const DecodeArgs& a, int n, int s) {
  int len;
  if (a.len_mode == 0)
    len = a.pos[n] + 1;
  else if (a.len_mode == 1)
    len = (a.indptr[s + 1] - a.indptr[s] - 1) * a.pd.page + a.pos[s];
  else
    len = a.dense_base + n % a.dense_per + 1;
  return min(len, a.context);
}

// Keys per split of a row of `len` keys: ceil(len / chunk) splits (at most
// the plan's), of equal length rounded up to 32 keys, so no split is a short
// remainder. A multiple of 32 keeps every key group a kernel loads inside one
// page when the page is a multiple of the group.
__device__ __forceinline__ int decode_split_len(const DecodeArgs& a, int len) {
  const int ns = len <= a.chunk ? 1 : min(a.splits, (len + a.chunk - 1) / a.chunk);
  return ((len + ns - 1) / ns + 31) & ~31;
}

__device__ __forceinline__ int decode_nsplit(int len, int split_len) {
  return len <= 0 ? 1 : (len + split_len - 1) / split_len;
}

// Merge the four waves' (m, l, o) of one (split, kv head, row) workgroup and
// write the row's output (one split) or the split's normalised partial.
template <int G>
__device__ __forceinline__ void merge_waves(const DecodeArgs& a, int n, int kh, int split, int nsplit, int len,
                                            const float (*sm_m)[G], const float (*sm_l)[G],
                                            const float (*sm_o)[G][kHead]) {
  for (int i = threadIdx.x; i < G * kHead; i += kDecodeThreads) {
    const int g = i / kHead, d = i % kHead;
    float top = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) top = fmaxf(top, sm_m[w][g]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) {
      const float e = sm_m[w][g] == -INFINITY ? 0.f : fast_exp2(sm_m[w][g] - top);
      num = fmaf(sm_o[w][g][d], e, num);
      den = fmaf(sm_l[w][g], e, den);
    }
    const int64_t h = (int64_t)n * a.hq + kh * G + g;
    if (nsplit == 1) {
      a.out[h * kHead + d] = (bf16_t)f2bf(len > 0 ? num / den : 0.f);
    } else {
      a.ws_o[(h * a.splits + split) * kHead + d] = num / den;
      if (d == 0) a.ws_lse[h * a.splits + split] = top + __log2f(den);
    }
  }
}

// Where key t of a row lives. kSlotsUniform: every group of 4 key rows
// (page a multiple of 4) lies in one page, so its page id is one wave-uniform
// scalar load; kSlotsLane: each lane loads its own page id; kSlotsDense: a
// dense workspace, slot (n / per) * span + t (qwen3_attend_dense).
constexpr int kSlotsLane = 0, kSlotsUniform = 1, kSlotsDense = 2;

// Page index and slot of token t. A power-of-two page (every engine's 16)
// takes a shift and a mask; DIV: any other page, a multiply-high division.
template <bool DIV>
__device__ __forceinline__ int key_page(const PageDiv& d, int t) {
  return DIV ? page_index(d, t) : t >> d.shift;
}
template <bool DIV>
__device__ __forceinline__ int64_t key_slot(const PageDiv& d, int pid, int t) {
  return DIV ? page_slot(d, pid, t) : (((int64_t)pid << d.shift) | (t & ((1 << d.shift) - 1)));
}

// ROPE: the fused Qwen3 rotary (omni_qwen3_rope_attend), decode rows only
// (each row its own sequence, len = pos[n] + 1, so the row's new key is its
// last). Every workgroup of the row turns its G q heads itself, as qwen3_rope
// would have (RMSNorm, rotary, bf16 rounding), from the row's angle table in
// LDS. The one split holding key pos[n] also turns the row's k head kh,
// writes K and V into slot slots[n], and in the tile that holds key pos[n]
// replaces the loaded K and V of that key (which may predate the write) by
// the values in its registers.
template <int G, int SLOTS, bool DIV, bool ROPE>
__global__ __launch_bounds__(kDecodeThreads) void decode_split(DecodeArgs a) {
  const int kh = blockIdx.y, n = blockIdx.z;
  const int split = rotated_split(blockIdx.x, kh + a.hk * n, a.splits);
  const int s = a.ragged ? a.seq[n] : n;
  const int len = decode_len(a, n, s);
  const int split_len = decode_split_len(a, len);
  const int nsplit = decode_nsplit(len, split_len);
  if (split >= nsplit) return;
  const int t0 = split * split_len;
  const int t1 = min(len, t0 + split_len);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: tile starts are scalar
  const int r = lane >> 4, c = lane & 15;

  float q[G][8];
  const bf16_t* qp = a.qkv + (int64_t)n * a.q_stride + (int64_t)kh * G * kHead + c * 8;
  const int64_t per_slot = 2LL * a.hk * kHead;
  int cur = -1;  // ROPE: the row's new key, when this split holds it
  uint4 k_cur = {}, v_cur = {};
  if constexpr (ROPE) {
    // Every load of the prologue (q, the norm weights, the new key's k and v
    // rows) is issued before the angle table's math and barrier.
    const int p = len - 1;  // pos[n]: decode rows see pos[n] + 1 keys
    uint4 q_raw[G];
#pragma unroll
    for (int g = 0; g < G; ++g) q_raw[g] = ldg16(qp + g * kHead);
    const uint4 wq_raw = ldg16(a.q_norm + 8 * c);
    uint4 wk_raw = {};
    if (t0 <= p && p < t1) {
      cur = p;
      const bf16_t* row = a.qkv + (int64_t)n * a.q_stride + c * 8;
      wk_raw = ldg16(a.k_norm + 8 * c);
      k_cur = ldg16(row + (int64_t)(a.hq + kh) * kHead);
      v_cur = ldg16(row + (int64_t)(a.hq + a.hk + kh) * kHead);
    }
    __shared__ float s_cos[kHead / 2], s_sin[kHead / 2];
    if (threadIdx.x < kHead / 2) sincosf(qwen3_angle(p, threadIdx.x, a.theta), &s_sin[threadIdx.x], &s_cos[threadIdx.x]);
    __syncthreads();
    float cs[8], sn[8], w[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      cs[e] = s_cos[8 * (c & 7) + e];
      sn[e] = s_sin[8 * (c & 7) + e];
    }
    const bool lo = c < 8;
    widen8(wq_raw, w);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float x[8], v[8], o[8];
      widen8(q_raw[g], x);
      rms_norm_head(x, w, a.eps, v);
      rotate_half(v, cs, sn, lo, o);
#pragma unroll
      for (int e = 0; e < 8; ++e) q[g][e] = round_bf16(o[e]) * a.scale_log2;
    }
    if (cur >= 0) {
      float x[8], v[8], o[8];
      widen8(wk_raw, w);
      widen8(k_cur, x);
      rms_norm_head(x, w, a.eps, v);
      rotate_half(v, cs, sn, lo, o);
      k_cur = pack8(o);
    }
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      widen8(ldg16(qp + g * kHead), q[g]);
#pragma unroll
      for (int e = 0; e < 8; ++e) q[g][e] *= a.scale_log2;
    }
  }

  const int32_t* pg = SLOTS == kSlotsDense ? nullptr : a.pages + a.indptr[s];
  const int64_t dense_first = SLOTS == kSlotsDense ? (int64_t)(n / a.dense_per) * a.dense_span : 0;
  const bf16_t* kb = a.kv + (int64_t)kh * kHead + c * 8;
  const bf16_t* vb = a.kv + (int64_t)(a.hk + kh) * kHead + c * 8;

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  }

  // Key tb + 4 i + r of a tile, clamped to the split (a clamped key has p = 0
  // and reads a valid slot). Page ids are loaded one tile ahead, so the K/V
  // loads of a tile never wait on its page-table reads.
  auto page_of = [&](int tb, int i) -> int {
    if constexpr (SLOTS == kSlotsDense)
      return 0;
    else if constexpr (SLOTS == kSlotsUniform)
      return pg[key_page<DIV>(a.pd, __builtin_amdgcn_readfirstlane(min(tb + 4 * i, t1 - 1)))];
    else
      return pg[key_page<DIV>(a.pd, min(tb + 4 * i + r, t1 - 1))];
  };
  constexpr int kStride = kDecodeWaves * kTileKeys;
  // G = 1: two register tiles, the next tile's loads (and the page ids of the
  // one after) issued before this tile's math. The tile after the split's
  // last is loaded too, its keys clamped to slot t1 - 1 (cached), so every
  // wait is a plain in-order count.
  struct KVTile {
    uint4 kr[8], vr[8];
  };
  auto load_tile = [&](KVTile& x, int tb, const int* pid) __attribute__((always_inline)) {
    int64_t off[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int t = min(tb + 4 * i + r, t1 - 1);
      if constexpr (SLOTS == kSlotsDense)
        off[i] = (dense_first + t) * per_slot;
      else
        off[i] = key_slot<DIV>(a.pd, pid[i], t) * per_slot;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) x.kr[i] = ldg16_stream(kb + off[i]);
#pragma unroll
    for (int i = 0; i < 8; ++i) x.vr[i] = ldg16_stream(vb + off[i]);
  };
  // ROPE: the row's new key from registers (cur is wave-uniform). It is the
  // split's last key (t1 - 1), so the keys clamped past the split read its
  // slot too; they are replaced as well (their p is 0, but 0 times a stale
  // NaN or infinity in the slot would still reach the sum).
  auto patch_tile = [&](KVTile& x, int tb) __attribute__((always_inline)) {
    if constexpr (ROPE) {
      if (cur >= 0 && tb + kTileKeys > cur) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (tb + 4 * i + r >= cur) {
            x.kr[i] = k_cur;
            x.vr[i] = v_cur;
          }
      }
    }
  };
  auto compute_tile = [&](const KVTile& x, int tb) __attribute__((always_inline)) {
    float sc[G][8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float kf[8];
      widen8(x.kr[i], kf);
      const bool valid = tb + 4 * i + r < t1;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) d = fmaf(q[g][e], kf[e], d);
        d = row16_sum(d);
        sc[g][i] = valid ? d : -INFINITY;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = sc[g][0];
#pragma unroll
      for (int i = 1; i < 8; ++i) mx = fmaxf(mx, sc[g][i]);
      mx = fmaxf(mx, xor_lane(mx, 16));
      mx = fmaxf(mx, xor_lane(mx, 32));
      const float mn = fmaxf(m[g], mx);
      const float corr = fast_exp2(m[g] - mn);
      m[g] = mn;
      float ps = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        sc[g][i] = fast_exp2(sc[g][i] - mn);
        ps += sc[g][i];
      }
      l[g] = fmaf(l[g], corr, ps);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] *= corr;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float vf[8];
      widen8(x.vr[i], vf);
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(sc[g][i], vf[e], acc[g][e]);
    }
  };
  const int tb0 = t0 + wave * kTileKeys;
  if (G > 1 && tb0 < t1) {
    // One tile at a time (G > 1: twice the math per tile, and the second
    // register tile would cost more occupancy than it hides).
    int pid[8] = {};
    KVTile ta;
#pragma unroll
    for (int i = 0; i < 8; ++i) pid[i] = page_of(tb0, i);
    for (int tb = tb0; tb < t1; tb += kStride) {
      load_tile(ta, tb, pid);
      if (tb + kStride < t1) {
#pragma unroll
        for (int i = 0; i < 8; ++i) pid[i] = page_of(tb + kStride, i);
      }
      patch_tile(ta, tb);
      compute_tile(ta, tb);
    }
  } else if (tb0 < t1) {
    int pid[8] = {};
    KVTile ta, tn;
#pragma unroll
    for (int i = 0; i < 8; ++i) pid[i] = page_of(tb0, i);
    load_tile(ta, tb0, pid);
#pragma unroll
    for (int i = 0; i < 8; ++i) pid[i] = page_of(tb0 + kStride, i);
    for (int tb = tb0;; tb += 2 * kStride) {
      load_tile(tn, tb + kStride, pid);
#pragma unroll
      for (int i = 0; i < 8; ++i) pid[i] = page_of(tb + 2 * kStride, i);
      __builtin_amdgcn_sched_barrier(0);  // keep the next tile's loads ahead of this tile's math
      patch_tile(ta, tb);
      compute_tile(ta, tb);
      if (tb + kStride >= t1) break;
      load_tile(ta, tb + 2 * kStride, pid);
#pragma unroll
      for (int i = 0; i < 8; ++i) pid[i] = page_of(tb + 3 * kStride, i);
      __builtin_amdgcn_sched_barrier(0);
      patch_tile(tn, tb + kStride);
      compute_tile(tn, tb + kStride);
      if (tb + 2 * kStride >= t1) break;
    }
  }

  // ROPE: the new key's slot is written after the key loop (a store counts in
  // vmcnt: issued before the loop, the first tile's wait would wait for it).
  if (ROPE && cur >= 0 && threadIdx.x < 16) {  // one DPP row writes the slot's K and V head kh
    bf16_t* slot = a.kv_w + (int64_t)a.slots[n] * per_slot + c * 8;
    *reinterpret_cast<uint4*>(slot + (int64_t)kh * kHead) = k_cur;
    *reinterpret_cast<uint4*>(slot + (int64_t)(a.hk + kh) * kHead) = v_cur;
  }

  // Rows of the wave hold disjoint keys under one shared max: add them up.
#pragma unroll
  for (int g = 0; g < G; ++g) {
    l[g] += xor_lane(l[g], 16);
    l[g] += xor_lane(l[g], 32);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      acc[g][e] += xor_lane(acc[g][e], 16);
      acc[g][e] += xor_lane(acc[g][e], 32);
    }
  }

  __shared__ float sm_m[kDecodeWaves][G], sm_l[kDecodeWaves][G];
  __shared__ float sm_o[kDecodeWaves][G][kHead];
  if (r == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sm_o[wave][g][c * 8 + e] = acc[g][e];
      if (c == 0) {
        sm_m[wave][g] = m[g];
        sm_l[wave][g] = l[g];
      }
    }
  }
  __syncthreads();
  merge_waves<G>(a, n, kh, split, nsplit, len, sm_m, sm_l, sm_o);
}

// ------------------------------------------- K/V head groups over bf16 slots
//
// decode_split's work with H adjacent K/V heads per workgroup, so that every
// load instruction reads whole contiguous runs of a slot: lane (r, hl, c) =
// (lane / 16H, lane / 16 % H, lane % 16) owns the 16-byte chunk c of K/V head
// kh = kg H + hl for key row r, so one load instruction moves R = 4 / H keys x
// H heads x 256 bytes. Each lane dots its chunk with the G query heads of kh.
// The plan picks H = 2 for MHA rows (lm_attend's tick over bf16 slots): 505-508
// us per 128-session layer against 512-515 with one head per workgroup
// (decode_split<1>), where H = 4 took 526-540. A plan may fix H for GQA rows
// too (G = 2: slower on the 64-row talker bucket, whose call is short).
// Everything else is decode_split's: two register tiles for G = 1 and one for
// G > 1, base-2 online softmax with the scale in q, per-lane V accumulation,
// waves merged in LDS, splits by decode_combine. The grid is one-dimensional,
// split index fastest, then head group, then row, so the head groups of one
// row run close together.

// Combine the R = 4 / H key rows of a wave (lanes 16H apart), per lane.
template <int H, bool MAX>
__device__ __forceinline__ float across_key_rows16(float v) {
  if constexpr (H == 1) v = MAX ? fmaxf(v, xor_lane(v, 16)) : v + xor_lane(v, 16);
  if constexpr (H <= 2) v = MAX ? fmaxf(v, xor_lane(v, 32)) : v + xor_lane(v, 32);
  return v;
}

template <int G, int H, bool UP, bool DIV>
__global__ __launch_bounds__(kDecodeThreads) void decode_split_mh(DecodeArgs a, int rows) {
  constexpr int R = 4 / H;       // keys per load instruction
  constexpr int NI = 8;          // load instructions per wave and tile
  constexpr int kKeys = R * NI;  // keys per wave and tile
  const int groups = a.hk / H;
  const int slot = (int)blockIdx.x % a.splits, rest = (int)blockIdx.x / a.splits;
  const int kg = rest % groups, n = rest / groups;
  if (n >= rows) return;
  const int split = rotated_split(slot, kg + groups * n, a.splits);
  const int s = a.ragged ? a.seq[n] : n;
  const int len = decode_len(a, n, s);
  const int split_len = decode_split_len(a, len);
  const int nsplit = decode_nsplit(len, split_len);
  if (split >= nsplit) return;
  const int t0 = split * split_len;
  const int t1 = min(len, t0 + split_len);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane / (16 * H), hl = (lane >> 4) % H, c = lane & 15;
  const int kh = kg * H + hl;

  // The G query heads kh G .. kh G + G - 1 that share K/V head kh.
  float q[G][8];
  const bf16_t* qp = a.qkv + (int64_t)n * a.q_stride + (int64_t)kh * G * kHead + c * 8;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    widen8(ldg16(qp + g * kHead), q[g]);
#pragma unroll
    for (int e = 0; e < 8; ++e) q[g][e] *= a.scale_log2;
  }

  const int32_t* pg = a.pages + a.indptr[s];
  const int64_t per_slot = 2LL * a.hk * kHead;
  const bf16_t* kb = a.kv + (int64_t)kh * kHead + c * 8;
  const bf16_t* vb = a.kv + (int64_t)(a.hk + kh) * kHead + c * 8;

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  }

  // Key tb + R i + r, clamped to the split (a clamped key has p = 0 and reads
  // a valid slot). UP: the R keys of one instruction share a page (page a
  // multiple of R), so its id is a scalar load.
  auto page_of = [&](int tb, int i) -> int {
    if constexpr (UP)
      return pg[key_page<DIV>(a.pd, __builtin_amdgcn_readfirstlane(min(tb + R * i, t1 - 1)))];
    else
      return pg[key_page<DIV>(a.pd, min(tb + R * i + r, t1 - 1))];
  };
  struct KVTile {
    uint4 kr[NI], vr[NI];
  };
  auto load_tile = [&](KVTile& x, int tb, const int* pid) __attribute__((always_inline)) {
    int64_t off[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) off[i] = key_slot<DIV>(a.pd, pid[i], min(tb + R * i + r, t1 - 1)) * per_slot;
#pragma unroll
    for (int i = 0; i < NI; ++i) x.kr[i] = ldg16_stream(kb + off[i]);
#pragma unroll
    for (int i = 0; i < NI; ++i) x.vr[i] = ldg16_stream(vb + off[i]);
  };
  auto compute_tile = [&](const KVTile& x, int tb) __attribute__((always_inline)) {
    float sc[G][NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      float kf[8];
      widen8(x.kr[i], kf);
      const bool valid = tb + R * i + r < t1;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) d = fmaf(q[g][e], kf[e], d);
        d = row16_sum(d);
        sc[g][i] = valid ? d : -INFINITY;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = sc[g][0];
#pragma unroll
      for (int i = 1; i < NI; ++i) mx = fmaxf(mx, sc[g][i]);
      mx = across_key_rows16<H, true>(mx);
      const float mn = fmaxf(m[g], mx);
      const float corr = fast_exp2(m[g] - mn);
      m[g] = mn;
      float ps = 0.f;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        sc[g][i] = fast_exp2(sc[g][i] - mn);
        ps += sc[g][i];
      }
      l[g] = fmaf(l[g], corr, ps);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] *= corr;
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      float vf[8];
      widen8(x.vr[i], vf);
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(sc[g][i], vf[e], acc[g][e]);
    }
  };
  constexpr int kStride = kDecodeWaves * kKeys;
  const int tb0 = t0 + wave * kKeys;
  if (G > 1 && tb0 < t1) {
    // One register tile at a time (as decode_split does for G > 1).
    int pid[NI];
    KVTile ta;
#pragma unroll
    for (int i = 0; i < NI; ++i) pid[i] = page_of(tb0, i);
    for (int tb = tb0; tb < t1; tb += kStride) {
      load_tile(ta, tb, pid);
      if (tb + kStride < t1) {
#pragma unroll
        for (int i = 0; i < NI; ++i) pid[i] = page_of(tb + kStride, i);
      }
      compute_tile(ta, tb);
    }
  } else if (tb0 < t1) {
    int pid[NI];
    KVTile ta, tn;
#pragma unroll
    for (int i = 0; i < NI; ++i) pid[i] = page_of(tb0, i);
    load_tile(ta, tb0, pid);
#pragma unroll
    for (int i = 0; i < NI; ++i) pid[i] = page_of(tb0 + kStride, i);
    for (int tb = tb0;; tb += 2 * kStride) {
      load_tile(tn, tb + kStride, pid);
#pragma unroll
      for (int i = 0; i < NI; ++i) pid[i] = page_of(tb + 2 * kStride, i);
      __builtin_amdgcn_sched_barrier(0);  // keep the next tile's loads ahead of this tile's math
      compute_tile(ta, tb);
      if (tb + kStride >= t1) break;
      load_tile(ta, tb + 2 * kStride, pid);
#pragma unroll
      for (int i = 0; i < NI; ++i) pid[i] = page_of(tb + 3 * kStride, i);
      __builtin_amdgcn_sched_barrier(0);
      compute_tile(tn, tb + kStride);
      if (tb + 2 * kStride >= t1) break;
    }
  }

  // The key rows of the wave hold disjoint keys under one shared max.
#pragma unroll
  for (int g = 0; g < G; ++g) {
    l[g] = across_key_rows16<H, false>(l[g]);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = across_key_rows16<H, false>(acc[g][e]);
  }
  __shared__ float sm_m[kDecodeWaves][H * G], sm_l[kDecodeWaves][H * G];
  __shared__ float sm_o[kDecodeWaves][H * G][kHead];
  if (r == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sm_o[wave][hl * G + g][c * 8 + e] = acc[g][e];
      if (c == 0) {
        sm_m[wave][hl * G + g] = m[g];
        sm_l[wave][hl * G + g] = l[g];
      }
    }
  }
  __syncthreads();
  // K/V heads kg H .. kg H + H - 1 serve q heads kg H G .. kg H G + H G - 1:
  // merge_waves with G' = H G and kv head index kg.
  merge_waves<H * G>(a, n, kg, split, nsplit, len, sm_m, sm_l, sm_o);
}

// ------------------------------------------------------------------ FP8 slots
//
// lm_attend's real cache (crates/omni-personaplex/kernels/lm.cu:196-290): a
// slot is [K heads x 128 B | V heads x 128 B | K scales f32 x heads | V scales
// f32 x heads] with FP8 E4M3 values; score = dot(q, k) * k_scale * scale and
// the V row is weighted by p * v_scale. MHA (one q head per K/V head), as
// lm_attend is.
//
// A workgroup takes H adjacent heads of one (row, split). Lane l works on head
// kh0 + (l % 8H) / 8, dims 16 (l % 8) .. + 15 (one 16-byte load of 16 E4M3
// values), key row l / 8H: a load instruction covers R = 8 / H keys, each an
// H * 128-byte contiguous run of K (and of V), and one scale word load serves
// H heads from one sector. E4M3 widens to f32 on the hardware converter
// (v_cvt_pk_f32_fp8, OCP E4M3 on gfx950).

typedef float f32x2_fp8_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void widen16_fp8(const uint4& u, float* v) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f32x2_fp8_t lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], false);
    const f32x2_fp8_t hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], true);
    v[4 * i + 0] = lo.x;
    v[4 * i + 1] = lo.y;
    v[4 * i + 2] = hi.x;
    v[4 * i + 3] = hi.y;
  }
}

// Sum over the 8 lanes of an aligned lane octet.
__device__ __forceinline__ float row8_sum(float v) {
  v += dpp<kQuadSwap1>(v);
  v += dpp<kQuadSwap2>(v);
  v += dpp<kRowHalfMirror>(v);
  return v;
}

// Combine the R = 8 / H key rows of a wave (lanes 8H apart), per lane.
template <int H, bool MAX>
__device__ __forceinline__ float across_key_rows(float v) {
  if constexpr (H == 1) v = MAX ? fmaxf(v, dpp<kRowRor8>(v)) : v + dpp<kRowRor8>(v);
  if constexpr (H <= 2) v = MAX ? fmaxf(v, xor_lane(v, 16)) : v + xor_lane(v, 16);
  if constexpr (H <= 4) v = MAX ? fmaxf(v, xor_lane(v, 32)) : v + xor_lane(v, 32);
  return v;
}

// NI load instructions (NI * R keys) per wave and iteration. UP: the R keys of
// one instruction share a page (page a multiple of R), so its id is a scalar
// load.
// ROPE: lm_rope fused in (omni_lm_rope_attend_fp8), decode rows only. Every
// workgroup of row n turns its q heads as lm_rope does (rounded to bf16) from
// the row's angle table in LDS. The split holding ring index pos[n] % context
// (the row's new key) also turns k, quantizes K and V to E4M3 with their
// per-head scales exactly as lm_rope does, writes them into slot slots[n],
// and takes that key (and any key clamped onto it) from registers.
template <int H, int NI, bool UP, bool DIV, bool ROPE>
__global__ __launch_bounds__(kDecodeThreads) void decode_split_fp8(DecodeArgs a, int rows) {
  constexpr int R = 8 / H;
  // Workgroup i runs on XCD i % 8: the head groups of one (row, split) unit
  // share an XCD (and the slot's scale lines in its L2), while consecutive
  // units spread over the XCDs.
  const int groups = a.hk / H;
  const int x = blockIdx.x & 7, rest = blockIdx.x >> 3;
  const int kg = rest % groups, unit = (rest / groups) * 8 + x;
  const int n = unit / a.splits, split = rotated_split(unit % a.splits, n, a.splits);
  if (n >= rows) return;
  const int s = a.ragged ? a.seq[n] : n;
  const int len = decode_len(a, n, s);
  const int split_len = decode_split_len(a, len);
  const int nsplit = decode_nsplit(len, split_len);
  if (split >= nsplit) return;
  const int t0 = split * split_len;
  const int t1 = min(len, t0 + split_len);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane / (8 * H), hl = (lane % (8 * H)) >> 3, c = lane & 7;
  const int kh = kg * H + hl;

  float q[16];
  int cur = -1;  // ROPE: the row's new key, when this split holds it
  uint4 kq_cur = {}, vq_cur = {};
  float ks_cur = 0.f, vs_cur = 0.f;
  [[maybe_unused]] int p_rope = 0;
  [[maybe_unused]] uint4 q0r = {}, q1r = {}, k0r = {}, k1r = {}, v0r = {}, v1r = {};
  {
    const bf16_t* qp = a.qkv + (int64_t)n * a.q_stride + (int64_t)kh * kHead + c * 16;
    if constexpr (ROPE) {
      // The prologue's loads go out here; its math runs after the first
      // tile's K/V loads are issued too (rope_prologue below).
      p_rope = a.pos[n];
      const int ring = p_rope % a.context;  // lm_rope writes slot(p % context)
      // Loaded on every path (only the split holding the new key uses k and
      // v), so the wait counts before the rotary math are the same on all paths.
      q0r = ldg16(qp), q1r = ldg16(qp + 8);
      const bf16_t* kp = a.qkv + (int64_t)n * a.q_stride + (int64_t)(a.hk + kh) * kHead + c * 16;
      const bf16_t* vp = kp + (int64_t)a.hk * kHead;
      k0r = ldg16(kp), k1r = ldg16(kp + 8), v0r = ldg16(vp), v1r = ldg16(vp + 8);
      if (t0 <= ring && ring < t1) cur = ring;
    } else {
      widen8(ldg16(qp), q);
      widen8(ldg16(qp + 8), q + 8);
#pragma unroll
      for (int e = 0; e < 16; ++e) q[e] *= a.scale_log2;
    }
  }

  const int32_t* pg = a.pages + a.indptr[s];
  const uint8_t* kvb = reinterpret_cast<const uint8_t*>(a.kv);
  const int64_t sb = a.slot_bytes;
  const int64_t koff = (int64_t)kh * kHead + c * 16, voff = (int64_t)(a.hk + kh) * kHead + c * 16;
  const int64_t ksoff = 2LL * a.hk * kHead + kh * 4, vsoff = 2LL * a.hk * kHead + (a.hk + kh) * 4;

  float m = -INFINITY, l = 0.f, acc[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;

  constexpr int kKeys = R * NI;  // keys per wave per iteration
  // Key tb + R i + r, clamped to the split (a clamped key has p = 0 and reads
  // a valid slot). Two register tiles: the loads of the next tile are in
  // flight while this one is computed, and page ids are read a tile earlier
  // still. The tile after the split's last is loaded too, unconditionally
  // (all its keys clamp to slot t1 - 1, already cached), so every wait is a
  // plain in-order count.
  auto page_of = [&](int tb, int i) -> int {
    if constexpr (UP)
      return pg[key_page<DIV>(a.pd, __builtin_amdgcn_readfirstlane(min(tb + R * i, t1 - 1)))];
    else
      return pg[key_page<DIV>(a.pd, min(tb + R * i + r, t1 - 1))];
  };
  struct Tile {
    uint4 kr[NI], vr[NI];
    float ks[NI], vs[NI];
  };
  auto load_tile = [&](Tile& x, int tb, const int* pid) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int t = min(tb + R * i + r, t1 - 1);
      const uint8_t* sp = kvb + key_slot<DIV>(a.pd, pid[i], t) * sb;
      x.kr[i] = ldg16_stream(sp + koff);
      x.vr[i] = ldg16_stream(sp + voff);
      x.ks[i] = *reinterpret_cast<const float*>(sp + ksoff);
      x.vs[i] = *reinterpret_cast<const float*>(sp + vsoff);
    }
  };
  // ROPE: the row's new key from registers, for the lanes whose key (after
  // clamping to the split) is it (cur is wave-uniform).
  auto patch_tile = [&](Tile& x, int tb) {
    if constexpr (ROPE) {
      if (cur >= tb && (cur < tb + kKeys || cur == t1 - 1)) {
#pragma unroll
        for (int i = 0; i < NI; ++i)
          if (min(tb + R * i + r, t1 - 1) == cur) {
            x.kr[i] = kq_cur;
            x.vr[i] = vq_cur;
            x.ks[i] = ks_cur;
            x.vs[i] = vs_cur;
          }
      }
    }
  };
  auto compute_tile = [&](const Tile& x, int tb) {
    float sc[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      float kf[16];
      widen16_fp8(x.kr[i], kf);
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) d = fmaf(q[e], kf[e], d);
      d = row8_sum(d) * x.ks[i];
      sc[i] = tb + R * i + r < t1 ? d : -INFINITY;
    }
    float mx = sc[0];
#pragma unroll
    for (int i = 1; i < NI; ++i) mx = fmaxf(mx, sc[i]);
    mx = across_key_rows<H, true>(mx);
    const float mn = fmaxf(m, mx);
    const float corr = fast_exp2(m - mn);
    m = mn;
    float ps = 0.f;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      sc[i] = fast_exp2(sc[i] - mn);
      ps += sc[i];
    }
    l = fmaf(l, corr, ps);
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] *= corr;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      float vf[16];
      widen16_fp8(x.vr[i], vf);
      const float pv = sc[i] * x.vs[i];
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = fmaf(pv, vf[e], acc[e]);
    }
  };
  constexpr int kStride = kDecodeWaves * kKeys;
  // ROPE: the rotary math (all waves: the angle table needs a barrier).
  auto rope_prologue = [&]() {
    __shared__ float s_cos[kHead / 2], s_sin[kHead / 2];
    if (threadIdx.x < kHead / 2)
      sincosf(expf((float)threadIdx.x * a.coef) * (float)p_rope, &s_sin[threadIdx.x], &s_cos[threadIdx.x]);
    __syncthreads();
    // Lane c holds pairs 8c .. 8c + 7 (elements 16c .. 16c + 15).
    float cs[8], sn[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      cs[j] = s_cos[8 * c + j];
      sn[j] = s_sin[8 * c + j];
    }
    widen8(q0r, q);
    widen8(q1r, q + 8);
    rotate_interleaved<8>(q, cs, sn);
#pragma unroll
    for (int e = 0; e < 16; ++e) q[e] = round_bf16(q[e]) * a.scale_log2;
    if (cur >= 0) {
      // K rotated (unrounded) and V as read, each quantized with its head's
      // scale: the head's 128 values sit on 8 lanes, so its absmax is an
      // 8-lane max (exact in any order).
      float kx[16], vx[16];
      widen8(k0r, kx);
      widen8(k1r, kx + 8);
      widen8(v0r, vx);
      widen8(v1r, vx + 8);
      rotate_interleaved<8>(kx, cs, sn);
      float ka = 0.f, va = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        ka = fmaxf(ka, fabsf(kx[e]));
        va = fmaxf(va, fabsf(vx[e]));
      }
      ka = fmaxf(ka, dpp<kQuadSwap1>(ka));
      ka = fmaxf(ka, dpp<kQuadSwap2>(ka));
      ka = fmaxf(ka, dpp<kRowHalfMirror>(ka));
      va = fmaxf(va, dpp<kQuadSwap1>(va));
      va = fmaxf(va, dpp<kQuadSwap2>(va));
      va = fmaxf(va, dpp<kRowHalfMirror>(va));
      ks_cur = e4m3_scale(ka);
      vs_cur = e4m3_scale(va);
      const float kinv = 1.f / ks_cur, vinv = 1.f / vs_cur;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        kx[e] *= kinv;
        vx[e] *= vinv;
      }
      const uint2 klo = e4m3x8(kx), khi = e4m3x8(kx + 8), vlo = e4m3x8(vx), vhi = e4m3x8(vx + 8);
      kq_cur = make_uint4(klo.x, klo.y, khi.x, khi.y);
      vq_cur = make_uint4(vlo.x, vlo.y, vhi.x, vhi.y);
    }
  };
  const int tb0 = t0 + wave * kKeys;
  int pid[NI];
  Tile ta, tb_;
  // ROPE: on every wave, even one with no tile (its keys clamp to the split's
  // last, a valid slot). A load issued on one path only would make the
  // compiler's wait counts in the prologue assume it is the newest, and the
  // prologue would wait for this whole tile before the loop issues the next.
  if (ROPE || tb0 < t1) {
#pragma unroll
    for (int i = 0; i < NI; ++i) pid[i] = page_of(tb0, i);
    load_tile(ta, tb0, pid);
#pragma unroll
    for (int i = 0; i < NI; ++i) pid[i] = page_of(tb0 + kStride, i);
  }
  if constexpr (ROPE) rope_prologue();  // every wave: it holds a barrier
  if (tb0 < t1) {
    for (int tb = tb0;; tb += 2 * kStride) {
      load_tile(tb_, tb + kStride, pid);
#pragma unroll
      for (int i = 0; i < NI; ++i) pid[i] = page_of(tb + 2 * kStride, i);
      __builtin_amdgcn_sched_barrier(0);  // keep the next tile's loads ahead of this tile's math
      patch_tile(ta, tb);
      compute_tile(ta, tb);
      if (tb + kStride >= t1) break;
      load_tile(ta, tb + 2 * kStride, pid);
#pragma unroll
      for (int i = 0; i < NI; ++i) pid[i] = page_of(tb + 3 * kStride, i);
      __builtin_amdgcn_sched_barrier(0);
      patch_tile(tb_, tb + kStride);
      compute_tile(tb_, tb + kStride);
      if (tb + 2 * kStride >= t1) break;
    }
  }

  // ROPE: the new key's slot is written after the key loop. A store counts
  // in vmcnt, so one issued before the loop would make the first tile's wait
  // wait for its acknowledgement too.
  if (ROPE && cur >= 0 && threadIdx.x < 8 * H) {  // wave 0's key-row-0 lanes: heads kg H ..
    uint8_t* slot = reinterpret_cast<uint8_t*>(a.kv_w) + (int64_t)a.slots[n] * a.slot_bytes;
    *reinterpret_cast<uint4*>(slot + (int64_t)kh * kHead + c * 16) = kq_cur;
    *reinterpret_cast<uint4*>(slot + (int64_t)(a.hk + kh) * kHead + c * 16) = vq_cur;
    if (c == 0) {
      float* scales = reinterpret_cast<float*>(slot + 2LL * a.hk * kHead);
      scales[kh] = ks_cur;
      scales[a.hk + kh] = vs_cur;
    }
  }
  // The key rows of the wave hold disjoint keys under one shared max.
  l = across_key_rows<H, false>(l);
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = across_key_rows<H, false>(acc[e]);
  __shared__ float sm_m[kDecodeWaves][H], sm_l[kDecodeWaves][H];
  __shared__ float sm_o[kDecodeWaves][H][kHead];
  if (r == 0) {
#pragma unroll
    for (int e = 0; e < 16; ++e) sm_o[wave][hl][c * 16 + e] = acc[e];
    if (c == 0) {
      sm_m[wave][hl] = m;
      sm_l[wave][hl] = l;
    }
  }
  __syncthreads();
  // Heads kg H .. kg H + H - 1 are q heads kh G + g of merge_waves with G = H.
  merge_waves<H>(a, n, kg, split, nsplit, len, sm_m, sm_l, sm_o);
}

// Merge the splits of every (row, q head) that used more than one: one wave
// per (q head, row), two dims per lane (d and d + 64; half the waves of a
// thread per dim, 0.2-0.4% faster on every decode workload). A thread's
// loads (the row's split lse values and its dim of every split's partial) are
// all issued before any is used, so the merge costs one memory round trip
// rather than one per split (up to kCombineBatch splits per round trip; 12
// covers the ten splits of the Qwen3-TTS bucket's 256-key plan in one: config 2
// 63.2 against 63.6-63.7 us per call with 8).
constexpr int kCombineBatch = 12;

__global__ __launch_bounds__(64) void decode_combine(DecodeArgs a) {
  const int h = blockIdx.x, n = blockIdx.y, d = threadIdx.x;  // dims d and d + 64
  const int s = a.ragged ? a.seq[n] : n;
  const int len = decode_len(a, n, s);
  const int nsplit = decode_nsplit(len, decode_split_len(a, len));
  if (nsplit <= 1) return;
  const int64_t hh = (int64_t)n * a.hq + h;
  const float* lse = a.ws_lse + hh * a.splits;
  const float* po = a.ws_o + hh * a.splits * kHead + d;
  float top = -INFINITY, num0 = 0.f, num1 = 0.f, den = 0.f;
  for (int i0 = 0; i0 < nsplit; i0 += kCombineBatch) {
    float lv[kCombineBatch], o0[kCombineBatch], o1[kCombineBatch];
#pragma unroll
    for (int k = 0; k < kCombineBatch; ++k) {
      const bool in = i0 + k < nsplit;
      lv[k] = in ? lse[i0 + k] : -INFINITY;
      o0[k] = in ? po[(int64_t)(i0 + k) * kHead] : 0.f;
      o1[k] = in ? po[(int64_t)(i0 + k) * kHead + 64] : 0.f;
    }
    float bt = top;
#pragma unroll
    for (int k = 0; k < kCombineBatch; ++k) bt = fmaxf(bt, lv[k]);
    const float c = top == -INFINITY ? 0.f : fast_exp2(top - bt);
    num0 *= c;
    num1 *= c;
    den *= c;
#pragma unroll
    for (int k = 0; k < kCombineBatch; ++k) {
      const float w = lv[k] == -INFINITY ? 0.f : fast_exp2(lv[k] - bt);
      den += w;
      num0 = fmaf(w, o0[k], num0);
      num1 = fmaf(w, o1[k], num1);
    }
    top = bt;
  }
  a.out[hh * kHead + d] = (bf16_t)f2bf(num0 / den);
  a.out[hh * kHead + d + 64] = (bf16_t)f2bf(num1 / den);
}

// Heads per workgroup: the most that still leaves about 4 workgroups per CU.
static int fp8_heads_per_group(const DecodeArgs& a, int rows) {
  if (a.group_heads) return a.group_heads;
  for (int h = 8; h > 1; h >>= 1)
    if (a.hk % h == 0 && (int64_t)rows * (a.hk / h) * a.splits >= 2048) return h;
  return 1;
}

// Dynamic LDS the FP8 launch reserves and leaves unused. With the kernel's
// static LDS (8.25 KiB at 4 heads per workgroup, 16.25 KiB at 8) it holds the
// launch to two workgroups per CU at 4 heads and to one at 8, where its
// 142-148 VGPRs would allow three. Fewer reads in flight per CU read faster
// here: config 3 over FP8 slots at 4 heads 280.8-280.9 against 282.7-283.1 us
// per call with three per CU; at 8 heads (the FP8 plan's) 275.0-275.4 against
// 280.4-281.0 with two per CU and 281.2-281.8 with three.
constexpr int kFp8OccupancyLds = 64 << 10;

// Dynamic LDS that holds a head-group launch to one workgroup per CU (the
// head-group launch below says when).
constexpr int kMhSoloLds = 80 << 10;

template <int H, bool ROPE>
static void launch_fp8_hr(const DecodeArgs& a, int rows, hipStream_t stream) {
  const int units = rows * a.splits;
  const dim3 grid(8 * (a.hk / H) * ((units + 7) / 8));
  constexpr int R = 8 / H;
  const bool up = a.pd.page % R == 0;
  if (!page_pow2(a.pd)) {
    if (up)
      decode_split_fp8<H, 4, true, true, ROPE><<<grid, kDecodeThreads, kFp8OccupancyLds, stream>>>(a, rows);
    else
      decode_split_fp8<H, 4, false, true, ROPE><<<grid, kDecodeThreads, kFp8OccupancyLds, stream>>>(a, rows);
  } else if (up) {
    decode_split_fp8<H, 4, true, false, ROPE><<<grid, kDecodeThreads, kFp8OccupancyLds, stream>>>(a, rows);
  } else {
    decode_split_fp8<H, 4, false, false, ROPE><<<grid, kDecodeThreads, kFp8OccupancyLds, stream>>>(a, rows);
  }
}

template <int H>
static void launch_fp8_h(const DecodeArgs& a, int rows, hipStream_t stream) {
  if (a.rope)
    launch_fp8_hr<H, true>(a, rows, stream);
  else
    launch_fp8_hr<H, false>(a, rows, stream);
}

static int launch_decode_fp8(const DecodeArgs& a, int rows, hipStream_t stream) {
  if (a.hq != a.hk) return -2;
  if (a.rope && (a.len_mode != 0 || a.ragged || a.context <= 0 || a.context == INT32_MAX)) return -2;
  // The one-dimensional grid (at most hk (rows splits + 7) workgroups) must fit an int.
  if ((int64_t)a.hk * ((int64_t)rows * a.splits + 7) > INT32_MAX) return -2;
  switch (fp8_heads_per_group(a, rows)) {
    case 8: launch_fp8_h<8>(a, rows, stream); break;
    case 4: launch_fp8_h<4>(a, rows, stream); break;
    case 2: launch_fp8_h<2>(a, rows, stream); break;
    case 1: launch_fp8_h<1>(a, rows, stream); break;
    default: return -2;
  }
  if (check_launch() != 0) return -3;
  if (a.splits > 1) {
    decode_combine<<<dim3(a.hq, rows), 64, 0, stream>>>(a);
    if (check_launch() != 0) return -3;
  }
  return 0;
}

int launch_decode(const DecodeArgs& a, int rows, hipStream_t stream) {
  const dim3 grid(a.splits, a.hk, rows);
  if (a.fp8) return launch_decode_fp8(a, rows, stream);
  const int slots = a.len_mode == 2 ? kSlotsDense : a.pd.page % 4 == 0 ? kSlotsUniform : kSlotsLane;
  const bool div = !page_pow2(a.pd);
#define OMNI_DECODE_R(K, G, R)                                                                                  \
  (slots == kSlotsDense   ? K<G, kSlotsDense, false, false><<<grid, kDecodeThreads, 0, stream>>>(a)             \
   : div && slots == kSlotsUniform ? K<G, kSlotsUniform, true, R><<<grid, kDecodeThreads, 0, stream>>>(a)       \
   : div                           ? K<G, kSlotsLane, true, R><<<grid, kDecodeThreads, 0, stream>>>(a)          \
   : slots == kSlotsUniform        ? K<G, kSlotsUniform, false, R><<<grid, kDecodeThreads, 0, stream>>>(a)      \
                                   : K<G, kSlotsLane, false, R><<<grid, kDecodeThreads, 0, stream>>>(a))
#define OMNI_DECODE(K, G) (a.rope ? OMNI_DECODE_R(K, G, true) : OMNI_DECODE_R(K, G, false))
  // Paged bf16 slots: H adjacent K/V heads per workgroup (the plan's
  // group_heads; 0 picks 2 for MHA when that still leaves >= 2048 workgroups,
  // else 1). Measured on the 128-session MHA tick: H = 2 505-508 us against
  // 512-515 for H = 1, H = 4 526-540.
  // The head-group kernel's one-dimensional grid (rows x hk / H x splits
  // workgroups) must fit an int; the plan's pick falls back to one head per
  // workgroup (a three-dimensional grid) when it would not.
  const int64_t mh_units = (int64_t)rows * a.hk * a.splits;
  int mh = 0;
  if (a.rope && (slots == kSlotsDense || a.len_mode != 0 || a.ragged || a.group_heads > 1)) return -2;
  if (slots != kSlotsDense && !a.rope)
    mh = a.group_heads > 0 ? a.group_heads
                           : (a.hq == a.hk && a.hk % 2 == 0 && mh_units / 2 >= 2048 && mh_units / 2 <= INT32_MAX ? 2 : 1);
  if (mh > 1 && mh_units / mh > INT32_MAX) return -2;
  if (mh > 1) {
    const int H = mh;
    const dim3 g1((unsigned)(rows * (a.hk / H) * a.splits));
    // One workgroup (four waves) per CU for large MHA launches of long splits:
    // dynamic LDS the kernel does not use, beyond half the CU's 160 KiB with
    // the kernel's static LDS, where its registers allow two. Fewer reads in
    // flight per CU read faster there. lm_attend over bf16 slots (32 heads,
    // lengths U[100, 3000], the plan's 1024-key splits, two heads per
    // workgroup), us per call, one box, two alternations: 128 rows 483.0
    // against 491.4-491.9, 256 rows 978 against 992-995, 512 rows 1868 against
    // 1900. Shorter launches lose (16 rows on 256-key splits: 88 against
    // 78 us; 32 rows on 512-key splits +1%), 64 rows on 1024-key splits
    // (3072 workgroups) is even.
    const int solo_lds = a.hq == a.hk && a.chunk >= 1024 && g1.x >= 4096 ? kMhSoloLds : 0;
#define OMNI_MH(GG, HH)                                                                                  \
  {                                                                                                      \
    constexpr int kR = 4 / HH;                                                                           \
    const bool up = a.pd.page % kR == 0;                                                                 \
    if (div)                                                                                             \
      up ? decode_split_mh<GG, HH, true, true><<<g1, kDecodeThreads, solo_lds, stream>>>(a, rows)        \
         : decode_split_mh<GG, HH, false, true><<<g1, kDecodeThreads, solo_lds, stream>>>(a, rows);      \
    else                                                                                                 \
      up ? decode_split_mh<GG, HH, true, false><<<g1, kDecodeThreads, solo_lds, stream>>>(a, rows)       \
         : decode_split_mh<GG, HH, false, false><<<g1, kDecodeThreads, solo_lds, stream>>>(a, rows);     \
  }
    switch (a.hq / a.hk * 8 + H) {
      case 8 + 4: OMNI_MH(1, 4) break;
      case 8 + 2: OMNI_MH(1, 2) break;
      case 16 + 4: OMNI_MH(2, 4) break;
      case 16 + 2: OMNI_MH(2, 2) break;
      case 32 + 2: OMNI_MH(4, 2) break;
      default: return -2;
    }
#undef OMNI_MH
    if (check_launch() != 0) return -3;
    if (a.splits > 1) {
      decode_combine<<<dim3(a.hq, rows), 64, 0, stream>>>(a);
      if (check_launch() != 0) return -3;
    }
    return 0;
  }
  switch (a.hq / a.hk) {
    case 1: OMNI_DECODE(decode_split, 1); break;
    case 2: OMNI_DECODE(decode_split, 2); break;
    case 4: OMNI_DECODE(decode_split, 4); break;
    default: return -2;
  }
#undef OMNI_DECODE
#undef OMNI_DECODE_R
  if (check_launch() != 0) return -3;
  if (a.splits > 1) {
    decode_combine<<<dim3(a.hq, rows), 64, 0, stream>>>(a);
    if (check_launch() != 0) return -3;
  }
  return 0;
}

// ------------------------------------------------- allocation-free workspace
//
// Split partials for callers that cannot allocate (omni_qwen3_attend_noalloc):
// a file-scope device array, one copy per GPU the library runs on, held until
// the process ends. Host code never passes the array's name to a kernel (on
// the host it only stands in for the symbol); it passes the device address
// hipGetSymbolAddress returns, looked up once per device with that device
// current. Every call on one GPU shares the array, so calls that overlap on
// one GPU race. Nothing in it needs clearing: a split writes its partial
// before decode_combine reads it, and combine reads only the splits a row has.
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

int noalloc_scratch(float** ptr) {
  static std::mutex mu;
  static float* addr[kMaxDevices] = {};
  int dev = -1;
  const hipError_t drc = hipGetDevice(&dev);
  if (drc != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    g_launch_status = drc != hipSuccess ? drc : hipErrorInvalidDevice;
    return -1;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    // The first call on a device may come while the caller's stream is being
    // captured into a graph. The lookup is no stream work, but it may load
    // this library's code object onto the device, which a capture in global
    // mode refuses; relaxed mode for this thread, for the lookup only,
    // admits it without touching the capture.
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    const hipError_t mrc = hipThreadExchangeStreamCaptureMode(&mode);
    void* p = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (mrc == hipSuccess) hipThreadExchangeStreamCaptureMode(&mode);
    if (rc != hipSuccess || !p) {
      g_launch_status = rc;
      return -1;
    }
    addr[dev] = static_cast<float*>(p);
  }
  *ptr = addr[dev];
  return 0;
}

// ------------------------------------------------------------- slot copies

// lm_copy_kv (crates/omni-personaplex/kernels/lm.cu:583-593): slot dst[r] of
// one layer's cache takes the bytes of slot src[r]. A workgroup per copied
// slot, 16-byte words, slot_bytes a multiple of 16.
__global__ __launch_bounds__(256) void copy_slots_kernel(uint8_t* kv, const int32_t* src, const int32_t* dst,
                                                         int slot_bytes) {
  const int r = blockIdx.x;
  const uint4* from = reinterpret_cast<const uint4*>(kv + (int64_t)src[r] * slot_bytes);
  uint4* to = reinterpret_cast<uint4*>(kv + (int64_t)dst[r] * slot_bytes);
  for (int i = threadIdx.x; i < slot_bytes / 16; i += 256) to[i] = from[i];
}

int launch_copy_slots(void* kv, const int32_t* src, const int32_t* dst, int tokens, int slot_bytes,
                      hipStream_t stream) {
  if (tokens == 0) return 0;
  copy_slots_kernel<<<tokens, 256, 0, stream>>>(static_cast<uint8_t*>(kv), src, dst, slot_bytes);
  return check_launch();
}

// ------------------------------------------------------------------ gather

// Block per sequence i: copy its first lens[i] tokens' slots to dense rows.
// Each slot is 2 * hk * 256 bytes, copied as 16-byte words.
__global__ __launch_bounds__(256) void gather_kv_kernel(const uint4* kv, int hk, const int32_t* indptr,
                                                        const int32_t* pages, PageDiv pd, const int32_t* seq_ids,
                                                        const int32_t* lens, const int32_t* out_indptr, uint4* out) {
  const int i = blockIdx.x;
  const int s = seq_ids[i], len = lens[i];
  const int64_t words = 2LL * hk * kHead * 2 / 16;
  const int32_t* pg = pages + indptr[s];
  uint4* dst = out + (int64_t)out_indptr[i] * words;
  const int64_t total = (int64_t)len * words;
  for (int64_t w = blockIdx.y * 256 + threadIdx.x; w < total; w += (int64_t)gridDim.y * 256) {
    const int t = (int)(w / words);
    const int64_t slot = page_slot(pd, pg[page_index(pd, t)], t);
    dst[w] = kv[slot * words + (w % words)];
  }
}

int launch_gather_kv(const void* kv, int hk, const int32_t* indptr, const int32_t* pages, PageDiv pd,
                     const int32_t* seq_ids, const int32_t* lens, const int32_t* out_indptr, int nseq, void* out,
                     hipStream_t stream) {
  if (nseq == 0) return 0;
  gather_kv_kernel<<<dim3(nseq, 16), 256, 0, stream>>>(static_cast<const uint4*>(kv), hk, indptr, pages, pd,
                                                      seq_ids, lens, out_indptr, static_cast<uint4*>(out));
  return check_launch();
}

}  // namespace omni
