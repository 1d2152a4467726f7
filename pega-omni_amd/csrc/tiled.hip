// Tiled flash attention on bf16 MFMA (gfx950) for the ragged causal prefill
// over the paged cache and the HiDream-O1 DiT attention over dense K/V.
//
// Semantics: prefill rows are qwen3_attend(ragged = 1) rows
// (crates/omni-qwen3/kernels/qwen3.cu:234-240): row n sees keys 0..pos[n] of
// sequence seq[n]. DiT rows are hidream_attend rows (crates/omni-hidream-o1/
// kernels/hidream.cu:209-347): row n sees the first *kv_len_at keys, with
// `causal` only keys 0..n; softmax in base 2 with P rounded to bf16 for P.V.
//
// A workgroup (8 waves, one per CU) owns 256 packed query rows: (256 / G positions) x (the
// G query heads of one K/V head), so one K/V tile in LDS serves G heads. Wave w
// owns packed rows 32w..32w+31. Keys stream through LDS kBN = 128 at a time, double
// buffered: global loads of tile s+1 are in flight while tile s is computed.
//
// Per wave and key tile, on v_mfma_f32_32x32x16_bf16:
//   S^T (128 keys x 32 rows) = K (128 x 128) . Q^T (128 x 32): 4 x 8 MFMAs,
//     K from LDS as the A operand, Q held in registers as the B operand.
//     In the 32x32 accumulator a lane holds one query column (lane % 32) and 16
//     keys, so the row max and sum are lane-local plus one exchange with lane ^ 32.
//   O^T (128 dims x 32 rows) += V^T (128 x 128) . P^T (128 x 32): 4 x 8 MFMAs.
//     P^T's B operand is the S accumulator itself (rounded to bf16): lane half h
//     of K-step ks holds keys 16 ks + 4 h + {0..3, 8..11}. V stays row-major in
//     LDS and the V^T operand at exactly those keys comes from two transposing
//     LDS reads (ds_read_b64_tr_b16) per MFMA.
// LDS layouts keep the MFMA operand reads conflict-free (see kTileElems).
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace omni {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBM = kTiledRows;  // packed query rows per workgroup
constexpr int kBN = 128;         // keys per tile
constexpr int kMB = kBN / 32;    // 32-key blocks per tile
constexpr int kWaves = kTiledRows / 32;  // one 32-row query block per wave
constexpr int kThreads = 64 * kWaves;
constexpr int kRowsPerWave = kBN / kWaves;  // K/V tile rows each wave loads
// LDS per buffer: the K tile then the V tile, each [128 keys][128] bf16 in
// 256-byte rows, filled straight from global memory by LDS DMA
// (buffer_load_dwordx4 ... lds for full tiles, global_load_lds_dwordx4 for the
// clamped last tile: lane l of a wave's load lands at M0 + 16 l, so one load
// fills 4 rows). The
// rows are XOR-swizzled for conflict-free operand reads on an LDS of 64 banks
// x 4 bytes; the swizzle is applied by choosing which global 16-byte chunk
// each lane loads.
//   K: 16-byte chunk c of row r sits in slot c ^ (r & 15): the 16 rows of one
//      phase of an A-operand read (ds_read_b128) hit 16 different slots.
//   V: 64-byte unit u of row r sits in unit u ^ (r & 3): the 4 rows x 64 bytes
//      of one phase of a transposing read (ds_read_b64_tr_b16) are disjoint.
constexpr int kTileElems = kBN * kHead;
// Buffer resource word 3 for raw (untyped) buffer loads on gfx9-family GPUs.
constexpr int kBufferFlags = 0x00020000;

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

// A raw buffer resource over a wave-uniform base address, `bytes` long:
// loads at offsets past it return zeros without touching memory.
__device__ __forceinline__ i32x4 buffer_rsrc(const void* base, int bytes = -1) {
  const uint64_t b = (uint64_t)base;
  return i32x4{__builtin_amdgcn_readfirstlane((int)b), __builtin_amdgcn_readfirstlane((int)(b >> 32)),
               __builtin_amdgcn_readfirstlane(bytes), kBufferFlags};
}

// LDS DMA of 16 bytes per lane into lds + 16 * lane (lds wave-uniform), issued
// from inline asm: the compiler's wait-count model cannot order an LDS DMA
// against LDS reads and falls back to lgkmcnt(0) before every LDS operand read
// while one is in flight. Out of its sight, the reads keep their partial waits;
// the kernel waits for these loads itself (vmcnt(0) before each tile barrier).
// M0 (the LDS base of a DMA) is an input operand, so the compiler sets it.
// The compiler's hazard recognizer does not see inside the asm, so the asm
// carries its own wait states: s_nop 4 (five) covers both the M0 write and a
// VALU write (v_readfirstlane) of the resource SGPRs right before the load,
// which a VMEM read of an SGPR needs five wait states after; with fewer the
// load can use a stale base address.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_void*)p;
}
__device__ __forceinline__ void dma_buffer16(i32x4 rsrc, uint32_t voff, const void* lds) {
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(rsrc), "{m0}"(lds_addr(lds))
               : "memory");
}
__device__ __forceinline__ void dma_global16(const void* src, const void* lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "{m0}"(lds_addr(lds))
               : "memory");
}
constexpr int kBufElems = 2 * kTileElems;

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives element
// i % 4 of the 8-byte chunks addressed by lanes 4 e + i / 4, e = 0..3.
__device__ __forceinline__ bf16x4 lds_read_tr(const bf16_t* p) {
  typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p));
}

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& u) { return __builtin_bit_cast(bf16x8, u); }

// Pack 8 f32 to 8 bf16 (RNE) as an MFMA operand.
__device__ __forceinline__ bf16x8 pack8(const float* v) {
  uint4 u;
  u.x = pack_bf16x2(v[0], v[1]);
  u.y = pack_bf16x2(v[2], v[3]);
  u.z = pack_bf16x2(v[4], v[5]);
  u.w = pack_bf16x2(v[6], v[7]);
  return as_bf16x8(u);
}

struct Tile {
  const bf16_t* q;    // row p of the tile at q + p * q_stride (head offset added per row)
  bf16_t* out;        // row p at out + p * hq * 128
  int nq;             // positions in the tile (<= 128 / G)
  int len;            // keys of the source
  int last;           // keys any row of the tile sees
  int qpos0;          // DiT: position of row 0 (causal rule n sees 0..n)
  const int32_t* pos; // prefill: positions of the tile's rows
  // key sources
  const bf16_t* kbase;
  const bf16_t* vbase;
  int64_t kv_stride;         // dense: elements between keys
  const int32_t* pg;         // paged: the sequence's pages
  int64_t per_slot;          // paged: elements per slot
};

template <int G, bool PAGED, bool HALVES = false, bool EXACT = false>
__global__ __launch_bounds__(kThreads, 1) void tiled_attn(TiledArgs a, int items, int ntiles) {
  // DiT, XCD-aware order: workgroup id i runs on XCD i % 8; give each XCD a
  // contiguous block of work items so the tiles sharing one K/V head (and
  // batch) share that XCD's L2.
  // Prefill: the work list gives each XCD a range of (tile, kv head) items,
  // ordered so the workgroups resident on an XCD share one (sequence, kv
  // head) and its K/V stays in that XCD's L2; workgroup i takes item
  // start[i % 8] + i / 8 of its XCD's range.
  // DiT tail split: the first split_from items run whole, then every later
  // item runs as split_k key chunks (workgroups dispatched after all whole
  // items, so they fill the last round), each with its own XCD-aware order.
  // DiT row halves (HALVES): the last `halved` items run as two workgroups
  // of kBM / 2 packed rows, in the same order as the split chunks; waves
  // 0..3 (one per SIMD) compute the first half, waves 4..7 the second, and
  // all eight load the K/V tiles.
  int idx, chunk = -1, half = -1;
  if constexpr (HALVES) {
    const int halves_from = items - a.halved;
    const int whole8 = ((halves_from + 7) >> 3) << 3;
    if ((int)blockIdx.x < whole8) {
      const int per = whole8 >> 3;
      idx = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
      if (idx >= halves_from) return;
    } else {
      const int b2 = blockIdx.x - whole8;
      const int units = a.halved * 2;
      const int per = (units + 7) >> 3;
      const int u = (b2 & 7) * per + (b2 >> 3);
      if (u >= units) return;
      idx = halves_from + (u >> 1);
      half = u & 1;
    }
  } else if (!PAGED && a.split_k > 0) {
    const int whole8 = ((a.split_from + 7) >> 3) << 3;
    if ((int)blockIdx.x < whole8) {
      const int per = whole8 >> 3;
      idx = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
      if (idx >= a.split_from) return;
    } else {
      const int b2 = blockIdx.x - whole8;
      const int units = (items - a.split_from) * a.split_k;
      const int per = (units + 7) >> 3;
      const int u = (b2 & 7) * per + (b2 >> 3);
      if (u >= units) return;
      idx = a.split_from + u / a.split_k;
      chunk = u % a.split_k;
    }
  } else if (PAGED) {
    const int x = blockIdx.x & 7;
    idx = a.work[x] + (int)(blockIdx.x >> 3);
    if (idx >= a.work[x + 1]) return;
  } else {
    const int per = (items + 7) >> 3;
    idx = (int)((blockIdx.x & 7) * per + (blockIdx.x >> 3));
    if (idx >= items) return;
  }
  const int32_t* item = PAGED ? a.work + kPrefillWorkHeader + 4 * idx : nullptr;
  const int tile = PAGED ? 0 : idx % ntiles;
  const int kvh = PAGED ? item[3] : (idx / ntiles) % a.hk;
  const int b = PAGED ? 0 : idx / (ntiles * a.hk);
  constexpr int kPos = kBM / G;  // positions per tile

  Tile t;
  if constexpr (PAGED) {
    const int s = item[0], first = item[1];
    t.nq = item[2];
    t.pos = a.pos + first;
    t.q = a.q + (int64_t)first * a.q_stride;
    t.out = a.out + (int64_t)first * a.hq * kHead;
    t.last = t.pos[t.nq - 1] + 1;
    t.len = t.last;
    t.pg = a.pages + a.indptr[s];
    t.per_slot = 2LL * a.hk * kHead;
    t.kbase = a.kv + (int64_t)kvh * kHead;
    t.vbase = a.kv + (int64_t)(a.hk + kvh) * kHead;
    t.qpos0 = 0;
  } else {
    const int q0 = tile * kPos;
    t.nq = min(kPos, a.q_len - q0);
    t.q = a.q + b * a.q_bstride + (int64_t)q0 * a.q_stride;
    t.out = a.out + b * a.out_bstride + (int64_t)q0 * a.hq * kHead;
    t.len = *a.kv_len_at;
    // A half's rows end at position (kBM / 2) (half + 1) / G of the tile.
    const int np = half < 0 ? t.nq : min(t.nq, (kBM / 2) * (half + 1) / G);
    if (half > 0 && (kBM / 2) * half / G >= t.nq) return;  // a second half with no rows
    t.last = a.causal ? min(t.len, q0 + np) : t.len;
    t.qpos0 = q0;
    t.kv_stride = (int64_t)a.hk * kHead;
    t.kbase = a.k + b * a.kv_bstride + (int64_t)kvh * kHead;
    t.vbase = a.v + b * a.kv_bstride + (int64_t)kvh * kHead;
  }

  // Two tile buffers (K tile, then V tile), separate objects so the compiler
  // can see that loads landing in one never alias reads of the other.
  __shared__ __align__(16) bf16_t smem0[kBufElems];
  __shared__ __align__(16) bf16_t smem1[kBufElems];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;

  // This lane's query column: packed row r = 32 wave + j.
  const int r = wave * 32 + j;
  const int p = r / G, head = kvh * G + r % G;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  // Waves outside this workgroup's half, and waves none of whose 32 rows is a
  // position of the tile (a short last tile), only load K/V tiles and meet
  // the barriers (wave-uniform).
  const bool active = (half < 0 || (wave_u >> 2) == half) && (32 * wave_u) / G < t.nq;
  const bool row_ok = p < t.nq && active;
  int lim;  // keys this row sees
  if constexpr (PAGED)
    lim = row_ok ? t.pos[p] + 1 : 0;
  else
    lim = row_ok ? (a.causal ? min(t.len, t.qpos0 + p + 1) : t.len) : 0;

  // Q^T as the B operand: K-step kk holds dims 16 kk + 8 h .. + 7 of row r.
  bf16x8 qf[8];
  {
    const bf16_t* qp = t.q + (int64_t)(row_ok ? p : 0) * a.q_stride + (int64_t)head * kHead + 8 * h;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      uint4 u = ldg16(qp + 16 * kk);  // rows past the tile read row 0, then become zero
      if (!row_ok) u = make_uint4(0, 0, 0, 0);
      qf[kk] = as_bf16x8(u);
    }
    // Q is loaded once: wait for it here, so the key loop's first MFMA does
    // not wait on the next tile's prefetch (vmcnt(0), other counters free).
    __builtin_amdgcn_s_waitcnt(0x0F70);
  }

  // Loader: wave w fills rows kRowsPerWave w .. of the K and V tiles, four
  // rows per load; lane l takes row kRowsPerWave w + 4 i + l / 16 and LDS
  // slot l % 16.
  // Keys past `last` repeat the last key (their scores are masked).
  // Dense sources: within a full tile a lane's rows and chunks are fixed, so
  // its element offsets from the tile's first key are constants (32-bit) and a
  // tile adds one uniform base: loads take a scalar base and a vector offset.
  // Paged sources with a page that is a multiple of kRowsPerWave: a wave's
  // rows of a tile are consecutive keys of one page, so a tile needs one
  // (scalar) page id per wave, read a tile ahead, and the rows are
  // consecutive slots.
  const bool page_wave = PAGED && a.pd.page % kRowsPerWave == 0;
  // Element offsets of this lane's rows from the first row of the wave's
  // block (dense: from the tile's first key): constants for every tile.
  uint32_t koff[kRowsPerWave / 4], voff[kRowsPerWave / 4];
  {
    const int64_t stride = PAGED ? t.per_slot : t.kv_stride;
#pragma unroll
    for (int i = 0; i < kRowsPerWave / 4; ++i) {
      const int wrow = 4 * i + (lane >> 4);  // row within the wave's block
      const int row = kRowsPerWave * wave_u + wrow;
      const int cs = lane & 15;
      const int kc = cs ^ (row & 15);
      const int vc = (((cs >> 2) ^ (row & 3)) << 2) | (cs & 3);
      const int64_t r0 = PAGED ? wrow : row;
      koff[i] = (uint32_t)(r0 * stride + 8 * kc);
      voff[i] = (uint32_t)(r0 * stride + 8 * vc);
    }
  }
  // Page id of this wave's rows of the tile at key n (page_wave only).
  // Loaded as a vector load a tile before use and made scalar only then, so
  // reading it does not wait for the tile loads issued in between.
  const __amdgpu_buffer_rsrc_t pg_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(PAGED ? (void*)t.pg : nullptr, 0, -1, kBufferFlags);
  auto wave_page = [&](int n) -> int {
    const int i = page_index(a.pd, __builtin_amdgcn_readfirstlane(min(n + kRowsPerWave * wave_u, t.last - 1)));
    return __builtin_amdgcn_raw_buffer_load_b32(pg_rsrc, 0, 4 * i, 0);
  };
  int next_pid = 0;  // page id for the next tile to issue (page_wave), per lane
  auto issue_tile = [&](int n0, bf16_t* kd) {
    bf16_t* vd = kd + kTileElems;
    if (!PAGED || page_wave) {
      // Rows past `last` (the key tile's tail) fall outside the buffer
      // range and read as zeros: masked scores and zero V rows, so they add
      // nothing, and no slot past the sequence's keys is read.
      const bf16_t* kb;
      const bf16_t* vb;
      const int first = PAGED ? n0 + kRowsPerWave * wave_u : n0;  // key of this lane's row 0
      const int rows = min(max(t.last - first, 0), PAGED ? kRowsPerWave : kBN);
      const int64_t stride_bytes = 2 * (PAGED ? t.per_slot : t.kv_stride);
      const int bytes = rows == (PAGED ? kRowsPerWave : kBN) ? -1 : (int)(rows * stride_bytes);
      if constexpr (PAGED) {
        const int64_t slot0 = page_slot(a.pd, __builtin_amdgcn_readfirstlane(next_pid), n0 + kRowsPerWave * wave_u);
        kb = t.kbase + slot0 * t.per_slot;
        vb = t.vbase + slot0 * t.per_slot;
      } else {
        kb = t.kbase + (int64_t)n0 * t.kv_stride;
        vb = t.vbase + (int64_t)n0 * t.kv_stride;
      }
      // Buffer loads to LDS: the tile's base in a scalar resource, the
      // lane's constant byte offsets in VGPRs, no per-lane address math.
      const i32x4 kr = buffer_rsrc(kb, bytes), vr = buffer_rsrc(vb, bytes);
#pragma unroll
      for (int i = 0; i < kRowsPerWave / 4; ++i) {
        const int lrow = (kRowsPerWave * wave_u + 4 * i) * kHead;
        dma_buffer16(kr, 2 * koff[i], kd + lrow);
        dma_buffer16(vr, 2 * voff[i], vd + lrow);
      }
      return;
    }
    // Offsets first, then the loads (the paged offsets need the page ids).
    int64_t koffs[kRowsPerWave / 4], voffs[kRowsPerWave / 4];
#pragma unroll
    for (int i = 0; i < kRowsPerWave / 4; ++i) {
      const int row = kRowsPerWave * wave_u + 4 * i + (lane >> 4);
      const int key = min(n0 + row, t.last - 1);
      const int cs = lane & 15;
      const int kc = cs ^ (row & 15);
      const int vc = (((cs >> 2) ^ (row & 3)) << 2) | (cs & 3);
      int64_t off;
      if constexpr (PAGED) {
        off = page_slot(a.pd, t.pg[page_index(a.pd, key)], key) * t.per_slot;
      } else {
        off = (int64_t)key * t.kv_stride;
      }
      koffs[i] = off + 8 * kc;
      voffs[i] = off + 8 * vc;
    }
#pragma unroll
    for (int i = 0; i < kRowsPerWave / 4; ++i) {
      const int lrow = (kRowsPerWave * wave_u + 4 * i) * kHead;
      dma_global16(t.kbase + koffs[i], kd + lrow);
      dma_global16(t.vbase + voffs[i], vd + lrow);
    }
  };

  f32x16 o[4];
#pragma unroll
  for (int md = 0; md < 4; ++md)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[md][e] = 0.f;
  float m = -INFINITY, l = 0.f;
  const float sl2 = a.scale_log2;

  // Per-lane LDS bases (elements). S's A operand: K row 32 mb + j, chunk
  // 2 kk + h, in slot (2 kk + h) ^ (j & 15): elem = (k_lane ^ 16 kk) + 4096 mb.
  // P.V's A operand (V^T, 32 dims x 16 keys of K-step ks) is two transposing
  // reads, keys 16 ks + 8 q + 4 h + {0..3} (q = 0, 1): lane i of 16-lane group
  // g addresses V row 16 ks + 8 q + 4 (g / 2) + i / 4 at dims
  // 32 md + 16 (g % 2) + 4 (i % 4) (unit md of a row with row % 4 = i / 4),
  // and receives dim 32 md + j of those 4 keys: elem = (v_lane ^ 32 md) +
  // (16 ks + 8 q) * 128.
  const int k_lane = j * kHead + 8 * (h ^ (j & 15));
  const int vg = lane >> 4, vi = lane & 15;
  const int v_lane = (4 * (vg >> 1) + (vi >> 2)) * kHead + 32 * (vi >> 2) + 16 * (vg & 1) + 4 * (vi & 3);

  // Key tiles [s_lo, s_hi): all of them, or this chunk's share.
  const int steps = (t.last + kBN - 1) / kBN;
  const int s_lo = chunk < 0 ? 0 : chunk * steps / a.split_k;
  const int s_hi = chunk < 0 ? steps : (chunk + 1) * steps / a.split_k;
  if (page_wave && s_hi > s_lo) next_pid = wave_page(s_lo * kBN);
  if (s_hi > s_lo) issue_tile(s_lo * kBN, smem0);
  if (page_wave && s_lo + 1 < s_hi) next_pid = wave_page((s_lo + 1) * kBN);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the first tile is in LDS
  __syncthreads();
  // One key tile: start loading the next tile into `nxt`, compute from `cur`.
  auto tile_step = [&](int st, const bf16_t* cur, bf16_t* nxt) {
    const int n0 = st * kBN;
    if (st + 1 < s_hi) issue_tile(n0 + kBN, nxt);  // lands while this tile computes
    if (page_wave && st + 2 < s_hi) next_pid = wave_page(n0 + 2 * kBN);  // a tile ahead
    const bf16_t* kt = cur;
    const bf16_t* vt = cur + kTileElems;  // V tile

    // S^T = K . Q^T for keys n0 .. n0 + kBN - 1: kMB interleaved MFMA chains
    // (32-key blocks mb) over the 8 K-steps, with the K fragments read
    // from LDS two K-steps ahead of use; the stages are pinned in this order.
    f32x16 sc[kMB];
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) sc[mb][e] = 0.f;
    uint4 kf[8][kMB];
    auto read_k = [&](int kk) {
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb) kf[kk][mb] = *reinterpret_cast<const uint4*>(kt + (k_lane ^ (16 * kk)) + mb * 4096);
    };
    read_k(0);
    read_k(1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb)
        sc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kf[kk][mb]), qf[kk], sc[mb], 0, 0, 0);
      if (kk + 2 < 8) read_k(kk + 2);
      __builtin_amdgcn_sched_barrier(0);
    }

    // Register e of block mb is key n0 + 32 mb + 8 (e / 4) + 4 h + e % 4.
    if (__any(n0 + kBN > lim)) {
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (n0 + 32 * mb + 8 * (e >> 2) + 4 * h + (e & 3) >= lim) sc[mb][e] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, sc[mb][e]);
    {  // lanes l and l ^ 32 hold the two halves of the row's keys
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    }
    // The running base m moves only when the max grows by more than 8 (log2):
    // p = 2^(s - m) <= 2^8 stays exact in f32 and l, O share the same base,
    // so the result is unchanged while most tiles skip rescaling O.
    const float mt = mx * sl2;
    const bool grow = mt > m + 8.f;
    if (__any(grow)) {
      const float alpha = grow ? fast_exp2(m - mt) : 1.f;
      m = grow ? mt : m;
      l *= alpha;
#pragma unroll
      for (int md = 0; md < 4; ++md)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[md][e] *= alpha;
    }
    const float base = m == -INFINITY ? 0.f : m;
    float psum = 0.f;
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        sc[mb][e] = fast_exp2(fmaf(sc[mb][e], sl2, -base));
        psum += sc[mb][e];
      }
    l += psum;

    // O^T += V^T . P^T: K-step ks covers keys 16 ks + 4 h + {0..3, 8..11}.
#pragma unroll
    for (int ks_ = 0; ks_ < 2 * kMB; ++ks_) {
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = sc[ks_ >> 1][8 * (ks_ & 1) + e];
      const bf16x8 pf = pack8(pv);
      // EXACT: P = P_hi + P_lo, both bf16 (P_lo = bf16(P - P_hi), P - P_hi
      // exact in f32), and P.V as two MFMAs: P carries 16 significant bits
      // into the accumulation instead of 8.
      bf16x8 pfl;
      if constexpr (EXACT) {
        float pl[8];
        widen8(__builtin_bit_cast(uint4, pf), pl);
#pragma unroll
        for (int e = 0; e < 8; ++e) pl[e] = pv[e] - pl[e];
        pfl = pack8(pl);
      }
#pragma unroll
      for (int md = 0; md < 4; ++md) {
        const bf16_t* vb = vt + (v_lane ^ (32 * md)) + 16 * ks_ * kHead;
        const bf16x4 lo = lds_read_tr(vb);
        const bf16x4 hi = lds_read_tr(vb + 8 * kHead);
        const bf16x8 vf = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        o[md] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, o[md], 0, 0, 0);
        if constexpr (EXACT) o[md] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pfl, o[md], 0, 0, 0);
      }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the next tile has landed
    __syncthreads();
  };
  // A wave that computes nothing: the same loads (its rows of every K/V
  // tile, with the page ids a tile ahead) and barriers.
  auto load_step = [&](int st, bf16_t* nxt) {
    if (st + 1 < s_hi) issue_tile((st + 1) * kBN, nxt);
    if (page_wave && st + 2 < s_hi) next_pid = wave_page((st + 2) * kBN);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
  };
  if (!active) {
    for (int st = s_lo; st < s_hi; st += 2) {
      load_step(st, smem1);
      if (st + 1 < s_hi) load_step(st + 1, smem0);
    }
    return;
  }
  for (int st = s_lo; st < s_hi; st += 2) {
    tile_step(st, smem0, smem1);
    if (st + 1 < s_hi) tile_step(st + 1, smem1, smem0);
  }

  // Register e of block md is dim 32 md + 8 (e / 4) + 4 h + e % 4.
  l += xor_lane(l, 32);
  if (chunk >= 0) {  // a chunk's partial: unnormalised O with its base m and sum l, for dit_combine
    if (!row_ok) return;  // dit_combine reads the tile's positions only
    float* seg = a.ws + (int64_t)((idx - a.split_from) * a.split_k + chunk) * (kBM * (kHead + 2));
#pragma unroll
    for (int md = 0; md < 4; ++md)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
        *reinterpret_cast<float4*>(seg + r * kHead + 32 * md + 8 * q4 + 4 * h) =
            make_float4(o[md][4 * q4], o[md][4 * q4 + 1], o[md][4 * q4 + 2], o[md][4 * q4 + 3]);
    if (h == 0) *reinterpret_cast<float2*>(seg + kBM * kHead + 2 * r) = make_float2(m, l);
    return;
  }
  // Normalise and store. A row that sees no key (*kv_len_at = 0) has l = 0 and
  // O = 0, and stores 0 * (1 / 0) = NaN, as hidream.cu:333-346 does.
  if (!row_ok) return;
  const float inv = 1.f / l;
  bf16_t* dst = t.out + ((int64_t)p * a.hq + head) * kHead;
#pragma unroll
  for (int md = 0; md < 4; ++md)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = 32 * md + 8 * q4 + 4 * h;
      uint2 w;
      w.x = pack_bf16x2(o[md][4 * q4 + 0] * inv, o[md][4 * q4 + 1] * inv);
      w.y = pack_bf16x2(o[md][4 * q4 + 2] * inv, o[md][4 * q4 + 3] * inv);
      *reinterpret_cast<uint2*>(dst + d) = w;
    }
}

// Merge the split_k chunk partials of each split DiT item into its output
// rows: one workgroup per (item, 16 packed rows), 16 threads per row, 8 dims
// each (two 16-byte partial loads per chunk). Two passes over the chunks, the
// row's max base, then the weighted sums, each issuing the loads of
// kCombineBatch chunks before using them (clamped to the last chunk, the
// extra ones unused), so a pass costs one memory round trip per batch rather
// than one per chunk.
constexpr int kCombineRows = 16;
constexpr int kCombineBatch = 8;

__global__ __launch_bounds__(256) void dit_combine(TiledArgs a, int ntiles) {
  const int idx = a.split_from + blockIdx.x;
  const int G = a.hq / a.hk, kpos = kBM / G;
  const int tile = idx % ntiles, kvh = (idx / ntiles) % a.hk, b = idx / (ntiles * a.hk);
  const int q0 = tile * kpos, nq = min(kpos, a.q_len - q0);
  const int r = blockIdx.y * kCombineRows + (threadIdx.x >> 4), d0 = 8 * (threadIdx.x & 15);
  const int p = r / G, head = kvh * G + r % G;
  if (p >= nq) return;
  constexpr int kSeg = kBM * (kHead + 2);
  const int nk = a.split_k;
  const float* seg0 = a.ws + (int64_t)(blockIdx.x * nk) * kSeg;
  const float* ml0 = seg0 + kBM * kHead + 2 * r;  // chunk c's (m, l) at ml0 + c * kSeg
  float top = -INFINITY;
  for (int c0 = 0; c0 < nk; c0 += kCombineBatch) {
    float m[kCombineBatch];
#pragma unroll
    for (int i = 0; i < kCombineBatch; ++i) m[i] = ml0[min(c0 + i, nk - 1) * kSeg];
#pragma unroll
    for (int i = 0; i < kCombineBatch; ++i) top = fmaxf(top, m[i]);  // a repeated chunk changes no max
  }
  float num[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float den = 0.f;
  for (int c0 = 0; c0 < nk; c0 += kCombineBatch) {
    float2 ml[kCombineBatch];
    float4 v0[kCombineBatch], v1[kCombineBatch];
#pragma unroll
    for (int i = 0; i < kCombineBatch; ++i) {
      const float* seg = seg0 + min(c0 + i, nk - 1) * kSeg;
      ml[i] = *reinterpret_cast<const float2*>(seg + kBM * kHead + 2 * r);
      v0[i] = *reinterpret_cast<const float4*>(seg + r * kHead + d0);
      v1[i] = *reinterpret_cast<const float4*>(seg + r * kHead + d0 + 4);
    }
#pragma unroll
    for (int i = 0; i < kCombineBatch; ++i) {
      if (c0 + i >= nk) break;
      const float w = ml[i].x == -INFINITY ? 0.f : fast_exp2(ml[i].x - top);
      den = fmaf(ml[i].y, w, den);
      num[0] = fmaf(v0[i].x, w, num[0]);
      num[1] = fmaf(v0[i].y, w, num[1]);
      num[2] = fmaf(v0[i].z, w, num[2]);
      num[3] = fmaf(v0[i].w, w, num[3]);
      num[4] = fmaf(v1[i].x, w, num[4]);
      num[5] = fmaf(v1[i].y, w, num[5]);
      num[6] = fmaf(v1[i].z, w, num[6]);
      num[7] = fmaf(v1[i].w, w, num[7]);
    }
  }
  // den = 0 only when no chunk saw a key: NaN, as the unsplit kernel stores.
  const float inv = 1.f / den;
  uint4 o;
  o.x = pack_bf16x2(num[0] * inv, num[1] * inv);
  o.y = pack_bf16x2(num[2] * inv, num[3] * inv);
  o.z = pack_bf16x2(num[4] * inv, num[5] * inv);
  o.w = pack_bf16x2(num[6] * inv, num[7] * inv);
  *reinterpret_cast<uint4*>(a.out + b * a.out_bstride + ((int64_t)(q0 + p) * a.hq + head) * kHead + d0) = o;
}

// Prefill with exact_p set: the hi + lo P.V variant (prefill only; DiT rounds
// P to bf16 as hidream.cu does). Returns whether it launched.
template <int G, bool PAGED>
bool launch_exact(const TiledArgs& a, int grid, int items, int ntiles, hipStream_t stream) {
  if constexpr (PAGED) {
    if (a.exact_p) {
      tiled_attn<G, true, false, true><<<grid, kThreads, 0, stream>>>(a, items, ntiles);
      return true;
    }
  }
  return false;
}

template <bool PAGED>
int launch_tiled(const TiledArgs& a, int items, int ntiles, hipStream_t stream) {
  if (items <= 0) return 0;
  int grid = ((items + 7) >> 3) << 3;
  if (!PAGED && a.split_k > 0)
    grid = (((a.split_from + 7) >> 3) << 3) + ((((items - a.split_from) * a.split_k + 7) >> 3) << 3);
  const bool halves = !PAGED && a.split_k == 0 && a.halved > 0;
  if (halves) grid = (((items - a.halved + 7) >> 3) << 3) + (((a.halved * 2 + 7) >> 3) << 3);
  switch (a.hq / a.hk) {
#define OMNI_CASE(G)                                                                       \
  case G:                                                                                  \
    if (halves)                                                                            \
      tiled_attn<G, false, true><<<grid, kThreads, 0, stream>>>(a, items, ntiles);         \
    else if (!launch_exact<G, PAGED>(a, grid, items, ntiles, stream))                      \
      tiled_attn<G, PAGED><<<grid, kThreads, 0, stream>>>(a, items, ntiles);               \
    break;
    OMNI_CASE(1)
    OMNI_CASE(2)
    OMNI_CASE(4)
    OMNI_CASE(8)
#undef OMNI_CASE
    default: return -2;
  }
  if (check_launch() != 0) return -3;
  if (!PAGED && a.split_k > 0) {
    dit_combine<<<dim3(items - a.split_from, kBM / kCombineRows), 256, 0, stream>>>(a, ntiles);
    return check_launch();
  }
  return 0;
}

int launch_prefill(const TiledArgs& a, int workgroups, hipStream_t stream) {
  return launch_tiled<true>(a, workgroups, 0, stream);
}

int launch_dit(const TiledArgs& a, int batch, hipStream_t stream) {
  const int G = a.hq / a.hk;
  if (G <= 0 || kBM % G != 0) return -2;
  const int ntiles = (a.q_len + kBM / G - 1) / (kBM / G);
  const long long items = (long long)ntiles * a.hk * batch;
  if (items > (1LL << 30)) return -2;
  if (a.halved < 0 || a.halved > items || a.halved > (1 << 29)) return -2;
  return launch_tiled<false>(a, (int)items, ntiles, stream);
}

// Without a workspace: when the last round holds at most half the resident
// workgroups, its items run as row halves (two workgroups each, on twice the
// CUs); with one computing wave per SIMD such a round takes about 0.7 of a
// full round's time.
int dit_halves(const TiledArgs& a, int batch, int resident) {
  const int G = a.hq / a.hk;
  const int ntiles = (a.q_len + kBM / G - 1) / (kBM / G);
  const long long n = (long long)ntiles * a.hk * batch;
  if (resident <= 0 || n <= 0 || n > (1LL << 30)) return 0;
  const int rem = (int)(n % resident);
  return 2 * rem > resident ? 0 : rem;
}

// With `resident` workgroups in flight (one per CU), items - items % resident
// run whole and the rest each split into resident / (items % resident) key
// chunks, so the last round is full instead of a fraction; but no chunk of
// fewer than kMinChunkTiles key tiles, counted on q_len (the key count is on
// the device; DiT attends over about as many keys as queries): a shorter chunk
// is mostly prologue and partial writes, and every chunk is one more partial
// for dit_combine to merge.
constexpr int kMinChunkTiles = 4;

void dit_split(const TiledArgs& a, int batch, int resident, int* items, int* split_from, int* split_k) {
  const int G = a.hq / a.hk;
  const int ntiles = (a.q_len + kBM / G - 1) / (kBM / G);
  const long long n = (long long)ntiles * a.hk * batch;
  *items = (int)n;
  *split_from = (int)n;
  *split_k = 0;
  if (resident <= 0 || n <= 0 || n > (1LL << 30)) return;
  const int rem = (int)(n % resident);
  if (rem == 0 || resident / rem < 2) return;
  const int chunks = std::min(resident / rem, std::max(2, (a.q_len + kBN - 1) / kBN / kMinChunkTiles));
  *split_from = (int)n - rem;
  *split_k = chunks;
}

}  // namespace omni
