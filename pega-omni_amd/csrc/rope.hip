// The step before attention: rotary embedding of q and k, and the K/V scatter
// of each new row into its cache slot (gfx950, wave64).
//
//   norm_rope<MODE, STREAM>: per-head RMSNorm of q and k, half-split rotary (pair i =
//     elements i and i + 64), q in place, K and V to the row's slot. MODE
//     kPaged = qwen3_rope (crates/omni-qwen3/kernels/qwen3.cu:64-103),
//     kDense = qwen3_rope_dense (qwen3.cu:105-111), kMRope = hidream_qk_rope
//     (crates/omni-hidream-o1/kernels/hidream.cu:55-106: interleaved M-RoPE,
//     separate K and V caches).
//   lm_rope_fp8: PersonaPlex's lm_rope (crates/omni-personaplex/kernels/
//     lm.cu:125-182): interleaved rotary (pair i = elements 2i and 2i + 1) of q
//     in place and of k, then K and V quantized to FP8 E4M3 per (slot, head)
//     with scale max(amax / 448, 1e-12) into the row's 8448-byte slot.
//
// Layout of the work: one 256-thread workgroup per row (per row and group of
// 16 heads when rows are few). Its first 64 threads
// compute the row's 64 rotary angles (cos, sin) into LDS once; then each
// 16-lane DPP row takes heads grp, grp + 16, ... of the row, lane c holding
// elements 8c .. 8c + 7 (one 16-byte load and one 16-byte store). The RMS sum
// and the FP8 absmax are DPP row reductions; in the half-split rotary the
// partner of element i (< 64) is element i + 64, held by lane c + 8 in the
// same slot of its registers, one row_ror:8 DPP move away.
#include "common.h"
#include "kernels.h"
#include "rotary.h"

#include <algorithm>

namespace omni {

namespace {

constexpr int kRopeThreads = 256;
constexpr int kHeadsPerGroup = kRopeThreads / 16;

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<kQuadSwap1>(v));
  v = fmaxf(v, dpp<kQuadSwap2>(v));
  v = fmaxf(v, dpp<kRowHalfMirror>(v));
  v = fmaxf(v, dpp<kRowMirror>(v));
  return v;
}

constexpr int kPaged = 0, kDense = 1, kMRope = 2, kLm = 3;

// The row's 64 rotary angles, cos and sin, into LDS: thread i < 64 takes pair
// i. Every head of the row turns by the same angles, so they are computed once
// per row (one powf / expf and one sincosf per pair) instead of per head.
template <int MODE>
__device__ __forceinline__ void row_angles(const RopeArgs& a, int n, int p, float* s_cos, float* s_sin) {
  const int i = threadIdx.x;
  if (i < kHead / 2) {
    float ang;
    if constexpr (MODE == kLm) {
      ang = expf((float)i * a.coef) * (float)p;
    } else {
      int pe = p;
      if constexpr (MODE == kMRope) pe = a.pos[3LL * n + (i < 3 * a.mrope_hw ? i % 3 : 0)];
      ang = qwen3_angle(pe, i, a.theta);
    }
    sincosf(ang, &s_sin[i], &s_cos[i]);
  }
  __syncthreads();
}

// The streaming path (STREAM below) with its first kRopePrefetch head loads
// issued before the row's angle table is computed: their latency runs under
// the sincos work and all of them are in flight at once, where the in-place q
// stores would otherwise keep each head's load behind the previous head's
// store. Measured on qwen3_rope over config 4's 25,499 prefill rows: 102.8-103.8
// against 109.2-109.5 us per call (one box, alternating). The cached-load path keeps one head at a
// time (with the same prefetch, hidream_qk_rope over config 5's rows took
// 35.5-36.1 against 34.8-35.3 us).
constexpr int kRopePrefetch = 4;

template <int MODE>
__device__ __forceinline__ void norm_rope_stream(const RopeArgs& a) {
  const int n = blockIdx.x;
  const int c = threadIdx.x & 15, grp = threadIdx.x >> 4;
  const int nh = a.hq + 2 * a.hk;
  bf16_t* row = a.qkv + (int64_t)n * a.ld;
  const int h0 = blockIdx.y * kHeadsPerGroup + grp, hstep = kHeadsPerGroup * gridDim.y;
  uint4 pre[kRopePrefetch];
#pragma unroll
  for (int t = 0; t < kRopePrefetch; ++t)
    if (h0 + t * hstep < nh) pre[t] = ldg16_stream(row + (int64_t)(h0 + t * hstep) * kHead + 8 * c);

  int64_t slot;
  int p = 0;
  if constexpr (MODE == kDense) {
    p = a.base + n % a.per;
    slot = (int64_t)(n / a.per) * a.span + p;
  } else {
    slot = a.slots[n];
    if constexpr (MODE == kPaged) p = a.pos[n];
  }
  __shared__ float s_cos[kHead / 2], s_sin[kHead / 2];
  row_angles<MODE>(a, n, p, s_cos, s_sin);
  float cs[8], sn[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    cs[e] = s_cos[8 * (c & 7) + e];
    sn[e] = s_sin[8 * (c & 7) + e];
  }
  float w[2][8];
  widen8(ldg16(a.q_norm + 8 * c), w[0]);
  widen8(ldg16(a.k_norm + 8 * c), w[1]);
  const bool lo = c < 8;

  auto head_out = [&](int head, const uint4& raw) {
    if (head >= a.hq + a.hk) {  // V: a copy into the slot
      bf16_t* dst = MODE == kMRope ? a.v_cache + (slot * a.hk + (head - a.hq - a.hk)) * kHead
                                   : a.kv + (slot * 2 * a.hk + (head - a.hq)) * kHead;
      *reinterpret_cast<uint4*>(dst + 8 * c) = raw;
      return;
    }
    float x[8];
    widen8(raw, x);
    const bool is_q = head < a.hq;
    float ws[8], v[8], o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) ws[e] = is_q ? w[0][e] : w[1][e];
    rms_norm_head(x, ws, a.eps, v);
    rotate_half(v, cs, sn, lo, o);
    bf16_t* dst = is_q ? row + (int64_t)head * kHead
                       : (MODE == kMRope ? a.k_cache + (slot * a.hk + (head - a.hq)) * kHead
                                         : a.kv + (slot * 2 * a.hk + (head - a.hq)) * kHead);
    *reinterpret_cast<uint4*>(dst + 8 * c) = pack8(o);
  };
  // Whole DPP rows take the same trip count.
#pragma unroll
  for (int t = 0; t < kRopePrefetch; ++t)
    if (h0 + t * hstep < nh) head_out(h0 + t * hstep, pre[t]);
  for (int head = h0 + kRopePrefetch * hstep; head < nh; head += hstep)
    head_out(head, ldg16_stream(row + (int64_t)head * kHead + 8 * c));
}

// STREAM: the qkv rows are read with nontemporal loads. Worth it when they
// exceed what the device's last-level cache would hold from the producing
// kernel (measured: qwen3_rope over 313 MB of prefill rows -9%; over 107 MB
// of DiT rows the cached loads are 16% faster).
template <int MODE, bool STREAM>
__global__ __launch_bounds__(kRopeThreads) void norm_rope(RopeArgs a) {
  if constexpr (STREAM) {
    norm_rope_stream<MODE>(a);
    return;
  }
  const int n = blockIdx.x;
  const int c = threadIdx.x & 15, grp = threadIdx.x >> 4;

  int64_t slot;
  int p = 0;
  if constexpr (MODE == kDense) {
    p = a.base + n % a.per;
    slot = (int64_t)(n / a.per) * a.span + p;
  } else {
    slot = a.slots[n];
    if constexpr (MODE == kPaged) p = a.pos[n];
  }
  __shared__ float s_cos[kHead / 2], s_sin[kHead / 2];
  row_angles<MODE>(a, n, p, s_cos, s_sin);
  // Lane c's pair indices are 8 (c & 7) .. + 7, the same for every head.
  float cs[8], sn[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    cs[e] = s_cos[8 * (c & 7) + e];
    sn[e] = s_sin[8 * (c & 7) + e];
  }
  float w[2][8];
  widen8(ldg16(a.q_norm + 8 * c), w[0]);
  widen8(ldg16(a.k_norm + 8 * c), w[1]);
  const bool lo = c < 8;
  const int nh = a.hq + 2 * a.hk;
  bf16_t* row = a.qkv + (int64_t)n * a.ld;

  // Whole DPP rows take the same trip count.
  for (int head = blockIdx.y * kHeadsPerGroup + grp; head < nh; head += kHeadsPerGroup * gridDim.y) {
    const uint4 raw = STREAM ? ldg16_stream(row + (int64_t)head * kHead + 8 * c) : ldg16(row + (int64_t)head * kHead + 8 * c);
    if (head >= a.hq + a.hk) {  // V: a copy into the slot
      bf16_t* dst = MODE == kMRope ? a.v_cache + (slot * a.hk + (head - a.hq - a.hk)) * kHead
                                   : a.kv + (slot * 2 * a.hk + (head - a.hq)) * kHead;
      *reinterpret_cast<uint4*>(dst + 8 * c) = raw;
      continue;
    }
    float x[8];
    widen8(raw, x);
    const bool is_q = head < a.hq;
    float ws[8], v[8], o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) ws[e] = is_q ? w[0][e] : w[1][e];
    rms_norm_head(x, ws, a.eps, v);
    rotate_half(v, cs, sn, lo, o);
    bf16_t* dst = is_q ? row + (int64_t)head * kHead
                       : (MODE == kMRope ? a.k_cache + (slot * a.hk + (head - a.hq)) * kHead
                                         : a.kv + (slot * 2 * a.hk + (head - a.hq)) * kHead);
    *reinterpret_cast<uint4*>(dst + 8 * c) = pack8(o);
  }
}

__global__ __launch_bounds__(kRopeThreads) void lm_rope_fp8(RopeArgs a) {
  const int n = blockIdx.x;
  const int c = threadIdx.x & 15, grp = threadIdx.x >> 4;
  const int heads = a.hq;
  __shared__ float s_cos[kHead / 2], s_sin[kHead / 2];
  row_angles<kLm>(a, n, a.pos[n], s_cos, s_sin);
  // Interleaved pairs: lane c holds pairs 4c .. 4c + 3 (elements 8c .. 8c + 7).
  float cs[4], sn[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    cs[j] = s_cos[4 * c + j];
    sn[j] = s_sin[4 * c + j];
  }
  bf16_t* row = a.qkv + (int64_t)n * a.ld;
  uint8_t* slot = static_cast<uint8_t*>(a.kv_bytes) + (int64_t)a.slots[n] * a.slot_bytes;
  float* scales = reinterpret_cast<float*>(slot + 2LL * heads * kHead);

  for (int head = blockIdx.y * kHeadsPerGroup + grp; head < 3 * heads; head += kHeadsPerGroup * gridDim.y) {
    float x[8];
    widen8(ldg16(row + (int64_t)head * kHead + 8 * c), x);
    if (head < 2 * heads) {  // q or k: rotate
      rotate_interleaved<4>(x, cs, sn);
      if (head < heads) {
        *reinterpret_cast<uint4*>(row + (int64_t)head * kHead + 8 * c) = pack8(x);
        continue;
      }
    }
    // K (rotated, unrounded) or V (as read): FP8 with a per-(slot, head) scale.
    const int kv_head = head - heads;  // K heads 0 .. heads-1, then V heads
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(x[e]));
    amax = row16_max(amax);
    const float sc = e4m3_scale(amax);
    const float inv = 1.f / sc;
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] *= inv;
    *reinterpret_cast<uint2*>(slot + (int64_t)kv_head * kHead + 8 * c) = e4m3x8(x);
    if (c == 0) scales[kv_head] = sc;
  }
}

}  // namespace

int launch_rope(const RopeArgs& a, int mode, hipStream_t stream) {
  if (a.rows == 0) return 0;
  // One workgroup per row, or per (row, 16 heads) when there are few rows, so
  // that a launch still has about 1024 workgroups; each computes the row's
  // angle table.
  const int heads = mode == kRopeLm ? 3 * a.hq : a.hq + 2 * a.hk;
  const int ysplit = std::max(1, std::min((heads + kHeadsPerGroup - 1) / kHeadsPerGroup, (1024 + a.rows - 1) / a.rows));
  const dim3 grid(a.rows, ysplit);
  // Nontemporal qkv loads above 128 MiB of rows (half the MI355X's 256 MiB
  // Infinity Cache), cached loads below.
  const bool big = (int64_t)a.rows * a.ld * (int64_t)sizeof(bf16_t) > (128LL << 20);
#define OMNI_ROPE(M)                                                    \
  (big ? norm_rope<M, true><<<grid, kRopeThreads, 0, stream>>>(a)       \
       : norm_rope<M, false><<<grid, kRopeThreads, 0, stream>>>(a))
  switch (mode) {
    case kRopeQwen3: OMNI_ROPE(kPaged); break;
    case kRopeQwen3Dense: OMNI_ROPE(kDense); break;
    case kRopeHidream: OMNI_ROPE(kMRope); break;
    case kRopeLm: lm_rope_fp8<<<grid, kRopeThreads, 0, stream>>>(a); break;
    default: return -2;
  }
#undef OMNI_ROPE
  return check_launch();
}

}  // namespace omni
