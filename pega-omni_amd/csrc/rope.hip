// The step before attention: rotary embedding of q and k, and the K/V scatter
// of each new row into its cache slot (gfx950, wave64).
//
//   norm_rope<MODE>: per-head RMSNorm of q and k, half-split rotary (pair i =
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
// Layout of the work: a 16-lane DPP row owns one 128-element head, lane c
// holding elements 8c .. 8c + 7 (one 16-byte load and one 16-byte store), so a
// 256-thread workgroup covers 16 heads of one row. The RMS sum and the FP8
// absmax are DPP row reductions; in the half-split rotary the partner of
// element i (< 64) is element i + 64, held by lane c + 8 in the same slot of
// its registers, one row_ror:8 DPP move away.
#include "common.h"
#include "kernels.h"

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

__device__ __forceinline__ uint4 pack8(const float* v) {
  return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                    pack_bf16x2(v[6], v[7]));
}

__device__ __forceinline__ float round_bf16(float v) { return __uint_as_float(f2bf(v) << 16); }

// Eight f32 to FP8 E4M3 (OCP, round to nearest even) on v_cvt_pk_fp8_f32.
// Callers pass values already scaled into [-448, 448].
__device__ __forceinline__ uint2 e4m3x8(const float* v) {
  int lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false);
  lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], lo, true);
  int hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[4], v[5], 0, false);
  hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[6], v[7], hi, true);
  return make_uint2((uint32_t)lo, (uint32_t)hi);
}

constexpr int kPaged = 0, kDense = 1, kMRope = 2;

template <int MODE>
__global__ __launch_bounds__(kRopeThreads) void norm_rope(RopeArgs a) {
  const int n = blockIdx.x;
  const int c = threadIdx.x & 15;
  const int head = blockIdx.y * kHeadsPerGroup + (threadIdx.x >> 4);
  if (head >= a.hq + 2 * a.hk) return;  // whole DPP rows leave together
  bf16_t* row = a.qkv + (int64_t)n * a.ld + (int64_t)head * kHead;
  const uint4 raw = ldg16(row + 8 * c);

  int64_t slot;
  int p = 0;
  if constexpr (MODE == kDense) {
    p = a.base + n % a.per;
    slot = (int64_t)(n / a.per) * a.span + p;
  } else {
    slot = a.slots[n];
    if constexpr (MODE == kPaged) p = a.pos[n];
  }

  if (head >= a.hq + a.hk) {  // V: a copy into the slot
    bf16_t* dst = MODE == kMRope ? a.v_cache + (slot * a.hk + (head - a.hq - a.hk)) * kHead
                                 : a.kv + (slot * 2 * a.hk + (head - a.hq)) * kHead;
    *reinterpret_cast<uint4*>(dst + 8 * c) = raw;
    return;
  }

  float x[8];
  widen8(raw, x);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
  const float r = rsqrtf(row16_sum(ss) / kHead + a.eps);
  const bool is_q = head < a.hq;
  float w[8];
  widen8(ldg16((is_q ? a.q_norm : a.k_norm) + 8 * c), w);
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = round_bf16(x[e] * r) * w[e];

  const bool lo = c < 8;
  const int32_t* p3 = MODE == kMRope ? a.pos + 3LL * n : nullptr;
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float partner = dpp<kRowRor8>(v[e]);
    const int i = 8 * (c & 7) + e;  // rotary pair index
    int pe = p;
    if constexpr (MODE == kMRope) pe = p3[i < 3 * a.mrope_hw ? i % 3 : 0];
    const float inv_freq = 1.f / powf(a.theta, (float)(2 * i) / kHead);
    float sn, cs;
    sincosf((float)pe * inv_freq, &sn, &cs);
    o[e] = lo ? v[e] * cs - partner * sn : v[e] * cs + partner * sn;
  }
  bf16_t* dst = is_q ? row
                     : (MODE == kMRope ? a.k_cache + (slot * a.hk + (head - a.hq)) * kHead
                                       : a.kv + (slot * 2 * a.hk + (head - a.hq)) * kHead);
  *reinterpret_cast<uint4*>(dst + 8 * c) = pack8(o);
}

__global__ __launch_bounds__(kRopeThreads) void lm_rope_fp8(RopeArgs a) {
  const int n = blockIdx.x;
  const int c = threadIdx.x & 15;
  const int heads = a.hq;
  const int head = blockIdx.y * kHeadsPerGroup + (threadIdx.x >> 4);
  if (head >= 3 * heads) return;
  bf16_t* row = a.qkv + (int64_t)n * a.ld + (int64_t)head * kHead;
  float x[8];
  widen8(ldg16(row + 8 * c), x);

  if (head < 2 * heads) {  // q or k: interleaved rotary, pairs i = 4c .. 4c + 3
    const float p = (float)a.pos[n];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float freq = expf((float)(4 * c + j) * a.coef);
      float sn, cs;
      sincosf(freq * p, &sn, &cs);
      const float re = x[2 * j], im = x[2 * j + 1];
      x[2 * j] = re * cs - im * sn;
      x[2 * j + 1] = re * sn + im * cs;
    }
    if (head < heads) {
      *reinterpret_cast<uint4*>(row + 8 * c) = pack8(x);
      return;
    }
  }
  // K (rotated, unrounded) or V (as read): FP8 with a per-(slot, head) scale.
  const int kv_head = head - heads;  // K heads 0 .. heads-1, then V heads
  float amax = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(x[e]));
  amax = row16_max(amax);
  const float sc = fmaxf(amax * (1.f / 448.f), 1e-12f);
  const float inv = 1.f / sc;
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] *= inv;
  uint8_t* slot = static_cast<uint8_t*>(a.kv_bytes) + (int64_t)a.slots[n] * a.slot_bytes;
  *reinterpret_cast<uint2*>(slot + (int64_t)kv_head * kHead + 8 * c) = e4m3x8(x);
  if (c == 0) reinterpret_cast<float*>(slot + 2LL * heads * kHead)[kv_head] = sc;
}

}  // namespace

int launch_rope(const RopeArgs& a, int mode, hipStream_t stream) {
  if (a.rows == 0) return 0;
  const int heads = mode == kRopeLm ? 3 * a.hq : a.hq + 2 * a.hk;
  const dim3 grid(a.rows, (heads + kHeadsPerGroup - 1) / kHeadsPerGroup);
  switch (mode) {
    case kRopeQwen3: norm_rope<kPaged><<<grid, kRopeThreads, 0, stream>>>(a); break;
    case kRopeQwen3Dense: norm_rope<kDense><<<grid, kRopeThreads, 0, stream>>>(a); break;
    case kRopeHidream: norm_rope<kMRope><<<grid, kRopeThreads, 0, stream>>>(a); break;
    case kRopeLm: lm_rope_fp8<<<grid, kRopeThreads, 0, stream>>>(a); break;
    default: return -2;
  }
  return check_launch();
}

}  // namespace omni
