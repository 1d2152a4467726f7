// Rotary and cache-write helpers shared by the rotary + scatter kernels
// (rope.hip) and the fused rotary + decode attention (decode.hip), so that
// both produce the same bits for the same row. Qwen3: a head is held by one
// 16-lane DPP row, lane c holding elements 8c .. 8c + 7.
#pragma once
#include "common.h"

namespace omni {

__device__ __forceinline__ float round_bf16(float v) { return __uint_as_float(f2bf(v) << 16); }

__device__ __forceinline__ uint4 pack8(const float* v) {
  return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                    pack_bf16x2(v[6], v[7]));
}

// Angle of rotary pair i (elements i and i + 64) at position p:
// p * theta^(-2i / 128) (crates/omni-qwen3/kernels/qwen3.cu:64-103).
__device__ __forceinline__ float qwen3_angle(int p, int i, float theta) {
  return (float)p * (1.f / powf(theta, (float)(2 * i) / kHead));
}

// Per-head RMSNorm times the weight w: x / rms rounded to bf16, then scaled
// by w (the reference rounds the normalised value before the weight).
__device__ __forceinline__ void rms_norm_head(const float* x, const float* w, float eps, float* v) {
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
  const float r = rsqrtf(row16_sum(ss) / kHead + eps);
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = round_bf16(x[e] * r) * w[e];
}

// Half-split rotary: element i < 64 pairs with i + 64, which lane c ^ 8 holds
// in the same register slot (one row_ror:8 DPP move). lo: lane c < 8. cs, sn:
// cos and sin of pairs 8 (c & 7) .. + 7.
__device__ __forceinline__ void rotate_half(const float* v, const float* cs, const float* sn, bool lo, float* o) {
  // No FMA contraction: whether a*b - c*d fuses, and which product, would
  // otherwise depend on the caller's surrounding code, and callers must agree.
#pragma clang fp contract(off)
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float partner = dpp<kRowRor8>(v[e]);  // element i + 64 for a low lane, i - 64 for a high one
    o[e] = lo ? v[e] * cs[e] - partner * sn[e] : v[e] * cs[e] + partner * sn[e];
  }
}

// PersonaPlex's interleaved rotary (crates/omni-personaplex/kernels/lm.cu:
// 125-182): pair j of x (elements 2j, 2j + 1) turns by the angle whose cos and
// sin are cs[j], sn[j]; PAIRS pairs, in f32.
template <int PAIRS>
__device__ __forceinline__ void rotate_interleaved(float* x, const float* cs, const float* sn) {
#pragma clang fp contract(off)  // as in rotate_half
#pragma unroll
  for (int j = 0; j < PAIRS; ++j) {
    const float re = x[2 * j], im = x[2 * j + 1];
    x[2 * j] = re * cs[j] - im * sn[j];
    x[2 * j + 1] = re * sn[j] + im * cs[j];
  }
}

// The FP8 E4M3 scale of a head whose largest magnitude is amax:
// max(amax / 448, 1e-12); the values are stored as x * (1 / scale).
__device__ __forceinline__ float e4m3_scale(float amax) { return fmaxf(amax * (1.f / 448.f), 1e-12f); }

// Eight f32 to FP8 E4M3 (OCP, round to nearest even) on v_cvt_pk_fp8_f32.
// Callers pass values already scaled into [-448, 448].
__device__ __forceinline__ uint2 e4m3x8(const float* v) {
  int lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false);
  lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], lo, true);
  int hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[4], v[5], 0, false);
  hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[6], v[7], hi, true);
  return make_uint2((uint32_t)lo, (uint32_t)hi);
}

}  // namespace omni
