// Device helpers shared by the attention kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace omni {

constexpr int kHead = 128;  // head_dim of every attention this library serves
constexpr float kLog2e = 1.4426950408889634f;

typedef uint16_t bf16_t;  // raw bf16 bits in memory

// bf16 -> f32 is exact: the 16 bits are the top half of the f32.
__device__ __forceinline__ float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// f32 -> bf16, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
__device__ __forceinline__ uint32_t f2bf(float f) { return pack_bf16x2(f, 0.f) & 0xffffu; }

// Eight bf16 (one 16-byte load) widened to f32.
__device__ __forceinline__ void widen8(const uint4& u, float* v) {
  v[0] = lo_bf16(u.x);
  v[1] = hi_bf16(u.x);
  v[2] = lo_bf16(u.y);
  v[3] = hi_bf16(u.y);
  v[4] = lo_bf16(u.z);
  v[5] = hi_bf16(u.z);
  v[6] = lo_bf16(u.w);
  v[7] = hi_bf16(u.w);
}

__device__ __forceinline__ uint4 ldg16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
// A 16-byte load of data read once (K/V streams): nontemporal, so it streams
// through the caches instead of displacing reusable lines.
__device__ __forceinline__ uint4 ldg16_stream(const void* p) {
  typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// 2^x on the transcendental unit (v_exp_f32); exp2(-inf) = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// DPP lane moves within a row of 16 lanes (gfx9 DPP controls).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
constexpr int kQuadSwap1 = 0xB1;      // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kQuadSwap2 = 0x4E;      // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kRowHalfMirror = 0x141; // lane i <- 7 - i within each 8
constexpr int kRowMirror = 0x140;     // lane i <- 15 - i within each 16
constexpr int kRowRor8 = 0x128;       // lane i <- (i + 8) % 16 within each 16: lane ^ 8

// Sum over the 16 lanes of a DPP row; every lane of the row gets the sum.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<kQuadSwap1>(v);
  v += dpp<kQuadSwap2>(v);
  v += dpp<kRowHalfMirror>(v);
  v += dpp<kRowMirror>(v);
  return v;
}

// Lane exchange across rows of 16 (xor 16, xor 32) via ds_swizzle-free bpermute.
__device__ __forceinline__ float xor_lane(float v, int mask) {
  const int lane = __lane_id();
  return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(v)));
}

}  // namespace omni
