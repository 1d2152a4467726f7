// Peak microbenchmarks for gfx950, used by bench.py to report the measured
// ceilings next to the published ones: bf16 MFMA throughput, v_exp_f32 and
// v_fma_f32 issue rates, and streaming HBM read bandwidth. A measurement
// probe of the benchmark, not part of the attention library: built into
// bench_peaks.so by `python bench.py --build-peaks` (bench.py builds it on
// first use when it is missing).
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ inline uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  return x ^ (x >> 16);
}

// Four independent 32x32x16 bf16 MFMA chains per wave, `iters` rounds of four
// steps. RANDOM = false: one smooth operand pair (few bits change between
// lanes). RANDOM = true: four operand pairs of hashed values uniform in
// [-2, 2), rotated between the steps, as attention tiles feed the MFMAs. The
// card lowers its clock under MFMA load by how many operand bits toggle, so
// the random form is the ceiling real data reaches.
template <bool RANDOM>
__global__ __launch_bounds__(256) void mfma_loop(float* sink, int iters) {
  bf16x8 a[4], b[4];
  for (int s = 0; s < 4; ++s)
    for (int i = 0; i < 8; ++i) {
      float x = 0.001f * (threadIdx.x + i), y = 0.002f * (threadIdx.x - i);
      if (RANDOM) {
        const uint32_t h = mix32(threadIdx.x * 977u + blockIdx.x * 131071u + s * 8u + i), g = mix32(h);
        x = ((int)(h & 0xffff) - 32768) / 16384.f;
        y = ((int)(g & 0xffff) - 32768) / 16384.f;
      }
      a[s][i] = (__bf16)x;
      b[s][i] = (__bf16)y;
    }
  f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[s], b[s], c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[(s + 1) & 3], b[s], c1, 0, 0, 0);
      c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[(s + 2) & 3], b[(s + 1) & 3], c2, 0, 0, 0);
      c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[(s + 3) & 3], b[(s + 2) & 3], c3, 0, 0, 0);
    }
  }
  float s = 0.f;
  for (int i = 0; i < 16; ++i) s += c0[i] + c1[i] + c2[i] + c3[i];
  if (s == 1234.5f) sink[threadIdx.x] = s;
}

// Eight independent v_exp_f32 (or v_fma_f32) chains per lane.
template <bool EXP>
__global__ __launch_bounds__(256) void valu_loop(float* sink, int iters) {
  float x[8];
  for (int i = 0; i < 8; ++i) x[i] = -0.001f * (threadIdx.x + i);
  for (int it = 0; it < iters; ++it)
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = EXP ? __builtin_amdgcn_exp2f(x[i]) - 1.0f : fmaf(x[i], 0.999f, 0.001f);
  float s = 0.f;
  for (int i = 0; i < 8; ++i) s += x[i];
  if (s == 1234.5f) sink[threadIdx.x] = s;
}

// Streaming read: every thread sums 16-byte words, grid-strided.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void read_stream(const u32x4* p, int64_t n, unsigned* sink) {
  unsigned acc = 0;
  for (int64_t i = blockIdx.x * 256LL + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const u32x4 v = __builtin_nontemporal_load(p + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x12345678u) sink[0] = acc;
}

// LDS read throughput: each lane reads 16 bytes per ds_read_b128 from a
// conflict-free pattern, 8 independent reads per round.
__global__ __launch_bounds__(256) void lds_loop(float* sink, int iters) {
  __shared__ __align__(16) float buf[16384];
  for (int i = threadIdx.x; i < 16384; i += 256) buf[i] = (float)i;
  __syncthreads();
  typedef float f4 __attribute__((ext_vector_type(4)));
  int base = (threadIdx.x & 63) * 4 + (threadIdx.x >> 6) * 2048;
  for (int it = 0; it < iters; ++it) {
    asm volatile("" : "+v"(base));  // the reads stay inside the loop
    f4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = *reinterpret_cast<const f4*>(buf + ((base + k * 256) & 0x3FFC));
    // Consumed without arithmetic, all 8 in flight together, so LDS is the limit.
    asm volatile("" ::"v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]), "v"(v[6]), "v"(v[7]));
  }
  if (iters < 0) sink[threadIdx.x] = buf[threadIdx.x];
}

extern "C" {
int omni_peaks_lds(void* sink, int blocks, int iters, void* stream) {
  lds_loop<<<blocks, 256, 0, (hipStream_t)stream>>>((float*)sink, iters);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
// Each returns 0 or -1; the caller times the launch on `stream`.
// 16 MFMAs per wave per iteration; random != 0 selects the random operands.
int omni_peaks_mfma(void* sink, int blocks, int iters, int random, void* stream) {
  if (random)
    mfma_loop<true><<<blocks, 256, 0, (hipStream_t)stream>>>((float*)sink, iters);
  else
    mfma_loop<false><<<blocks, 256, 0, (hipStream_t)stream>>>((float*)sink, iters);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
int omni_peaks_valu(void* sink, int blocks, int iters, int exp, void* stream) {
  if (exp)
    valu_loop<true><<<blocks, 256, 0, (hipStream_t)stream>>>((float*)sink, iters);
  else
    valu_loop<false><<<blocks, 256, 0, (hipStream_t)stream>>>((float*)sink, iters);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
int omni_peaks_read(const void* p, int64_t bytes, void* sink, int blocks, void* stream) {
  read_stream<<<blocks, 256, 0, (hipStream_t)stream>>>((const u32x4*)p, bytes / 16, (unsigned*)sink);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
}
