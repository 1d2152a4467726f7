// Head-64 attentions over short rings (gfx950, wave64): the Mimi codec
// transformer's ring attention and the rotary + ring write before it, the
// Qwen3-TTS codec decoder's fused rotary + ring write + attention, and the
// PersonaPlex depformer's fused K/V write + causal attention.
//
//   mimi_rope_kv64      crates/omni-personaplex/kernels/mimi.cu:226-246
//   mimi_attend64       crates/omni-personaplex/kernels/mimi.cu:248-263
//   codec_attention64   crates/omni-qwen3-tts/kernels/codec.cu:168-277
//   dep_kv_attend64     crates/omni-personaplex/kernels/lm.cu:314-366
//
// One wave per (row, head). Lane l holds dims 8c .. 8c + 7 (c = l % 8, one
// 16-byte load of a 128-byte K or V row) of key row r = l / 8, so one load
// instruction covers 8 keys; scores are 8-lane DPP sums and the softmax runs
// online in base 2 with the scale folded into q. The key a fused kernel has
// just produced (the current frame or step) stays in each lane's registers
// and replaces the loaded value by a select, so no lane reads memory another
// lane of the same kernel has just written.
#include "common.h"
#include "kernels.h"

namespace omni {

namespace {

constexpr int kD = 64;
constexpr int kCodecWindow = 72;
constexpr int kDepSteps = 8;

__device__ __forceinline__ float row8_sum64(float v) {
  v += dpp<kQuadSwap1>(v);
  v += dpp<kQuadSwap2>(v);
  v += dpp<kRowHalfMirror>(v);
  return v;
}

// Combine the 8 key rows of the wave (lanes 8 apart), per lane.
template <bool MAX>
__device__ __forceinline__ float across_rows8(float v) {
  v = MAX ? fmaxf(v, dpp<kRowRor8>(v)) : v + dpp<kRowRor8>(v);
  v = MAX ? fmaxf(v, xor_lane(v, 16)) : v + xor_lane(v, 16);
  v = MAX ? fmaxf(v, xor_lane(v, 32)) : v + xor_lane(v, 32);
  return v;
}

__device__ __forceinline__ uint4 pack8(const float* v) {
  return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                    pack_bf16x2(v[6], v[7]));
}

// Online-softmax state of one (row, head) spread over the wave.
struct Row64 {
  float q[8];  // q dims 8c .. 8c + 7, times scale * log2(e)
  float m, l, acc[8];

  __device__ void init(const float* qv, float scale) {
    const float s = scale * kLog2e;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      q[e] = qv[e] * s;
      acc[e] = 0.f;
    }
    m = -INFINITY;
    l = 0.f;
  }

  // The K and V rows of keys tb .. tb + 8 NI - 1 (clamped to len - 1): key
  // row r = lane / 8 of load i is key tb + 8 i + r.
  template <int NI>
  struct Tile {
    uint4 kr[NI], vr[NI];
  };
  template <int NI, class KV>
  __device__ static void load(Tile<NI>& x, int tb, int len, const KV& kv) {
    const int lane = threadIdx.x & 63, r = lane >> 3, c = lane & 7;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int t = min(tb + 8 * i + r, len - 1);
      x.kr[i] = ldg16(kv.k(t) + 8 * c);
      x.vr[i] = ldg16(kv.v(t) + 8 * c);
    }
  }

  // Online softmax over one loaded tile; key `cur` (if in it) comes from
  // (cur_k, cur_v) instead of memory.
  template <int NI>
  __device__ void step(Tile<NI>& x, int tb, int len, int cur, const uint4& cur_k, const uint4& cur_v) {
    const int lane = threadIdx.x & 63, r = lane >> 3;
    float sc[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int t = tb + 8 * i + r;
      if (t == cur) {
        x.kr[i] = cur_k;
        x.vr[i] = cur_v;
      }
      float kf[8];
      widen8(x.kr[i], kf);
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) d = fmaf(q[e], kf[e], d);
      d = row8_sum64(d);
      sc[i] = t < len ? d : -INFINITY;
    }
    float mx = sc[0];
#pragma unroll
    for (int i = 1; i < NI; ++i) mx = fmaxf(mx, sc[i]);
    mx = across_rows8<true>(mx);
    const float mn = fmaxf(m, mx);
    const float corr = fast_exp2(m - mn);
    m = mn;
    float ps = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= corr;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const float p = fast_exp2(sc[i] - mn);
      ps += p;
      float vf[8];
      widen8(x.vr[i], vf);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = fmaf(p, vf[e], acc[e]);
    }
    l = fmaf(l, corr, ps);
  }

  // Keys t = 0 .. len-1: K and V rows at kv.k(t), kv.v(t) (element pointers),
  // 8 NI keys per round trip. (Two register tiles, the next one's loads in
  // flight during this one's math, measured slower on Mimi's 250-key rings:
  // 22.6 against 21.3 us per launch.)
  template <int NI = 2, class KV>
  __device__ void run(int len, const KV& kv, int cur, const uint4& cur_k, const uint4& cur_v) {
    for (int tb = 0; tb < len; tb += 8 * NI) {
      Tile<NI> x;
      load(x, tb, len, kv);
      step(x, tb, len, cur, cur_k, cur_v);
    }
  }

  // Sum the 8 key rows and write dims 8c .. 8c + 7 (lanes of key row 0).
  __device__ void finish(bf16_t* out) {
    const int lane = threadIdx.x & 63, c = lane & 7;
    const float lt = across_rows8<false>(l);
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = across_rows8<false>(acc[e]) / lt;
    if (lane < 8) *reinterpret_cast<uint4*>(out + 8 * c) = pack8(o);
  }
};

// ----------------------------------------------------------------- Mimi ring
struct MimiRing {
  const bf16_t* ring;
  int first, context, heads, h;
  __device__ const bf16_t* k(int t) const {
    return ring + ((int64_t)((first + t) % context) * 2 * heads + h) * kD;
  }
  __device__ const bf16_t* v(int t) const {
    return ring + ((int64_t)((first + t) % context) * 2 * heads + heads + h) * kD;
  }
};

__global__ __launch_bounds__(64) void mimi_attend64(ShortArgs a) {
  const int n = blockIdx.x, h = blockIdx.y, c = threadIdx.x & 7;
  const int s = n / a.T;
  const int p = a.pos[s] * a.T + n % a.T;
  const int len = min(p + 1, a.context);
  float qv[8];
  widen8(ldg16(a.qkv + ((int64_t)n * 3 * a.heads + h) * kD + 8 * c), qv);
  Row64 st;
  st.init(qv, a.scale);
  const MimiRing ring{reinterpret_cast<const bf16_t*>(static_cast<const uint8_t*>(a.state) +
                                                      (int64_t)a.lines[s] * a.stride),
                      p - len + 1, a.context, a.heads, h};
  st.run(len, ring, -1, uint4{}, uint4{});
  st.finish(a.out + ((int64_t)n * a.heads + h) * kD);
}

// Mimi's rotary + ring write: row n of session s = n / T at p = pos[s] T +
// n % T. One 256-thread workgroup per row; the row's 32 angles (pair i turns
// by p exp(i coef), computed with expf and sincosf as the reference does) go
// to LDS once. Thread u takes the 16-byte chunk u % 8 (dims 8c .. 8c + 7,
// interleaved pairs 4c .. 4c + 3) of head u / 8 of [q | k | v]: q heads are
// turned in place, k heads turned into ring slot p % context (its K heads),
// v heads copied there (its V heads), each rotated value rounded to bf16.
__global__ __launch_bounds__(256) void mimi_rope_kv64(ShortArgs a) {
  const int n = blockIdx.x, s = n / a.T;
  const int p = a.pos[s] * a.T + n % a.T;
  __shared__ float s_cos[kD / 2], s_sin[kD / 2];
  if (threadIdx.x < kD / 2) {
    const float freq = expf((float)threadIdx.x * a.coef);
    sincosf(freq * (float)p, &s_sin[threadIdx.x], &s_cos[threadIdx.x]);
  }
  __syncthreads();
  bf16_t* row = a.qkv_rw + (int64_t)n * 3 * a.heads * kD;
  bf16_t* slot = reinterpret_cast<bf16_t*>(static_cast<uint8_t*>(a.state) + (int64_t)a.lines[s] * a.stride) +
                 (int64_t)(p % a.context) * 2 * a.heads * kD;
  for (int u = threadIdx.x; u < 3 * a.heads * 8; u += blockDim.x) {
    const int hh = u >> 3, c = u & 7;
    const uint4 w = ldg16(row + hh * kD + 8 * c);
    if (hh >= 2 * a.heads) {  // v: copied into the slot's V heads
      *reinterpret_cast<uint4*>(slot + (int64_t)(hh - a.heads) * kD + 8 * c) = w;
      continue;
    }
    float x[8], y[8];
    widen8(w, x);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float cs = s_cos[4 * c + j], sn = s_sin[4 * c + j];
      y[2 * j] = x[2 * j] * cs - x[2 * j + 1] * sn;
      y[2 * j + 1] = x[2 * j] * sn + x[2 * j + 1] * cs;
    }
    bf16_t* dst = hh < a.heads ? row + hh * kD : slot + (int64_t)(hh - a.heads) * kD;
    *reinterpret_cast<uint4*>(dst + 8 * c) = pack8(y);
  }
}

// ------------------------------------------------------ Qwen3-TTS codec ring
struct CodecRing {
  const bf16_t* ring;  // K[72][width] then V[72][width]
  int first, width, h;
  __device__ const bf16_t* k(int t) const { return ring + (int64_t)((first + t) % kCodecWindow) * width + h * kD; }
  __device__ const bf16_t* v(int t) const {
    return ring + ((int64_t)kCodecWindow + (first + t) % kCodecWindow) * width + h * kD;
  }
};

__global__ __launch_bounds__(64) void codec_attention64(ShortArgs a) {
  const int r = blockIdx.x, h = blockIdx.y;
  const int lane = threadIdx.x & 63, c = lane & 7;
  const int width = a.heads * kD;
  const bf16_t* row = a.qkv + (int64_t)r * 3 * width + h * kD;
  bf16_t* ring = reinterpret_cast<bf16_t*>(static_cast<uint8_t*>(a.state) + (int64_t)a.lines[r] * a.stride);
  const int p = a.pos[r];
  const int n = min(p + 1, kCodecWindow);
  // The whole window (at most 72 keys, 9 rows of 8) is loaded first, in one
  // round trip that overlaps the rotary below. The slot of frame p, written
  // below, reads stale here and is replaced by the registers' values.
  const CodecRing kv{ring, p - n + 1, width, h};
  Row64::Tile<kCodecWindow / 8> win;
  Row64::load(win, 0, n, kv);

  // Half-split rotary of q and k at p: pair i = dims i, i + 32; lane c holds
  // dims 8c .. 8c + 7, whose partners are in lane c ^ 4.
  float qk[2][8];
  widen8(ldg16(row + 8 * c), qk[0]);
  widen8(ldg16(row + width + 8 * c), qk[1]);
  const uint4 cur_v = ldg16(row + 2 * width + 8 * c);
  // The 32 angles once, one pair per lane, through LDS.
  __shared__ float s_cos[kD / 2], s_sin[kD / 2];
  if (lane < kD / 2) {
    const float inv_freq = 1.f / powf(a.theta, (float)(2 * lane) / kD);
    sincosf((float)p * inv_freq, &s_sin[lane], &s_cos[lane]);
  }
  __syncthreads();
  const bool lo = c < 4;
  float rot[2][8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int i = 8 * (c & 3) + e;
    const float cs = s_cos[i], sn = s_sin[i];
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const float partner = xor_lane(qk[w][e], 4);
      rot[w][e] = lo ? qk[w][e] * cs - partner * sn : qk[w][e] * cs + partner * sn;
    }
  }
  const uint4 qb = pack8(rot[0]), cur_k = pack8(rot[1]);  // both rounded to bf16
  float qv[8];
  widen8(qb, qv);
  if (lane < 8) {  // frame p % 72 of the ring: the rotated k and the v row
    const int64_t at = (int64_t)(p % kCodecWindow) * width + h * kD + 8 * c;
    *reinterpret_cast<uint4*>(ring + at) = cur_k;
    *reinterpret_cast<uint4*>(ring + (int64_t)kCodecWindow * width + at) = cur_v;
  }
  Row64 st;
  st.init(qv, 0.125f);  // 1 / sqrt(64)
  st.step(win, 0, n, n - 1, cur_k, cur_v);
  st.finish(a.out + (int64_t)r * width + h * kD);
}

// ------------------------------------------------------- depformer steps
struct DepSteps {
  const bf16_t* ws;  // the session's [8][K | V][width]
  int width, h;
  __device__ const bf16_t* k(int t) const { return ws + (int64_t)t * 2 * width + h * kD; }
  __device__ const bf16_t* v(int t) const { return ws + (int64_t)t * 2 * width + width + h * kD; }
};

__global__ __launch_bounds__(64) void dep_kv_attend64(ShortArgs a) {
  const int s = blockIdx.x, h = blockIdx.y;
  const int lane = threadIdx.x & 63, c = lane & 7;
  const int width = a.heads * kD;
  const bf16_t* row = a.qkv + (int64_t)s * 3 * width;
  bf16_t* ws = a.ws + (int64_t)s * kDepSteps * 2 * width;
  // Steps 0 .. step (at most 8, one row of 8 keys) load together with the
  // row; step `step`, written below, is replaced by the registers' values.
  Row64::Tile<kDepSteps / 8> win;
  Row64::load(win, 0, a.step + 1, DepSteps{ws, width, h});
  const uint4 cur_k = ldg16(row + width + h * kD + 8 * c);
  const uint4 cur_v = ldg16(row + 2 * width + h * kD + 8 * c);
  if (lane < 8) {
    *reinterpret_cast<uint4*>(ws + (int64_t)a.step * 2 * width + h * kD + 8 * c) = cur_k;
    *reinterpret_cast<uint4*>(ws + (int64_t)a.step * 2 * width + width + h * kD + 8 * c) = cur_v;
  }
  float qv[8];
  widen8(ldg16(row + h * kD + 8 * c), qv);
  Row64 st;
  st.init(qv, a.scale);
  st.step(win, 0, a.step + 1, a.step, cur_k, cur_v);
  st.finish(a.out + (int64_t)s * width + h * kD);
}

}  // namespace

int launch_short(const ShortArgs& a, int kind, hipStream_t stream) {
  if (a.rows == 0) return 0;
  const dim3 grid(a.rows, a.heads);
  switch (kind) {
    case kShortMimi: mimi_attend64<<<grid, 64, 0, stream>>>(a); break;
    case kShortCodec: codec_attention64<<<grid, 64, 0, stream>>>(a); break;
    case kShortDep: dep_kv_attend64<<<grid, 64, 0, stream>>>(a); break;
    case kShortMimiRope: mimi_rope_kv64<<<a.rows, 256, 0, stream>>>(a); break;
    default: return -2;
  }
  return check_launch();
}

}  // namespace omni
