/*
 * CPU ORACLE — test infrastructure only.
 *
 * A plain C restatement of the reference's attention math, used as the checker
 * for the HIP kernels (tests/, __graft_entry__.smoke(), bench.py's cpu_baseline
 * leg). Nothing in the product library links, loads or calls this file.
 *
 * Functions and the reference code each one restates (paths relative to the
 * pega-omni tree):
 *   oracle_slot           crates/omni-qwen3/kernels/qwen3.cu:210-214 (PagedSlots),
 *                         crates/omni-personaplex/kernels/lm.cu:184-192
 *   oracle_gather_kv      the same slot rule applied to every key of a row
 *   oracle_paged_attend   crates/omni-qwen3/kernels/qwen3.cu:123-208 (attend<G>),
 *                         :234-240 (qwen3_attend), and with `context` the ring cap
 *                         of crates/omni-personaplex/kernels/lm.cu:273-290
 *                         (lm_attend, bf16 slots as crates/omni-personaplex/
 *                         kernels/attend.cuh:41-106)
 *   oracle_dense_attend   crates/omni-hidream-o1/kernels/hidream.cu:209-347
 *                         (hidream_attend: base-2 online softmax over 64-key tiles,
 *                         P rounded to bf16 before P.V, l from unrounded P)
 *   oracle_lm_attend_fp8  crates/omni-personaplex/kernels/lm.cu:196-290 (lm_attend over
 *                         FP8 E4M3 slots with per-(slot, head) f32 scales), with
 *                         oracle_e4m3_to_f32 the OCP E4M3 decode
 *   oracle_qwen3_rope     crates/omni-qwen3/kernels/qwen3.cu:64-103 (rope_kv, qwen3_rope)
 *   oracle_qwen3_rope_dense  qwen3.cu:105-111 (qwen3_rope_dense)
 *   oracle_hidream_qk_rope   crates/omni-hidream-o1/kernels/hidream.cu:55-106
 *   oracle_lm_rope        crates/omni-personaplex/kernels/lm.cu:125-182 (lm_rope) with
 *                         attend.cuh:108-128 (rope_head); oracle_f32_to_e4m3 the
 *                         OCP E4M3 encode (round to nearest even, saturating)
 *   oracle_qwen3_attend_dense  crates/omni-qwen3/kernels/qwen3.cu:243-248
 *   oracle_mimi_attend    crates/omni-personaplex/kernels/mimi.cu:248-263 (head 64 ring in
 *                         the session's state, attend_row<64> of attend.cuh:41-106)
 *   oracle_mimi_rope_kv   crates/omni-personaplex/kernels/mimi.cu:226-246 (rotary of q in
 *                         place, of k into the ring slot, v copied; rope_head<64>)
 *   oracle_lm_copy_kv     crates/omni-personaplex/kernels/lm.cu:583-593 (slot copy)
 *   oracle_codec_attention  crates/omni-qwen3-tts/kernels/codec.cu:168-277 (rotary, 72-frame
 *                         ring write and attention, fused)
 *   oracle_lm_dep_kv_attend crates/omni-personaplex/kernels/lm.cu:314-366 (depformer step)
 *   oracle_fill_normal_bf16 / oracle_splitmix64  the synthetic-input rule
 *
 * Arithmetic follows the reference kernels: f32 accumulation, per-tile online
 * softmax with the same tile sizes (4 warps x 32 keys for the paged kernel, 64
 * keys for the dense kernel), then bf16 round-to-nearest-even of the output.
 * Cross-lane sums are taken in butterfly order like the warp reductions.
 * The exponentials use libm expf / exp2f, so results agree with the GPU
 * reference to within rounding, not bit for bit.
 *
 * Threads: the attention entry points take `nthreads` and split independent
 * (row, kv head) or (query block, kv head) work items over a pthread pool; the
 * result does not depend on the thread count.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef uint16_t bf16_t;

static inline float bf2f(bf16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Round-to-nearest-even f32 -> bf16 (NaN kept quiet). */
static inline bf16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (bf16_t)(u >> 16);
}

float oracle_bf16_to_f32(bf16_t h) { return bf2f(h); }
bf16_t oracle_f32_to_bf16(float f) { return f2bf(f); }

/* ---------------------------------------------------------------- inputs */

/* splitmix64 (Steele, Lea, Flood 2014): state += golden gamma, then mix. */
uint64_t oracle_splitmix64(uint64_t* state) {
  uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* n values of N(0,1) by Box-Muller in double (two uniforms from 53-bit
 * splitmix64 draws per pair), rounded to bf16 RNE. */
void oracle_fill_normal_bf16(bf16_t* out, int64_t n, uint64_t seed) {
  uint64_t st = seed;
  for (int64_t i = 0; i < n; i += 2) {
    double u1 = ((oracle_splitmix64(&st) >> 11) + 1.0) * (1.0 / 9007199254740993.0);
    double u2 = (oracle_splitmix64(&st) >> 11) * (1.0 / 9007199254740992.0);
    double r = sqrt(-2.0 * log(u1));
    out[i] = f2bf((float)(r * cos(6.283185307179586 * u2)));
    if (i + 1 < n) out[i + 1] = f2bf((float)(r * sin(6.283185307179586 * u2)));
  }
}

/* ------------------------------------------------------------ page table */

/* Physical slot of logical token t of the row whose page list starts at
 * pages + indptr[s]: pages[t / page] * page + t % page. */
int64_t oracle_slot(const int32_t* indptr, const int32_t* pages, int s, int t, int page) {
  const int32_t* p = pages + indptr[s];
  return (int64_t)p[t / page] * page + t % page;
}

/* Dense copy of the first `len` tokens of sequence s: out[t][2*hk][128] =
 * kv[slot(t)][2*hk][128], byte for byte. */
void oracle_gather_kv(const bf16_t* kv, int hk, const int32_t* indptr, const int32_t* pages, int page, int s,
                      int len, bf16_t* out) {
  const int64_t per = 2LL * hk * 128;
  for (int t = 0; t < len; ++t) memcpy(out + (int64_t)t * per, kv + oracle_slot(indptr, pages, s, t, page) * per,
                                       (size_t)per * sizeof(bf16_t));
}

/* ------------------------------------------------------- thread helper */

typedef void (*item_fn)(void* ctx, int64_t item);
typedef struct {
  item_fn fn;
  void* ctx;
  int64_t n;
  int64_t next;
  pthread_mutex_t mu;
} pool_t;

static void* pool_worker(void* arg) {
  pool_t* p = (pool_t*)arg;
  for (;;) {
    pthread_mutex_lock(&p->mu);
    int64_t i = p->next++;
    pthread_mutex_unlock(&p->mu);
    if (i >= p->n) return NULL;
    p->fn(p->ctx, i);
  }
}

static void run_items(item_fn fn, void* ctx, int64_t n, int nthreads) {
  if (nthreads <= 1 || n <= 1) {
    for (int64_t i = 0; i < n; ++i) fn(ctx, i);
    return;
  }
  pool_t p = {fn, ctx, n, 0, PTHREAD_MUTEX_INITIALIZER};
  if (nthreads > 256) nthreads = 256;
  pthread_t th[256];
  int started = 0;
  for (int i = 0; i < nthreads; ++i)
    if (pthread_create(&th[i], NULL, pool_worker, &p) == 0) ++started;
  if (started == 0) pool_worker(&p);
  for (int i = 0; i < started; ++i) pthread_join(th[i], NULL);
}

/* --------------------------------------------------- paged attention */

#define HEAD 128
#define WARPS 4
#define LANES 32
#define GMAX 8

/* Butterfly sum of 32 lane values in the order xor 16, 8, 4, 2, 1 (lane 0's
 * result), the order a 32-lane xor-shuffle reduction produces. */
static float bfly_sum(const float* v) {
  float a[LANES];
  memcpy(a, v, sizeof a);
  for (int o = 16; o > 0; o >>= 1) {
    float b[LANES];
    for (int l = 0; l < LANES; ++l) b[l] = a[l] + a[l ^ o];
    memcpy(a, b, sizeof a);
  }
  return a[0];
}

typedef struct {
  const bf16_t* qkv;
  const bf16_t* kv;
  const int32_t* pos;
  const int32_t* seq;
  int ragged;
  const int32_t* indptr;
  const int32_t* pages;
  int page;
  bf16_t* out;
  int hq, hk;
  float scale;
  int context;
  int dense_per, dense_base, dense_span; /* dense_per > 0: qwen3_attend_dense rows */
} paged_args;

/* One (row n, kv head kh) work item. Restates attend<G> (qwen3.cu:123-208):
 * warp w scores the 32-key tiles starting at w*32, w*32+128, ...; each tile
 * updates (m, l, acc) online with natural exp; the 4 warps' states merge as
 * num = sum_w acc_w * exp(m_w - top), den = sum_w l_w * exp(m_w - top), with
 * an empty warp (m = -inf) contributing 0 (attend.cuh:93). */
static void paged_item(void* vctx, int64_t item) {
  const paged_args* a = (const paged_args*)vctx;
  const int n = (int)(item / a->hk), kh = (int)(item % a->hk);
  const int G = a->hq / a->hk;
  const int s = a->ragged ? a->seq[n] : n;
  int len = a->dense_per > 0 ? a->dense_base + n % a->dense_per + 1 : a->pos[n] + 1;
  if (len > a->context) len = a->context;
  const int64_t dense_first = a->dense_per > 0 ? (int64_t)(n / a->dense_per) * a->dense_span : 0;
  const int64_t per_slot = 2LL * a->hk * HEAD;
  const bf16_t* q = a->qkv + ((int64_t)n * (a->hq + 2 * a->hk) + (int64_t)kh * G) * HEAD;
  float qs[GMAX][HEAD];
  for (int g = 0; g < G; ++g)
    for (int d = 0; d < HEAD; ++d) qs[g][d] = bf2f(q[g * HEAD + d]);

  float M[WARPS][GMAX], L[WARPS][GMAX], O[WARPS][GMAX][HEAD];
  for (int w = 0; w < WARPS; ++w) {
    for (int g = 0; g < G; ++g) {
      float m = -INFINITY, l = 0.f;
      float* acc = O[w][g];
      for (int d = 0; d < HEAD; ++d) acc[d] = 0.f;
      for (int base = w * LANES; base < len; base += WARPS * LANES) {
        float sv[LANES], p[LANES];
        int64_t slot[LANES];
        float tmax = -INFINITY;
        for (int lane = 0; lane < LANES; ++lane) {
          const int t = base + lane;
          const int valid = t < len;
          slot[lane] = a->dense_per > 0 ? dense_first + (valid ? t : base)
                                        : oracle_slot(a->indptr, a->pages, s, valid ? t : base, a->page);
          const bf16_t* k = a->kv + slot[lane] * per_slot + (int64_t)kh * HEAD;
          float dot = 0.f;
          for (int d = 0; d < HEAD; ++d) dot += qs[g][d] * bf2f(k[d]);
          sv[lane] = valid ? dot * a->scale : -INFINITY;
          if (sv[lane] > tmax) tmax = sv[lane];
        }
        const float m2 = fmaxf(m, tmax);
        const float corr = expf(m - m2);
        for (int lane = 0; lane < LANES; ++lane) p[lane] = expf(sv[lane] - m2);
        l = l * corr + bfly_sum(p);
        for (int d = 0; d < HEAD; ++d) acc[d] *= corr;
        m = m2;
        const int count = len - base < LANES ? len - base : LANES;
        for (int j = 0; j < count; ++j) {
          const bf16_t* v = a->kv + slot[j] * per_slot + (int64_t)(a->hk + kh) * HEAD;
          for (int d = 0; d < HEAD; ++d) acc[d] += p[j] * bf2f(v[d]);
        }
      }
      M[w][g] = m;
      L[w][g] = l;
    }
  }
  for (int g = 0; g < G; ++g) {
    float top = -INFINITY;
    for (int w = 0; w < WARPS; ++w) top = fmaxf(top, M[w][g]);
    for (int d = 0; d < HEAD; ++d) {
      float num = 0.f, den = 0.f;
      for (int w = 0; w < WARPS; ++w) {
        const float e = M[w][g] == -INFINITY ? 0.f : expf(M[w][g] - top);
        num += O[w][g][d] * e;
        den += L[w][g] * e;
      }
      a->out[((int64_t)n * a->hq + (int64_t)kh * G + g) * HEAD + d] = f2bf(num / den);
    }
  }
}

/* qwen3_attend / lm_attend (bf16 slots). Row n of sequence s = ragged ? seq[n]
 * : n sees min(pos[n] + 1, context) keys whose slots come from pages[indptr[s]..].
 * qkv rows are [(hq + 2 hk)][128] (q heads first); kv slots [2 hk][128];
 * out [rows][hq][128]. Returns 0, or -1 for an unsupported head shape. */
int oracle_paged_attend(const bf16_t* qkv, const bf16_t* kv, const int32_t* pos, const int32_t* seq, int ragged,
                        const int32_t* indptr, const int32_t* pages, int page, bf16_t* out, int rows, int hq, int hk,
                        float scale, int context, int nthreads) {
  if (hk <= 0 || hq % hk != 0 || hq / hk > GMAX || page <= 0) return -1;
  paged_args a = {qkv, kv, pos, seq, ragged, indptr, pages, page, out, hq, hk, scale, context > 0 ? context : 0x7fffffff, 0, 0, 0};
  run_items(paged_item, &a, (int64_t)rows * hk, nthreads);
  return 0;
}

/* qwen3_attend_dense (crates/omni-qwen3/kernels/qwen3.cu:243-248): row n sees
 * keys 0 .. base + n % per at dense slots (n / per) * span + t of kv. */
int oracle_qwen3_attend_dense(const bf16_t* qkv, const bf16_t* kv, int per, int base, int span, bf16_t* out, int rows,
                              int hq, int hk, float scale, int nthreads) {
  if (hk <= 0 || hq % hk != 0 || hq / hk > GMAX || per <= 0) return -1;
  paged_args a = {qkv, kv, NULL, NULL, 0, NULL, NULL, 1, out, hq, hk, scale, 0x7fffffff, per, base, span};
  run_items(paged_item, &a, (int64_t)rows * hk, nthreads);
  return 0;
}

/* --------------------------------------------------- dense (DiT) attention */

#define BN 64

typedef struct {
  const bf16_t* q;
  const bf16_t* k;
  const bf16_t* v;
  bf16_t* out;
  int q_len, kv_len, q_stride, hq, hk, causal;
  float scale_log2;
} dense_args;

/* One (query row n, q head h) item. Restates hidream_attend's per-row math
 * (hidream.cu:262-344): keys in 64-key tiles up to the block's last key; a
 * masked score is -inf; per tile m_new = max(m, max_s * scale_log2),
 * base = m_new or 0 while no key has been seen, alpha = 2^(m - base),
 * p = 2^(s * scale_log2 - base), l = l * alpha + sum(p) over the unrounded p,
 * O = O * alpha + bf16(p) . V; finally out = bf16(O * (1 / l)).
 * The reference's per-thread partial sums of l are merged over the 4 lanes
 * of a quad at the end; with f32 that changes rounding only. */
static void dense_item(void* vctx, int64_t item) {
  const dense_args* a = (const dense_args*)vctx;
  const int n = (int)(item / a->hq), h = (int)(item % a->hq);
  const int G = a->hq / a->hk, kvh = h / G;
  const int kv_stride = a->hk * HEAD;
  float qs[HEAD], o[HEAD];
  for (int d = 0; d < HEAD; ++d) {
    qs[d] = bf2f(a->q[(int64_t)n * a->q_stride + (int64_t)h * HEAD + d]);
    o[d] = 0.f;
  }
  const int lim = a->causal ? (n + 1 < a->kv_len ? n + 1 : a->kv_len) : a->kv_len;
  float m = -INFINITY, l = 0.f;
  for (int n0 = 0; n0 < lim; n0 += BN) {
    float sc[BN];
    float mx = -INFINITY;
    for (int j = 0; j < BN; ++j) {
      const int key = n0 + j;
      if (key >= lim) {
        sc[j] = -INFINITY;
        continue;
      }
      const bf16_t* k = a->k + (int64_t)key * kv_stride + (int64_t)kvh * HEAD;
      float dot = 0.f;
      for (int d = 0; d < HEAD; ++d) dot += qs[d] * bf2f(k[d]);
      sc[j] = dot;
      if (dot > mx) mx = dot;
    }
    const float m_new = fmaxf(m, mx * a->scale_log2);
    const float base = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2f(m - base);
    m = m_new;
    float sum = 0.f;
    for (int j = 0; j < BN; ++j) {
      sc[j] = exp2f(sc[j] * a->scale_log2 - base);
      sum += sc[j];
    }
    l = l * alpha + sum;
    for (int d = 0; d < HEAD; ++d) o[d] *= alpha;
    for (int j = 0; j < BN && n0 + j < lim; ++j) {
      const float p = bf2f(f2bf(sc[j]));
      const bf16_t* v = a->v + (int64_t)(n0 + j) * kv_stride + (int64_t)kvh * HEAD;
      for (int d = 0; d < HEAD; ++d) o[d] += p * bf2f(v[d]);
    }
  }
  const float inv = 1.f / l;
  for (int d = 0; d < HEAD; ++d) a->out[((int64_t)n * a->hq + h) * HEAD + d] = f2bf(o[d] * inv);
}

/* hidream_attend generalised to hq = G * hk for any G >= 1 (the reference
 * fixes G = 4): q rows at q + n * q_stride + h * 128, k and v [kv_len][hk][128],
 * out [q_len][hq][128]. With causal, row n sees keys 0..min(n, kv_len - 1). */
int oracle_dense_attend(const bf16_t* q, const bf16_t* k, const bf16_t* v, bf16_t* out, int q_len, int kv_len,
                        int q_stride, int hq, int hk, int causal, float scale_log2, int nthreads) {
  if (hk <= 0 || hq % hk != 0) return -1;
  dense_args a = {q, k, v, out, q_len, kv_len, q_stride, hq, hk, causal, scale_log2};
  run_items(dense_item, &a, (int64_t)q_len * hq, nthreads);
  return 0;
}

/* ------------------------------------------- FP8 (E4M3) ring attention */

/* OCP FP8 E4M3 ("e4m3fn": bias 7, no infinities, S.1111.111 is NaN, max 448,
 * subnormals m * 2^-9) to f32, exactly. */
float oracle_e4m3_to_f32(uint8_t b) {
  const int s = b >> 7, e = (b >> 3) & 15, m = b & 7;
  float v;
  if (e == 15 && m == 7)
    v = NAN;
  else if (e == 0)
    v = ldexpf((float)m, -9);
  else
    v = ldexpf((float)(8 + m), e - 10);
  return s ? -v : v;
}

typedef struct {
  const bf16_t* qkv;
  const uint8_t* kv;
  const int32_t* pos;
  const int32_t* seq;
  int ragged;
  const int32_t* indptr;
  const int32_t* pages;
  int page;
  bf16_t* out;
  int heads;
  float scale;
  int context;
} fp8_args;

/* One (row n, head h) item of lm_attend (lm.cu:196-290): slot =
 * [K heads x 128 B | V heads x 128 B | K scales (f32 x heads) | V scales];
 * s = dot(q, k) * (k_scale * scale); p * v_scale weights the fp8 V row.
 * 4 warps x 32-key tiles with natural-exp online softmax, then the warp merge
 * with empty warps contributing 0, as attend_row_fp8. */
static void fp8_item(void* vctx, int64_t item) {
  const fp8_args* a = (const fp8_args*)vctx;
  const int H = a->heads;
  const int n = (int)(item / H), h = (int)(item % H);
  const int s = a->ragged ? a->seq[n] : n;
  int len = a->pos[n] + 1;
  if (len > a->context) len = a->context;
  const int64_t slot_bytes = 2LL * H * HEAD + 2LL * H * 4;
  const bf16_t* q = a->qkv + (int64_t)n * 3 * H * HEAD + (int64_t)h * HEAD;
  float qs[HEAD];
  for (int d = 0; d < HEAD; ++d) qs[d] = bf2f(q[d]);
  float M[WARPS], L[WARPS], O[WARPS][HEAD];
  for (int w = 0; w < WARPS; ++w) {
    float m = -INFINITY, l = 0.f;
    float* acc = O[w];
    for (int d = 0; d < HEAD; ++d) acc[d] = 0.f;
    for (int base = w * LANES; base < len; base += WARPS * LANES) {
      float sv[LANES], pv[LANES];
      int64_t slot[LANES];
      float tmax = -INFINITY;
      for (int lane = 0; lane < LANES; ++lane) {
        const int t = base + lane;
        const int valid = t < len;
        slot[lane] = oracle_slot(a->indptr, a->pages, s, valid ? t : base, a->page);
        const uint8_t* sp = a->kv + slot[lane] * slot_bytes;
        const uint8_t* k = sp + (int64_t)h * HEAD;
        float ks, vs;
        memcpy(&ks, sp + 2LL * H * HEAD + (int64_t)h * 4, 4);
        memcpy(&vs, sp + 2LL * H * HEAD + (int64_t)(H + h) * 4, 4);
        float dot = 0.f;
        for (int c = 0; c < HEAD; c += 8) {
          float part = qs[c] * oracle_e4m3_to_f32(k[c]);
          for (int e = 1; e < 8; ++e) part += qs[c + e] * oracle_e4m3_to_f32(k[c + e]);
          dot += part;
        }
        sv[lane] = valid ? dot * (ks * a->scale) : -INFINITY;
        pv[lane] = vs;
        if (sv[lane] > tmax) tmax = sv[lane];
      }
      const float m2 = fmaxf(m, tmax);
      const float corr = expf(m - m2);
      float p[LANES];
      for (int lane = 0; lane < LANES; ++lane) p[lane] = expf(sv[lane] - m2);
      l = l * corr + bfly_sum(p);
      for (int d = 0; d < HEAD; ++d) acc[d] *= corr;
      m = m2;
      const int count = len - base < LANES ? len - base : LANES;
      for (int j = 0; j < count; ++j) {
        const float pvj = p[j] * pv[j];
        const uint8_t* v = a->kv + slot[j] * slot_bytes + (int64_t)(H + h) * HEAD;
        for (int d = 0; d < HEAD; ++d) acc[d] += pvj * oracle_e4m3_to_f32(v[d]);
      }
    }
    M[w] = m;
    L[w] = l;
  }
  float top = -INFINITY;
  for (int w = 0; w < WARPS; ++w) top = fmaxf(top, M[w]);
  for (int d = 0; d < HEAD; ++d) {
    float num = 0.f, den = 0.f;
    for (int w = 0; w < WARPS; ++w) {
      const float e = M[w] == -INFINITY ? 0.f : expf(M[w] - top);
      num += O[w][d] * e;
      den += L[w] * e;
    }
    a->out[((int64_t)n * H + h) * HEAD + d] = f2bf(num / den);
  }
}

/* lm_attend over FP8 E4M3 slots (crates/omni-personaplex/kernels/lm.cu:
 * 196-290): MHA, qkv rows [3 heads][128] bf16, slot bytes 2*heads*128 +
 * 2*heads*4, rows see min(pos + 1, context) ring slots. */
int oracle_lm_attend_fp8(const bf16_t* qkv, const uint8_t* kv, const int32_t* pos, const int32_t* seq, int ragged,
                         const int32_t* indptr, const int32_t* pages, int page, bf16_t* out, int rows, int heads,
                         float scale, int context, int nthreads) {
  if (heads <= 0 || page <= 0) return -1;
  fp8_args a = {qkv, kv, pos, seq, ragged, indptr, pages, page, out, heads, scale, context > 0 ? context : 0x7fffffff};
  run_items(fp8_item, &a, (int64_t)rows * heads, nthreads);
  return 0;
}

/* ------------------------------------------- rotary embedding + K/V scatter */

/* f32 -> OCP E4M3, round to nearest even, saturating to +-448 (the finite
 * range); NaN -> 0x7F with the sign. Derived from the format: 1 sign, 4
 * exponent bits with bias 7, 3 mantissa bits, subnormals of 2^-9 steps. */
uint8_t oracle_f32_to_e4m3(float x) {
  const uint8_t sign = signbit(x) ? 0x80 : 0;
  if (isnan(x)) return sign | 0x7F;
  const float a = fabsf(x);
  if (a >= 448.f) return sign | 0x7E;
  if (a < ldexpf(1.f, -6)) {  /* subnormal: multiples of 2^-9 */
    const float m = nearbyintf(ldexpf(a, 9)); /* 0 .. 8; 8 is the smallest normal */
    return sign | (uint8_t)m;
  }
  int e;
  frexpf(a, &e); /* a = f * 2^e, f in [0.5, 1): the leading bit is 2^(e-1) */
  e -= 1;
  float m = nearbyintf(ldexpf(a, 3 - e)); /* 8 .. 16 */
  if (m == 16.f) {
    m = 8.f;
    e += 1;
  }
  if (e > 8) return sign | 0x7E;
  return sign | (uint8_t)(((e + 7) << 3) | ((int)m - 8));
}

/* One head of rope_kv / hidream_qk_rope: RMSNorm (f32 sum, x * rsqrt rounded
 * to bf16, times the bf16 weight), then the half-split rotation of pair i
 * (elements i, i + 64) by pos_of[i] * theta^(-2i/128), rounded to bf16. */
static void norm_rope_head(const bf16_t* src, bf16_t* dst, const bf16_t* w, const int* pos_of, float eps,
                           float theta) {
  float x[HEAD];
  float ss = 0.f;
  for (int i = 0; i < HEAD; ++i) {
    x[i] = bf2f(src[i]);
    ss += x[i] * x[i];
  }
  const float r = 1.f / sqrtf(ss / HEAD + eps);
  float v[HEAD];
  for (int i = 0; i < HEAD; ++i) v[i] = bf2f(f2bf(x[i] * r)) * bf2f(w[i]);
  for (int i = 0; i < HEAD / 2; ++i) {
    const float inv_freq = 1.f / powf(theta, (float)(2 * i) / HEAD);
    const float ang = (float)pos_of[i] * inv_freq;
    const float sn = sinf(ang), cs = cosf(ang);
    const float a = v[i], b = v[HEAD / 2 + i];
    dst[i] = f2bf(a * cs - b * sn);
    dst[HEAD / 2 + i] = f2bf(b * cs + a * sn);
  }
}

static void rope_row(bf16_t* qkv, int64_t ld, const bf16_t* q_norm, const bf16_t* k_norm, int n, const int* pos_of,
                     bf16_t* kdst, int64_t kstride, bf16_t* vdst, int64_t vstride, int hq, int hk, float eps,
                     float theta) {
  bf16_t* row = qkv + (int64_t)n * ld;
  for (int h = 0; h < hq; ++h) norm_rope_head(row + h * HEAD, row + h * HEAD, q_norm, pos_of, eps, theta);
  for (int h = 0; h < hk; ++h) {
    norm_rope_head(row + (int64_t)(hq + h) * HEAD, kdst + h * kstride, k_norm, pos_of, eps, theta);
    memcpy(vdst + h * vstride, row + (int64_t)(hq + hk + h) * HEAD, HEAD * sizeof(bf16_t));
  }
}

/* qwen3_rope: q in place, K and V to slot slots[n] of kv [slot][2 hk][128]. */
void oracle_qwen3_rope(bf16_t* qkv, const bf16_t* q_norm, const bf16_t* k_norm, const int32_t* pos,
                       const int32_t* slots, bf16_t* kv, int rows, int hq, int hk, float eps, float theta) {
  const int64_t ld = (int64_t)(hq + 2 * hk) * HEAD;
  int pos_of[HEAD / 2];
  for (int n = 0; n < rows; ++n) {
    for (int i = 0; i < HEAD / 2; ++i) pos_of[i] = pos[n];
    bf16_t* k = kv + (int64_t)slots[n] * 2 * hk * HEAD;
    rope_row(qkv, ld, q_norm, k_norm, n, pos_of, k, HEAD, k + (int64_t)hk * HEAD, HEAD, hq, hk, eps, theta);
  }
}

/* qwen3_rope_dense: row n at position base + n % per, slot (n / per) * span + pos. */
void oracle_qwen3_rope_dense(bf16_t* qkv, const bf16_t* q_norm, const bf16_t* k_norm, bf16_t* kv, int rows, int per,
                             int base, int span, int hq, int hk, float eps, float theta) {
  const int64_t ld = (int64_t)(hq + 2 * hk) * HEAD;
  int pos_of[HEAD / 2];
  for (int n = 0; n < rows; ++n) {
    const int p = base + n % per;
    for (int i = 0; i < HEAD / 2; ++i) pos_of[i] = p;
    bf16_t* k = kv + ((int64_t)(n / per) * span + p) * 2 * hk * HEAD;
    rope_row(qkv, ld, q_norm, k_norm, n, pos_of, k, HEAD, k + (int64_t)hk * HEAD, HEAD, hq, hk, eps, theta);
  }
}

/* hidream_qk_rope: pair i turns by positions[3n + (i < 3 mrope_hw ? i % 3 : 0)];
 * K and V to row slots[n] of the caches [slots][hk][128]. */
void oracle_hidream_qk_rope(bf16_t* qkv, int ld, const bf16_t* q_norm, const bf16_t* k_norm, const int32_t* positions,
                            const int32_t* slots, bf16_t* k_cache, bf16_t* v_cache, int rows, int hq, int hk,
                            int mrope_hw, float eps, float theta) {
  int pos_of[HEAD / 2];
  for (int n = 0; n < rows; ++n) {
    for (int i = 0; i < HEAD / 2; ++i) pos_of[i] = positions[3 * (int64_t)n + (i < 3 * mrope_hw ? i % 3 : 0)];
    const int64_t s = slots[n];
    rope_row(qkv, ld, q_norm, k_norm, n, pos_of, k_cache + s * hk * HEAD, HEAD, v_cache + s * hk * HEAD, HEAD, hq,
             hk, eps, theta);
  }
}

/* Interleaved rotation of one head of d dims: pair (x[2i], x[2i+1]) by pos * exp(i * coef). */
static void rope_interleaved_d(const bf16_t* src, float* out, float pos, float coef, int d) {
  for (int i = 0; i < d / 2; ++i) {
    const float freq = expf((float)i * coef);
    const float ang = freq * pos;
    const float sn = sinf(ang), cs = cosf(ang);
    const float re = bf2f(src[2 * i]), im = bf2f(src[2 * i + 1]);
    out[2 * i] = re * cs - im * sn;
    out[2 * i + 1] = re * sn + im * cs;
  }
}

static void rope_interleaved(const bf16_t* src, float* out, float pos, float coef) {
  rope_interleaved_d(src, out, pos, coef, HEAD);
}

static void quantize_head(const float* x, uint8_t* dst, float* scale) {
  float amax = 0.f;
  for (int i = 0; i < HEAD; ++i) amax = fmaxf(amax, fabsf(x[i]));
  const float sc = fmaxf(amax * (1.f / 448.f), 1e-12f);
  const float inv = 1.f / sc;
  for (int i = 0; i < HEAD; ++i) dst[i] = oracle_f32_to_e4m3(x[i] * inv);
  *scale = sc;
}

/* lm_rope: q rotated in place (bf16), k rotated then FP8 with its scale, v FP8
 * with its scale, into slot slots[n] of [K heads | V heads | K scales | V scales]. */
void oracle_lm_rope(bf16_t* qkv, const int32_t* pos, const int32_t* slots, uint8_t* kv, int rows, int heads,
                    float coef) {
  const int64_t slot_bytes = 2LL * heads * HEAD + 2LL * heads * 4;
  float x[HEAD];
  for (int n = 0; n < rows; ++n) {
    bf16_t* row = qkv + (int64_t)n * 3 * heads * HEAD;
    const float p = (float)pos[n];
    uint8_t* slot = kv + (int64_t)slots[n] * slot_bytes;
    float* scales = (float*)(slot + 2LL * heads * HEAD);
    for (int h = 0; h < heads; ++h) {
      rope_interleaved(row + h * HEAD, x, p, coef);
      for (int i = 0; i < HEAD; ++i) row[h * HEAD + i] = f2bf(x[i]);
    }
    for (int h = 0; h < heads; ++h) {
      rope_interleaved(row + (int64_t)(heads + h) * HEAD, x, p, coef);
      quantize_head(x, slot + (int64_t)h * HEAD, &scales[h]);
    }
    for (int h = 0; h < heads; ++h) {
      const bf16_t* v = row + (int64_t)(2 * heads + h) * HEAD;
      for (int i = 0; i < HEAD; ++i) x[i] = bf2f(v[i]);
      quantize_head(x, slot + (int64_t)(heads + h) * HEAD, &scales[heads + h]);
    }
  }
}

/* ------------------------------------------------ head-64 ring attentions */

#define D64 64

/* mimi_rope_kv (mimi.cu:226-246 with rope_head<64>, attend.cuh:108-129): row n
 * of session s = n / T at p = pos[s] * T + n % T; the q heads of qkv row n
 * [q | k | v][heads][64] turned in place, the k heads turned into ring slot
 * p % context of the session's state (state + lines[s] * stride bytes, slots
 * [2 heads][64]: K heads then V heads), the v heads copied there. */
void oracle_mimi_rope_kv(bf16_t* qkv, const int32_t* pos, const int32_t* lines, uint8_t* state, int rows, int T,
                         int heads, float coef, int context, int64_t stride) {
  float x[D64];
  for (int n = 0; n < rows; ++n) {
    const int s = n / T;
    const int p = pos[s] * T + n % T;
    bf16_t* row = qkv + (int64_t)n * 3 * heads * D64;
    bf16_t* ring = (bf16_t*)(state + (int64_t)lines[s] * stride);
    bf16_t* slot = ring + (int64_t)(p % context) * 2 * heads * D64;
    for (int h = 0; h < 2 * heads; ++h) {
      rope_interleaved_d(row + (int64_t)h * D64, x, (float)p, coef, D64);
      bf16_t* dst = h < heads ? row + (int64_t)h * D64 : slot + (int64_t)(h - heads) * D64;
      for (int i = 0; i < D64; ++i) dst[i] = f2bf(x[i]);
    }
    memcpy(slot + (int64_t)heads * D64, row + (int64_t)2 * heads * D64, (size_t)heads * D64 * sizeof(bf16_t));
  }
}

/* lm_copy_kv (lm.cu:583-593): slot dst_slot[r] of one layer's cache takes the
 * bytes of slot src_slot[r], for r < tokens (prefix K/V reuse). */
void oracle_lm_copy_kv(uint8_t* kv, const int32_t* src_slot, const int32_t* dst_slot, int tokens, int slot_bytes) {
  for (int r = 0; r < tokens; ++r)
    memmove(kv + (int64_t)dst_slot[r] * slot_bytes, kv + (int64_t)src_slot[r] * slot_bytes, (size_t)slot_bytes);
}

/* attend_row<64> (attend.cuh:41-106) for one (row, head): q (64 f32), keys
 * t = 0 .. len-1 with K row krow(t) and V row vrow(t); 4 warps x 32-key tiles,
 * online softmax with natural exp per tile, warps merged at the end. */
static void attend_row64(const float* q, const bf16_t* const* krow, const bf16_t* const* vrow, int len, float scale,
                         bf16_t* out) {
  float M[WARPS], L[WARPS], O[WARPS][D64];
  for (int w = 0; w < WARPS; ++w) {
    float m = -INFINITY, l = 0.f;
    for (int d = 0; d < D64; ++d) O[w][d] = 0.f;
    for (int base = w * LANES; base < len; base += WARPS * LANES) {
      float sv[LANES], p[LANES];
      float tmax = -INFINITY;
      for (int lane = 0; lane < LANES; ++lane) {
        const int t = base + lane;
        const bf16_t* k = krow[t < len ? t : base];
        float dot = 0.f;
        for (int d = 0; d < D64; ++d) dot += q[d] * bf2f(k[d]);
        sv[lane] = t < len ? dot * scale : -INFINITY;
        if (sv[lane] > tmax) tmax = sv[lane];
      }
      const float m2 = fmaxf(m, tmax);
      const float corr = expf(m - m2);
      for (int lane = 0; lane < LANES; ++lane) p[lane] = expf(sv[lane] - m2);
      l = l * corr + bfly_sum(p);
      for (int d = 0; d < D64; ++d) O[w][d] *= corr;
      m = m2;
      const int count = len - base < LANES ? len - base : LANES;
      for (int j = 0; j < count; ++j)
        for (int d = 0; d < D64; ++d) O[w][d] += p[j] * bf2f(vrow[base + j][d]);
    }
    M[w] = m;
    L[w] = l;
  }
  float top = -INFINITY;
  for (int w = 0; w < WARPS; ++w) top = fmaxf(top, M[w]);
  for (int d = 0; d < D64; ++d) {
    float num = 0.f, den = 0.f;
    for (int w = 0; w < WARPS; ++w) {
      const float e = M[w] == -INFINITY ? 0.f : expf(M[w] - top);
      num += O[w][d] * e;
      den += L[w] * e;
    }
    out[d] = f2bf(num / den);
  }
}

/* mimi_attend: row n of session s = n / T at position p = pos[s] * T + n % T
 * sees len = min(p + 1, context) ring slots (p - len + 1 + t) % context of the
 * session's ring at state + lines[s] * stride bytes, slots [2 heads][64]. */
void oracle_mimi_attend(const bf16_t* qkv, const int32_t* pos, const int32_t* lines, const uint8_t* state,
                        bf16_t* out, int rows, int T, int heads, float scale, int context, int64_t stride) {
  const bf16_t** krow = (const bf16_t**)malloc(sizeof(bf16_t*) * (size_t)context);
  const bf16_t** vrow = (const bf16_t**)malloc(sizeof(bf16_t*) * (size_t)context);
  float q[D64];
  for (int n = 0; n < rows; ++n) {
    const int s = n / T, p = pos[s] * T + n % T;
    const int len = p + 1 < context ? p + 1 : context;
    const bf16_t* ring = (const bf16_t*)(state + (int64_t)lines[s] * stride);
    for (int h = 0; h < heads; ++h) {
      for (int t = 0; t < len; ++t) {
        const int64_t slot = (p - len + 1 + t) % context;
        krow[t] = ring + (slot * 2 * heads + h) * D64;
        vrow[t] = ring + (slot * 2 * heads + heads + h) * D64;
      }
      const bf16_t* qh = qkv + ((int64_t)n * 3 * heads + h) * D64;
      for (int d = 0; d < D64; ++d) q[d] = bf2f(qh[d]);
      attend_row64(q, krow, vrow, len, scale, out + ((int64_t)n * heads + h) * D64);
    }
  }
  free(krow);
  free(vrow);
}

#define CODEC_WINDOW 72

/* codec_attention for session r, head h: q and k turned by the half-split
 * rotary at p = pos[r] (pair i = elements i, i + 32, angle p * theta^(-2i/64))
 * and rounded to bf16; k and v written to frame p % 72 of the ring at
 * kv + lines[r] * stride bytes (K[72][heads * 64] then V[72][heads * 64]);
 * then q against frames p - n + 1 .. p, n = min(p + 1, 72), scale 1/8, one
 * softmax over all n scores (max, sum of exp, then the weighted V rows). */
void oracle_codec_attention(const bf16_t* qkv, const int32_t* pos, const int32_t* lines, uint8_t* kv, bf16_t* out,
                            int rows, int64_t stride, int heads, float theta) {
  const int width = heads * D64;
  for (int r = 0; r < rows; ++r) {
    bf16_t* ring = (bf16_t*)(kv + (int64_t)lines[r] * stride);
    const int p = pos[r];
    const int n = p + 1 < CODEC_WINDOW ? p + 1 : CODEC_WINDOW;
    const int64_t vofs = (int64_t)CODEC_WINDOW * width;
    for (int h = 0; h < heads; ++h) {
      const bf16_t* row = qkv + (int64_t)r * 3 * width + h * D64;
      float q[D64];
      bf16_t krot[D64];
      for (int w = 0; w < 2; ++w) {
        const bf16_t* src = row + (int64_t)w * width;
        for (int i = 0; i < D64 / 2; ++i) {
          const float inv_freq = 1.f / powf(theta, (float)(2 * i) / D64);
          const float ang = (float)p * inv_freq;
          const float sn = sinf(ang), cs = cosf(ang);
          const float lo = bf2f(src[i]), hi = bf2f(src[i + D64 / 2]);
          const bf16_t a = f2bf(lo * cs - hi * sn), b = f2bf(hi * cs + lo * sn);
          if (w == 0) {
            q[i] = bf2f(a);
            q[i + D64 / 2] = bf2f(b);
          } else {
            krot[i] = a;
            krot[i + D64 / 2] = b;
          }
        }
      }
      const int64_t at = (int64_t)(p % CODEC_WINDOW) * width + h * D64;
      memcpy(ring + at, krot, sizeof krot);
      memcpy(ring + vofs + at, row + 2LL * width, D64 * sizeof(bf16_t));
      float sc[CODEC_WINDOW];
      float m = -INFINITY;
      const int j0 = p - n + 1;
      for (int j = 0; j < n; ++j) {
        const bf16_t* k = ring + (int64_t)((j0 + j) % CODEC_WINDOW) * width + h * D64;
        float dot = 0.f;
        for (int d = 0; d < D64; ++d) dot += q[d] * bf2f(k[d]);
        sc[j] = dot * (1.f / sqrtf((float)D64));
        if (sc[j] > m) m = sc[j];
      }
      float l = 0.f, acc[D64];
      for (int d = 0; d < D64; ++d) acc[d] = 0.f;
      for (int j = 0; j < n; ++j) {
        const float pj = expf(sc[j] - m);
        l += pj;
        const bf16_t* v = ring + vofs + (int64_t)((j0 + j) % CODEC_WINDOW) * width + h * D64;
        for (int d = 0; d < D64; ++d) acc[d] += pj * bf2f(v[d]);
      }
      for (int d = 0; d < D64; ++d) out[(int64_t)r * width + h * D64 + d] = f2bf(acc[d] / l);
    }
  }
}

#define DEP_STEPS 8

/* lm_dep_kv_attend for session s, head h at depformer step `step`: K and V of
 * the row into step `step` of the session's workspace ws[s][8][K | V][heads*64],
 * then q against steps 0 .. step in order with a running (m, l) updated per key
 * in natural exp, output acc / l. */
void oracle_lm_dep_kv_attend(const bf16_t* qkv, bf16_t* ws, int step, bf16_t* out, int seqs, int heads, float scale) {
  const int width = heads * D64;
  for (int s = 0; s < seqs; ++s) {
    const bf16_t* row = qkv + (int64_t)s * 3 * width;
    const int64_t base = (int64_t)s * DEP_STEPS * 2 * width;
    for (int h = 0; h < heads; ++h) {
      memcpy(ws + base + (int64_t)step * 2 * width + h * D64, row + width + h * D64, D64 * sizeof(bf16_t));
      memcpy(ws + base + (int64_t)step * 2 * width + width + h * D64, row + 2 * width + h * D64,
             D64 * sizeof(bf16_t));
    }
    for (int h = 0; h < heads; ++h) {
      float m = -INFINITY, l = 0.f, acc[D64];
      for (int d = 0; d < D64; ++d) acc[d] = 0.f;
      for (int t = 0; t <= step; ++t) {
        const bf16_t* k = ws + base + (int64_t)t * 2 * width + h * D64;
        const bf16_t* v = k + width;
        float dot = 0.f;
        for (int d = 0; d < D64; ++d) dot += bf2f(row[h * D64 + d]) * bf2f(k[d]);
        const float sc = dot * scale;
        const float m2 = fmaxf(m, sc);
        const float corr = expf(m - m2), p = expf(sc - m2);
        l = l * corr + p;
        for (int d = 0; d < D64; ++d) acc[d] = acc[d] * corr + p * bf2f(v[d]);
        m = m2;
      }
      for (int d = 0; d < D64; ++d) out[(int64_t)s * width + h * D64 + d] = f2bf(acc[d] * (1.f / l));
    }
  }
}
