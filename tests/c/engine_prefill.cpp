// Native prefill and DiT steps over the C ABI, the way the engines' runtime
// drives them. No Python and no torch: HIP runtime calls and the omni_attn C
// ABI only.
//
// Higgs-style chunked prefill (crates/omni-higgs-audio/src/model.rs:277-313
// builds the rows; crates/omni-qwen3/src/stack.rs:207-241 runs qwen3_rope then
// qwen3_attend(ragged = 1)): sessions with cached tokens each append a chunk.
// The host builds the rows with omni_attn_rows_push (count > 1), checks the
// table, plans the MFMA prefill (omni_attn_prefill_plan_init, sized by a first
// call without a work list) and uploads the work list; the device runs
// omni_qwen3_rope, omni_attn_prefill_run, and the decode kernel on the same
// ragged rows. Checked against the CPU oracle (rotary + scatter, paged
// attention): both outputs within max-abs 2e-2 / mean-abs 2e-3, V of every
// written cache slot bit-exact, K within the rotary rounding bound.
//
// HiDream-O1 step (crates/omni-hidream-o1/src/model.rs:123-160): the prompt's
// text rows, then the generation rows from omni_hidream_rows, each through
// omni_hidream_qk_rope into the separate K and V caches, then
// omni_hidream_attend_ws over the generation rows with *kv_len_at keys. The
// generation step (rotary + attention) is captured once as a HIP graph and
// replayed with a new *kv_len_at written on the device; every replay is
// checked against an eager run (bit-identical) and the oracle (tolerance).
// Prints "engine_prefill: ok" and exits 0, or names the failed check and exits 1.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "omni_attn.h"

extern "C" {
// The CPU oracle (oracle/omni_attn_oracle.c), test infrastructure.
int oracle_paged_attend(const uint16_t* qkv, const uint16_t* kv, const int32_t* pos, const int32_t* seq, int ragged,
                        const int32_t* indptr, const int32_t* pages, int page, uint16_t* out, int rows, int hq, int hk,
                        float scale, int context, int nthreads);
void oracle_qwen3_rope(uint16_t* qkv, const uint16_t* q_norm, const uint16_t* k_norm, const int32_t* pos,
                       const int32_t* slots, uint16_t* kv, int rows, int hq, int hk, float eps, float theta);
int oracle_dense_attend(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out, int q_len, int kv_len,
                        int q_stride, int hq, int hk, int causal, float scale_log2, int nthreads);
void oracle_hidream_qk_rope(uint16_t* qkv, int ld, const uint16_t* q_norm, const uint16_t* k_norm,
                            const int32_t* positions, const int32_t* slots, uint16_t* k_cache, uint16_t* v_cache,
                            int rows, int hq, int hk, int mrope_hw, float eps, float theta);
}

namespace {

#define HIP_OK(x)                                                                              \
  do {                                                                                         \
    hipError_t e_ = (x);                                                                       \
    if (e_ != hipSuccess) {                                                                    \
      fprintf(stderr, "engine_prefill: %s failed: %s (line %d)\n", #x, hipGetErrorString(e_), \
              __LINE__);                                                                       \
      exit(1);                                                                                 \
    }                                                                                          \
  } while (0)
#define OMNI_OK(x)                                                                                               \
  do {                                                                                                           \
    int r_ = (x);                                                                                                \
    if (r_ != OMNI_ATTN_OK) {                                                                                    \
      fprintf(stderr, "engine_prefill: %s returned %d: %s (line %d)\n", #x, r_, omni_attn_last_error(), __LINE__); \
      exit(1);                                                                                                   \
    }                                                                                                            \
  } while (0)

void fail(const char* what) {
  fprintf(stderr, "engine_prefill: %s\n", what);
  exit(1);
}

uint64_t g_rng = 0x2545F4914F6CDD1Dull;
uint64_t next_u64() {  // splitmix64
  uint64_t z = (g_rng += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
float uniform() { return (float)((next_u64() >> 11) * (1.0 / 9007199254740992.0)); }
float normal() {
  const float u = uniform() + 1e-12f, v = uniform();
  return std::sqrt(-2.f * std::log(u)) * std::cos(6.2831853f * v);
}
uint16_t bf16(float f) {  // round to nearest even
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7FFF + ((u >> 16) & 1);
  return (uint16_t)(u >> 16);
}
float from_bf16(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
std::vector<uint16_t> normals(size_t n, float sd = 1.f) {
  std::vector<uint16_t> x(n);
  for (auto& e : x) e = bf16(sd * normal());
  return x;
}

template <typename T>
T* dev_upload(const std::vector<T>& h) {
  void* d = nullptr;
  HIP_OK(hipMalloc(&d, h.size() * sizeof(T) + 16));
  HIP_OK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
  return static_cast<T*>(d);
}
template <typename T>
std::vector<T> dev_download(const void* d, size_t n) {
  std::vector<T> h(n);
  HIP_OK(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
  return h;
}

// Max-abs and mean-abs of got against want (bf16 bits), within the tolerance.
void check_close(const std::vector<uint16_t>& got, const std::vector<uint16_t>& want, const char* what,
                 double* worst_max) {
  double mx = 0, sum = 0;
  for (size_t i = 0; i < got.size(); ++i) {
    const double g = from_bf16(got[i]), w = from_bf16(want[i]);
    if (!std::isfinite(g)) fail("non-finite output");
    mx = std::fmax(mx, std::fabs(g - w));
    sum += std::fabs(g - w);
  }
  const double mean = sum / (double)got.size();
  if (mx > 2e-2 || mean > 2e-3) {
    fprintf(stderr, "engine_prefill: %s: max-abs %.3g mean-abs %.3g\n", what, mx, mean);
    fail("output outside the tolerance against the oracle");
  }
  *worst_max = std::fmax(*worst_max, mx);
}

// ---------------------------------------------------------------- prefill
double prefill_step() {
  constexpr int kHq = 32, kHk = 8, kD = 128, kPage = 16, kSessions = 4, kLeasePages = 64;
  constexpr int kRow = (kHq + 2 * kHk) * kD, kSlot = 2 * kHk * kD;
  constexpr int kPool = kSessions * kLeasePages + 5;
  const float scale = 1.f / std::sqrt((float)kD), eps = 1e-6f, theta = 1e6f;

  std::vector<int32_t> perm(kPool);
  for (int i = 0; i < kPool; ++i) perm[i] = i;
  for (int i = kPool - 1; i > 0; --i) std::swap(perm[i], perm[next_u64() % (uint64_t)(i + 1)]);
  omni_attn_rows* rows = omni_attn_rows_new(kPage, 0);
  if (!rows) fail("rows_new");
  int max_len = 0;
  for (int s = 0; s < kSessions; ++s) {
    const int cached = (int)(next_u64() % 401), chunk = 50 + (int)(next_u64() % 251);
    OMNI_OK(omni_attn_rows_push(rows, perm.data() + s * kLeasePages, kLeasePages, cached, chunk, s));
    max_len = std::max(max_len, cached + chunk);
  }
  int nrows = 0, nseqs = 0, npages = 0;
  OMNI_OK(omni_attn_rows_count(rows, &nrows, &nseqs, &npages));
  const int32_t* pos_h = omni_attn_rows_get(rows, OMNI_ATTN_ROWS_POS);
  const int32_t* slot_h = omni_attn_rows_get(rows, OMNI_ATTN_ROWS_SLOT);
  const int32_t* seq_h = omni_attn_rows_get(rows, OMNI_ATTN_ROWS_SEQ);
  const int32_t* indptr_h = omni_attn_rows_get(rows, OMNI_ATTN_ROWS_INDPTR);
  const int32_t* pages_h = omni_attn_rows_get(rows, OMNI_ATTN_ROWS_PAGES);
  OMNI_OK(omni_attn_check_table(indptr_h, nseqs, pages_h, kPool, pos_h, seq_h, 1, nrows, kPage, 0));

  // The cache holds every session's cached tokens already (random contents).
  const std::vector<uint16_t> kv_h = normals((size_t)kPool * kPage * kSlot);
  const std::vector<uint16_t> qkv_h = normals((size_t)nrows * kRow);
  std::vector<uint16_t> qn_h(kD), kn_h(kD);
  for (int i = 0; i < kD; ++i) qn_h[i] = bf16(1.f + 0.1f * normal()), kn_h[i] = bf16(1.f + 0.1f * normal());
  uint16_t* kv = dev_upload(kv_h);
  uint16_t* qkv = dev_upload(qkv_h);
  uint16_t* qn = dev_upload(qn_h);
  uint16_t* kn = dev_upload(kn_h);
  int32_t* pos = dev_upload(std::vector<int32_t>(pos_h, pos_h + nrows));
  int32_t* slot = dev_upload(std::vector<int32_t>(slot_h, slot_h + nrows));
  int32_t* seq = dev_upload(std::vector<int32_t>(seq_h, seq_h + nrows));
  int32_t* indptr = dev_upload(std::vector<int32_t>(indptr_h, indptr_h + nseqs + 1));
  int32_t* pages = dev_upload(std::vector<int32_t>(pages_h, pages_h + npages));

  // Host plan: the first call reports the work list size.
  omni_attn_prefill_plan plan;
  if (omni_attn_prefill_plan_init(nrows, kHq, kHk, kPage, seq_h, pos_h, nullptr, 0, &plan) != OMNI_ATTN_EWORKSPACE)
    fail("prefill_plan without a work list must report its size");
  std::vector<int32_t> work_h((size_t)(plan.work_bytes / 4));
  OMNI_OK(omni_attn_prefill_plan_init(nrows, kHq, kHk, kPage, seq_h, pos_h, work_h.data(), (int64_t)work_h.size(),
                                      &plan));
  int32_t* work = dev_upload(work_h);
  omni_attn_decode_plan dplan;
  OMNI_OK(omni_attn_decode_plan_init(nrows, kHq, kHk, kPage, max_len, 0, &dplan));
  void* ws = nullptr;
  if (dplan.workspace_bytes > 0) HIP_OK(hipMalloc(&ws, (size_t)dplan.workspace_bytes));
  void *out_p, *out_d;
  HIP_OK(hipMalloc(&out_p, (size_t)nrows * kHq * kD * 2));
  HIP_OK(hipMalloc(&out_d, (size_t)nrows * kHq * kD * 2));

  hipStream_t st;
  HIP_OK(hipStreamCreate(&st));
  OMNI_OK(omni_qwen3_rope(qkv, qn, kn, pos, slot, kv, nrows, kHq, kHk, eps, theta, st));
  OMNI_OK(omni_attn_prefill_run(&plan, qkv, kv, pos, seq, indptr, pages, out_p, scale, work, st));
  OMNI_OK(omni_qwen3_attend(qkv, kv, pos, seq, 1, indptr, pages, kPage, out_d, kHq, kHk, scale, &dplan, ws, st));
  HIP_OK(hipStreamSynchronize(st));

  std::vector<uint16_t> q_o = qkv_h, kv_o = kv_h, out_o((size_t)nrows * kHq * kD);
  oracle_qwen3_rope(q_o.data(), qn_h.data(), kn_h.data(), pos_h, slot_h, kv_o.data(), nrows, kHq, kHk, eps, theta);
  if (oracle_paged_attend(q_o.data(), kv_o.data(), pos_h, seq_h, 1, indptr_h, pages_h, kPage, out_o.data(), nrows,
                          kHq, kHk, scale, 0, 8) != 0)
    fail("oracle");
  double worst = 0;
  check_close(dev_download<uint16_t>(out_p, out_o.size()), out_o, "prefill (MFMA)", &worst);
  check_close(dev_download<uint16_t>(out_d, out_o.size()), out_o, "prefill rows through decode", &worst);
  // The same plan with exact_p set (P as two bf16 terms, the reference's f32-P
  // numerics) on the rotated rows: within the tolerance too, and in bf16 bits
  // the decode kernel's output on all but a few elements.
  {
    omni_attn_prefill_plan xplan = plan;
    xplan.exact_p = 1;
    OMNI_OK(omni_attn_prefill_run(&xplan, qkv, kv, pos, seq, indptr, pages, out_p, scale, work, st));
    HIP_OK(hipStreamSynchronize(st));
    const std::vector<uint16_t> got_x = dev_download<uint16_t>(out_p, out_o.size());
    check_close(got_x, out_o, "prefill (MFMA, exact_p)", &worst);
    const std::vector<uint16_t> got_d = dev_download<uint16_t>(out_d, out_o.size());
    size_t same = 0;
    for (size_t i = 0; i < got_x.size(); ++i) same += got_x[i] == got_d[i];
    if (same * 100 < got_x.size() * 99) fail("exact_p prefill differs from the f32-P decode kernel on > 1% of elements");
    std::printf("prefill exact_p: %.4f of elements equal the decode kernel's\n", (double)same / got_x.size());
  }
  // V of every written slot is copied: bytes must match. K is rotated with
  // device math: within one bf16 ulp plus (2^-8 + pos * 2^-21) of its rotary
  // pair's magnitude (a last-bit difference in rsqrt or in the angle), and
  // mostly bit-identical.
  const std::vector<uint16_t> kv_g = dev_download<uint16_t>(kv, kv_h.size());
  size_t k_equal = 0;
  for (int n = 0; n < nrows; ++n) {
    const size_t s0 = (size_t)slot_h[n] * kSlot;
    if (std::memcmp(&kv_g[s0 + kHk * kD], &kv_o[s0 + kHk * kD], kHk * kD * 2) != 0)
      fail("V bytes of a written slot");
    for (int i = 0; i < kHk * kD; ++i) {
      const double g = from_bf16(kv_g[s0 + i]), w = from_bf16(kv_o[s0 + i]);
      const double pair = std::fmax(std::fabs(w), std::fabs(from_bf16(kv_o[s0 + (i ^ 64)])));
      const double ulp = std::ldexp(1.0, std::ilogb(std::fmax(std::fabs(w), 1e-30)) - 7);
      if (std::fabs(g - w) > ulp * 1.0001 + (std::ldexp(1.0, -8) + pos_h[n] * std::ldexp(1.0, -21)) * pair)
        fail("K of a written slot outside the rotary rounding bound");
      k_equal += kv_g[s0 + i] == kv_o[s0 + i];
    }
  }
  if (k_equal < (size_t)(0.95 * nrows * kHk * kD)) fail("K of the written slots mostly not bit-identical");
  printf("engine_prefill: prefill of %d rows over %d sessions ok (max-abs %.3g)\n", nrows, nseqs, worst);
  omni_attn_rows_free(rows);
  HIP_OK(hipStreamDestroy(st));
  return worst;
}

// ---------------------------------------------------------------- HiDream
double dit_step() {
  constexpr int kHq = 32, kHk = 8, kD = 128, kText = 77, kGridR = 8, kGridC = 8, kMropeHw = 20;
  constexpr int kLd = (kHq + 2 * kHk) * kD;
  constexpr int kGen = 1 + kGridR * kGridC, kKeys = kText + kGen;
  const float eps = 1e-6f, theta = 5e6f, scale_log2 = (1.f / std::sqrt((float)kD)) * 1.4426950408889634f;

  std::vector<int32_t> text_pos(3 * kText), text_slot(kText), gen_pos(3 * kGen), gen_slot(kGen);
  int32_t step_kv = 0;
  OMNI_OK(omni_hidream_rows(kText, kGridR, kGridC, 4096, text_pos.data(), text_slot.data(), gen_pos.data(),
                            gen_slot.data(), &step_kv));
  if (step_kv != kKeys) fail("hidream_rows key count");

  std::vector<uint16_t> qn_h(kD), kn_h(kD);
  for (int i = 0; i < kD; ++i) qn_h[i] = bf16(1.f + 0.1f * normal()), kn_h[i] = bf16(1.f + 0.1f * normal());
  const std::vector<uint16_t> text_h = normals((size_t)kText * kLd);
  uint16_t* qn = dev_upload(qn_h);
  uint16_t* kn = dev_upload(kn_h);
  uint16_t* text = dev_upload(text_h);
  uint16_t* gen_src = dev_upload(std::vector<uint16_t>((size_t)kGen * kLd));
  uint16_t* gen = dev_upload(std::vector<uint16_t>((size_t)kGen * kLd));
  uint16_t* kc = dev_upload(std::vector<uint16_t>((size_t)kKeys * kHk * kD));
  uint16_t* vc = dev_upload(std::vector<uint16_t>((size_t)kKeys * kHk * kD));
  int32_t* tpos = dev_upload(text_pos);
  int32_t* tslot = dev_upload(text_slot);
  int32_t* gpos = dev_upload(gen_pos);
  int32_t* gslot = dev_upload(gen_slot);
  int32_t* kv_len = dev_upload(std::vector<int32_t>{kKeys});
  void *out, *out_e, *ws;
  HIP_OK(hipMalloc(&out, (size_t)kGen * kHq * kD * 2));
  HIP_OK(hipMalloc(&out_e, (size_t)kGen * kHq * kD * 2));
  const int64_t ws_bytes = omni_hidream_workspace_bytes();
  HIP_OK(hipMalloc(&ws, (size_t)ws_bytes));

  hipStream_t st;
  HIP_OK(hipStreamCreate(&st));
  // The prompt: its text rows' K and V into the caches.
  OMNI_OK(omni_hidream_qk_rope(text, kLd, qn, kn, tpos, tslot, kc, vc, kText, kHq, kHk, kMropeHw, eps, theta, st));
  auto launch = [&](void* o) {
    HIP_OK(hipMemcpyAsync(gen, gen_src, (size_t)kGen * kLd * 2, hipMemcpyDeviceToDevice, st));
    OMNI_OK(omni_hidream_qk_rope(gen, kLd, qn, kn, gpos, gslot, kc, vc, kGen, kHq, kHk, kMropeHw, eps, theta, st));
    OMNI_OK(omni_hidream_attend_ws(gen, kc, vc, o, kGen, kv_len, kLd, 0, scale_log2, kHq, kHk, 1, 0, 0, 0, ws,
                                   ws_bytes, st));
  };
  hipGraph_t graph;
  hipGraphExec_t exec;
  HIP_OK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
  launch(out);
  HIP_OK(hipStreamEndCapture(st, &graph));
  HIP_OK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));

  std::vector<uint16_t> t_o = text_h, kc_o((size_t)kKeys * kHk * kD), vc_o(kc_o.size());
  oracle_hidream_qk_rope(t_o.data(), kLd, qn_h.data(), kn_h.data(), text_pos.data(), text_slot.data(), kc_o.data(),
                         vc_o.data(), kText, kHq, kHk, kMropeHw, eps, theta);
  double worst = 0;
  // Replays with a new generation input and fewer keys each time (the last
  // generation rows' keys dropped): the captured *kv_len_at is re-read.
  for (int rep = 0; rep < 3; ++rep) {
    const int keys = kKeys - 5 * rep;
    const std::vector<uint16_t> gen_h = normals((size_t)kGen * kLd);
    HIP_OK(hipMemcpy(gen_src, gen_h.data(), gen_h.size() * 2, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(kv_len, &keys, 4, hipMemcpyHostToDevice));
    HIP_OK(hipGraphLaunch(exec, st));
    HIP_OK(hipStreamSynchronize(st));
    launch(out_e);
    HIP_OK(hipStreamSynchronize(st));
    const std::vector<uint16_t> got = dev_download<uint16_t>(out, (size_t)kGen * kHq * kD);
    if (got != dev_download<uint16_t>(out_e, got.size())) fail("DiT graph replay differs from the eager step");
    std::vector<uint16_t> g_o = gen_h, kcr = kc_o, vcr = vc_o, out_o(got.size());
    oracle_hidream_qk_rope(g_o.data(), kLd, qn_h.data(), kn_h.data(), gen_pos.data(), gen_slot.data(), kcr.data(),
                           vcr.data(), kGen, kHq, kHk, kMropeHw, eps, theta);
    if (oracle_dense_attend(g_o.data(), kcr.data(), vcr.data(), out_o.data(), kGen, keys, kLd, kHq, kHk, 0, scale_log2,
                            8) != 0)
      fail("oracle");
    check_close(got, out_o, "DiT step", &worst);
  }
  printf("engine_prefill: HiDream step (%d text + %d generation rows, 3 graph replays) ok (max-abs %.3g)\n", kText,
         kGen, worst);
  HIP_OK(hipGraphExecDestroy(exec));
  HIP_OK(hipGraphDestroy(graph));
  HIP_OK(hipStreamDestroy(st));
  return worst;
}

}  // namespace

int main() {
  prefill_step();
  dit_step();
  printf("engine_prefill: ok\n");
  return 0;
}
