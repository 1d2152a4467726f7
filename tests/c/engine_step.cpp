// A native engine loop over the C ABI, the way the engines' runtime drives it
// (crates/omni-qwen3-tts/src/model.rs:266-303 builds a step's rows; the decode
// program of crates/omni-qwen3/src/stack.rs:207-241 runs qwen3_rope then
// qwen3_attend, captured as one graph per batch bucket per
// docs/qwen3-tts.md:28-29). No Python and no torch: HIP runtime calls and the
// omni_attn C ABI only.
//
// Per step: every session appends one token. The host builds the step's rows
// with omni_attn_rows_* from each session's page lease, checks the table with
// omni_attn_check_table and uploads the arrays into fixed device buffers; the
// step itself (omni_qwen3_rope + omni_qwen3_attend on one stream) is captured
// once into a HIP graph and replayed for every later step. Each replay is
// checked two ways:
//   - against an eager run of the same step on the same inputs: bit-identical
//     outputs and cache;
//   - against the CPU oracle (rotary + scatter, then paged attention): outputs
//     within max-abs 2e-2 / mean-abs 2e-3, V bytes of the written slots exact.
// Prints "engine_step: ok" and exits 0, or names the failed check and exits 1.
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
}

namespace {

#define HIP_OK(x)                                                                            \
  do {                                                                                       \
    hipError_t e_ = (x);                                                                     \
    if (e_ != hipSuccess) {                                                                  \
      fprintf(stderr, "engine_step: %s failed: %s (line %d)\n", #x, hipGetErrorString(e_), \
              __LINE__);                                                                     \
      exit(1);                                                                               \
    }                                                                                        \
  } while (0)
#define OMNI_OK(x)                                                                                             \
  do {                                                                                                         \
    int r_ = (x);                                                                                              \
    if (r_ != OMNI_ATTN_OK) {                                                                                  \
      fprintf(stderr, "engine_step: %s returned %d: %s (line %d)\n", #x, r_, omni_attn_last_error(), __LINE__); \
      exit(1);                                                                                                 \
    }                                                                                                          \
  } while (0)

void fail(const char* what, int step) {
  fprintf(stderr, "engine_step: step %d: %s\n", step, what);
  exit(1);
}

uint64_t g_rng = 0x9E3779B97F4A7C15ull;
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

}  // namespace

int main() {
  constexpr int kHq = 16, kHk = 8, kD = 128, kPage = 16, kSessions = 24, kBucket = 32, kMaxLen = 1024;
  constexpr int kSteps = 5;
  constexpr int kRow = (kHq + 2 * kHk) * kD;  // qkv row elements
  constexpr int kSlot = 2 * kHk * kD;         // cache slot elements
  constexpr int kLeasePages = kMaxLen / kPage;
  constexpr int kPool = kSessions * kLeasePages + 7;
  const float scale = 1.f / std::sqrt((float)kD), eps = 1e-6f, theta = 1e6f;

  // Sessions: a lease of page ids from a shuffled pool and a current length.
  std::vector<int32_t> perm(kPool);
  for (int i = 0; i < kPool; ++i) perm[i] = i;
  for (int i = kPool - 1; i > 0; --i) std::swap(perm[i], perm[next_u64() % (uint64_t)(i + 1)]);
  std::vector<std::vector<int32_t>> lease(kSessions);
  std::vector<int> len(kSessions);
  for (int s = 0; s < kSessions; ++s) {
    lease[s].assign(perm.begin() + s * kLeasePages, perm.begin() + (s + 1) * kLeasePages);
    len[s] = 50 + (int)(next_u64() % 700);
  }

  // Device state: the paged cache (filled with N(0,1) bf16), norm weights,
  // the step's inputs and outputs, fixed-size row arrays for the bucket.
  std::vector<uint16_t> kv_h((size_t)kPool * kPage * kSlot), qn_h(kD), kn_h(kD);
  for (auto& x : kv_h) x = bf16(normal());
  for (int i = 0; i < kD; ++i) qn_h[i] = bf16(1.f + 0.1f * normal()), kn_h[i] = bf16(1.f + 0.1f * normal());
  void *kv, *kv_eager, *qn, *kn, *qkv_src, *qkv, *out, *out_eager, *ws = nullptr;
  int32_t *pos_d, *slot_d, *indptr_d, *pages_d;
  const size_t kv_bytes = kv_h.size() * 2;
  HIP_OK(hipMalloc(&kv, kv_bytes));
  HIP_OK(hipMalloc(&kv_eager, kv_bytes));
  HIP_OK(hipMalloc(&qn, kD * 2));
  HIP_OK(hipMalloc(&kn, kD * 2));
  HIP_OK(hipMalloc(&qkv_src, (size_t)kBucket * kRow * 2));
  HIP_OK(hipMalloc(&qkv, (size_t)kBucket * kRow * 2));
  HIP_OK(hipMalloc(&out, (size_t)kBucket * kHq * kD * 2));
  HIP_OK(hipMalloc(&out_eager, (size_t)kBucket * kHq * kD * 2));
  HIP_OK(hipMalloc(&pos_d, kBucket * 4));
  HIP_OK(hipMalloc(&slot_d, kBucket * 4));
  HIP_OK(hipMalloc(&indptr_d, (kBucket + 1) * 4));
  HIP_OK(hipMalloc(&pages_d, (size_t)kBucket * kLeasePages * 4));
  HIP_OK(hipMemcpy(kv, kv_h.data(), kv_bytes, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(qn, qn_h.data(), kD * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(kn, kn_h.data(), kD * 2, hipMemcpyHostToDevice));

  // One plan and one workspace for the bucket (rows = kSessions real rows).
  omni_attn_decode_plan plan;
  OMNI_OK(omni_attn_decode_plan_init(kSessions, kHq, kHk, kPage, kMaxLen, 128, &plan));
  if (plan.workspace_bytes > 0) HIP_OK(hipMalloc(&ws, (size_t)plan.workspace_bytes));
  omni_attn_rows* rows = omni_attn_rows_new(kPage, 0);
  if (!rows) fail("rows_new", -1);

  hipStream_t st;
  HIP_OK(hipStreamCreate(&st));
  auto launch_step = [&](void* kv_buf, void* out_buf) {
    HIP_OK(hipMemcpyAsync(qkv, qkv_src, (size_t)kSessions * kRow * 2, hipMemcpyDeviceToDevice, st));
    OMNI_OK(omni_qwen3_rope(qkv, qn, kn, pos_d, slot_d, kv_buf, kSessions, kHq, kHk, eps, theta, st));
    OMNI_OK(omni_qwen3_attend(qkv, kv_buf, pos_d, nullptr, 0, indptr_d, pages_d, kPage, out_buf, kHq, kHk, scale, &plan,
                              ws, st));
  };

  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  double worst_max = 0, worst_mean = 0;
  for (int step = 0; step < kSteps; ++step) {
    // Host: this step's rows (one new token per session) and inputs.
    omni_attn_rows_clear(rows);
    for (int s = 0; s < kSessions; ++s)
      OMNI_OK(omni_attn_rows_push(rows, lease[s].data(), kLeasePages, len[s], 1, s));
    int nrows = 0, nseqs = 0, npages = 0;
    OMNI_OK(omni_attn_rows_count(rows, &nrows, &nseqs, &npages));
    if (nrows != kSessions || nseqs != kSessions) fail("row count", step);
    const int32_t* pos_h = omni_attn_rows_get(rows, OMNI_ATTN_ROWS_POS);
    const int32_t* slot_h = omni_attn_rows_get(rows, OMNI_ATTN_ROWS_SLOT);
    const int32_t* indptr_h = omni_attn_rows_get(rows, OMNI_ATTN_ROWS_INDPTR);
    const int32_t* pages_h = omni_attn_rows_get(rows, OMNI_ATTN_ROWS_PAGES);
    OMNI_OK(omni_attn_check_table(indptr_h, nseqs, pages_h, kPool, pos_h, nullptr, 0, nrows, kPage, 0));
    std::vector<uint16_t> qkv_h((size_t)kSessions * kRow);
    for (auto& x : qkv_h) x = bf16(normal());
    HIP_OK(hipMemcpy(pos_d, pos_h, nrows * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(slot_d, slot_h, nrows * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(indptr_d, indptr_h, (nseqs + 1) * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(pages_d, pages_h, (size_t)npages * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(qkv_src, qkv_h.data(), qkv_h.size() * 2, hipMemcpyHostToDevice));

    // The cache before the step, for the oracle and the eager twin.
    std::vector<uint16_t> kv_before(kv_h.size());
    HIP_OK(hipMemcpy(kv_before.data(), kv, kv_bytes, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(kv_eager, kv, kv_bytes, hipMemcpyDeviceToDevice));

    // The step: captured once (step 0), replayed afterwards.
    if (!exec) {
      HIP_OK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
      launch_step(kv, out);
      HIP_OK(hipStreamEndCapture(st, &graph));
      HIP_OK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    }
    HIP_OK(hipGraphLaunch(exec, st));
    HIP_OK(hipStreamSynchronize(st));
    // The same step eagerly, on the twin cache.
    launch_step(kv_eager, out_eager);
    HIP_OK(hipStreamSynchronize(st));

    std::vector<uint16_t> out_g((size_t)kSessions * kHq * kD), out_e(out_g.size());
    std::vector<uint16_t> kv_g(kv_h.size()), kv_e(kv_h.size());
    HIP_OK(hipMemcpy(out_g.data(), out, out_g.size() * 2, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(out_e.data(), out_eager, out_e.size() * 2, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(kv_g.data(), kv, kv_bytes, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(kv_e.data(), kv_eager, kv_bytes, hipMemcpyDeviceToHost));
    if (out_g != out_e) fail("graph replay output differs from the eager step", step);
    if (kv_g != kv_e) fail("graph replay cache differs from the eager step", step);

    // The oracle chain on the host copies.
    std::vector<uint16_t> q_o = qkv_h, kv_o = kv_before, out_o(out_g.size());
    oracle_qwen3_rope(q_o.data(), qn_h.data(), kn_h.data(), pos_h, slot_h, kv_o.data(), kSessions, kHq, kHk, eps, theta);
    if (oracle_paged_attend(q_o.data(), kv_o.data(), pos_h, nullptr, 0, indptr_h, pages_h, kPage, out_o.data(),
                            kSessions, kHq, kHk, scale, 0, 4) != 0)
      fail("oracle", step);
    double mx = 0, sum = 0;
    for (size_t i = 0; i < out_o.size(); ++i) {
      const double g = from_bf16(out_g[i]), w = from_bf16(out_o[i]);
      if (!std::isfinite(g)) fail("non-finite output", step);
      mx = std::fmax(mx, std::fabs(g - w));
      sum += std::fabs(g - w);
    }
    const double mean = sum / (double)out_o.size();
    if (mx > 2e-2 || mean > 2e-3) {
      fprintf(stderr, "engine_step: step %d: max-abs %.3g mean-abs %.3g\n", step, mx, mean);
      fail("output outside the tolerance against the oracle", step);
    }
    worst_max = std::fmax(worst_max, mx);
    worst_mean = std::fmax(worst_mean, mean);
    // V of every written slot is copied, not computed: bytes must match.
    for (int n = 0; n < kSessions; ++n) {
      const size_t v0 = (size_t)slot_h[n] * kSlot + kHk * kD;
      if (std::memcmp(&kv_g[v0], &kv_o[v0], kHk * kD * 2) != 0) fail("V bytes of a written slot", step);
    }
    for (int s = 0; s < kSessions; ++s) ++len[s];  // every session grew by one token
  }
  printf("engine_step: ok (%d steps of %d sessions, one graph replayed; worst max-abs %.3g mean-abs %.3g)\n", kSteps,
         kSessions, worst_max, worst_mean);
  omni_attn_rows_free(rows);
  HIP_OK(hipGraphExecDestroy(exec));
  HIP_OK(hipGraphDestroy(graph));
  HIP_OK(hipStreamDestroy(st));
  return 0;
}
