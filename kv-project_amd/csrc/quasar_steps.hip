// QUASAR coded-domain products over a side's step table (gfx950): the reference's kernel-wrapper
// call shapes quasar_scores / quasar_values (QUASAR_KV.py:1556-1577), for callers that hold the
// query coefficients or the weighted probabilities themselves.  The fused decode (quasar.hip)
// computes the same sums inside one launch and never writes them out.
//
// A side is the reference's stored code as QuasarState.__init__ lays it out (1883-1898): one flat
// uint8 buffer holding every step's (Hkv, n_s, nb) block of pack_rows rows (first code of a byte in
// its most significant bits), a step table of int32 rows [offset, n_s, nb, a, w, bits, level
// offset] (in step order; a step owns the token prefix [0, n_s) and the coefficient band [a, a + w)),
// and the stage codebooks concatenated (float32).
//
//   scores[h][r][j] = sum over the steps s with j < n_s of sum_i qt[h][r][a_s + i] * level_s(code)
//   values[h][r][c] = sum over the steps s with a_s <= c < a_s + w_s of sum_{j < n_s} pv[h][r][j]
//                                                                          * level_s(code(j, c - a_s))
// Both run in a fixed order (steps in table order, then band positions / tokens in increasing
// order): results are reproducible bit for bit.  The step table comes from host memory: it is
// checked against the code buffer, the levels and the band width before any launch and handed to
// the kernels by value, so no table entry can send a read outside the buffers.
#include <algorithm>

#include "common.hpp"

namespace kvq {
namespace {

constexpr int kMaxSteps = 64;
constexpr int kTokChunk = 1024;         // tokens of one values partial

struct StepTable {
  int n;
  int t[kMaxSteps * 7];
};

__device__ __forceinline__ int step_code(const uint8_t* flat, const int* st, int h, int j, int i) {
  const int nb = st[2], b = st[5];
  const int per = 8 / b;
  const uint32_t byte = flat[static_cast<int64_t>(st[0]) + (static_cast<int64_t>(h) * st[1] + j) * nb + i / per];
  return static_cast<int>((byte >> ((per - 1 - i % per) * b)) & ((1u << b) - 1u));
}

// one thread per (h, token j, row r): the token's score row, step by step
__global__ __launch_bounds__(256) void quasar_scores_kernel(const float* __restrict__ qt, int rows, int R,
                                                            const uint8_t* __restrict__ flat, StepTable tb,
                                                            const float* __restrict__ levels, int n_c,
                                                            float* __restrict__ out) {
  const int n_steps = tb.n;
  const int* tab = tb.t;
  const int h = blockIdx.x;
  const int j = blockIdx.y * 64 + threadIdx.x % 64;
  const int r = blockIdx.z * 4 + threadIdx.x / 64;
  if (j >= n_c || r >= rows) return;
  const float* q = qt + (static_cast<int64_t>(h) * rows + r) * R;
  float acc = 0.0f;
  for (int s = 0; s < n_steps; ++s) {
    const int* st = tab + 7 * s;
    if (j >= st[1]) continue;
    const int a = st[3], w = st[4], lo = st[6];
    float part = 0.0f;
    for (int i = 0; i < w; ++i) part = __builtin_fmaf(q[a + i], levels[lo + step_code(flat, st, h, j, i)], part);
    acc += part;
  }
  out[(static_cast<int64_t>(h) * rows + r) * n_c + j] = acc;
}

// one block per (h, row r, token chunk): thread c sums its coefficient over the chunk's tokens of
// every step covering it; partials (h, r, chunk, R) are summed in chunk order by the next kernel
__global__ __launch_bounds__(256) void quasar_values_partial_kernel(const float* __restrict__ pv, int rows, int n_c,
                                                                    const uint8_t* __restrict__ flat, StepTable tb,
                                                                    const float* __restrict__ levels, int R,
                                                                    int n_chunks, float* __restrict__ part) {
  const int n_steps = tb.n;
  const int* tab = tb.t;
  const int h = blockIdx.x, r = blockIdx.y, ch = blockIdx.z;
  const int j0 = ch * kTokChunk;
  const float* p = pv + (static_cast<int64_t>(h) * rows + r) * n_c;
  for (int c = threadIdx.x; c < R; c += 256) {
    float acc = 0.0f;
    for (int s = 0; s < n_steps; ++s) {
      const int* st = tab + 7 * s;
      const int a = st[3], w = st[4], lo = st[6];
      if (c < a || c >= a + w) continue;
      const int j1 = min(j0 + kTokChunk, st[1]);
      float sum = 0.0f;
      for (int j = j0; j < j1; ++j) sum = __builtin_fmaf(p[j], levels[lo + step_code(flat, st, h, j, c - a)], sum);
      acc += sum;
    }
    part[((static_cast<int64_t>(h) * rows + r) * n_chunks + ch) * R + c] = acc;
  }
}

__global__ __launch_bounds__(256) void quasar_values_sum_kernel(const float* __restrict__ part, int64_t hr, int R,
                                                                int n_chunks, float* __restrict__ out) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (u >= hr * R) return;
  const int64_t hr_i = u / R;
  const int c = static_cast<int>(u % R);
  float acc = 0.0f;
  for (int ch = 0; ch < n_chunks; ++ch) acc += part[(hr_i * n_chunks + ch) * R + c];
  out[u] = acc;
}

}  // namespace
}  // namespace kvq

using namespace kvq;

namespace {
// the host table checked against what the kernels read: codes inside the buffer, levels inside
// the codebooks, bands inside R, token prefixes inside n_c, widths that fill whole bytes
int load_table(const int32_t* table, int n_steps, int64_t flat_bytes, int64_t n_levels, int64_t Hkv, int64_t R,
               int64_t n_c, StepTable* tb) {
  KVQ_REQUIRE(n_steps >= 0 && n_steps <= kMaxSteps, "quasar steps: at most %d steps per side", kMaxSteps);
  KVQ_REQUIRE(n_steps == 0 || table, "quasar steps: null step table");
  tb->n = n_steps;
  for (int s = 0; s < n_steps; ++s) {
    const int32_t* r = table + 7 * s;
    const int64_t off = r[0], ns = r[1], nb = r[2], a = r[3], w = r[4], b = r[5], lo = r[6];
    KVQ_REQUIRE(b == 1 || b == 2 || b == 4 || b == 8, "quasar steps: step %d has %lld bits", s, (long long)b);
    KVQ_REQUIRE(w > 0 && nb * 8 == w * b, "quasar steps: step %d's rows do not hold its band", s);
    KVQ_REQUIRE(a >= 0 && a + w <= R, "quasar steps: step %d's band [%lld, %lld) leaves R = %lld", s, (long long)a,
                (long long)(a + w), (long long)R);
    KVQ_REQUIRE(ns >= 0 && ns <= n_c, "quasar steps: step %d owns %lld > n_c tokens", s, (long long)ns);
    KVQ_REQUIRE(off >= 0 && off + Hkv * ns * nb <= flat_bytes, "quasar steps: step %d's codes leave the buffer", s);
    KVQ_REQUIRE(lo >= 0 && lo + (1LL << b) <= n_levels, "quasar steps: step %d's levels leave the codebooks", s);
    for (int k = 0; k < 7; ++k) tb->t[7 * s + k] = r[k];
  }
  return KVQ_OK;
}
}  // namespace

extern "C" int kvq_quasar_scores(const float* qt, int64_t Hkv, int64_t rows, int64_t R, const uint8_t* flat,
                                 int64_t flat_bytes, const int32_t* table, int n_steps, const float* levels,
                                 int64_t n_levels, int64_t n_c, float* out, void* stream) {
  KVQ_REQUIRE(Hkv > 0 && Hkv < 65536 && rows > 0 && rows < 65536 * 4 && R > 0 && n_c >= 0 && n_c <= 65535LL * 64,
              "kvq_quasar_scores: bad sizes");
  StepTable tb;
  const int rc = load_table(table, n_steps, flat_bytes, n_levels, Hkv, R, n_c, &tb);
  if (rc != KVQ_OK) return rc;
  if (n_c == 0) return KVQ_OK;
  KVQ_REQUIRE(qt && out && (n_steps == 0 || (flat && levels)), "kvq_quasar_scores: null pointer");
  const dim3 grid(static_cast<unsigned>(Hkv), static_cast<unsigned>((n_c + 63) / 64), static_cast<unsigned>((rows + 3) / 4));
  hipLaunchKernelGGL(quasar_scores_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), qt,
                     static_cast<int>(rows), static_cast<int>(R), flat, tb, levels, static_cast<int>(n_c), out);
  KVQ_LAUNCH_CHECK("kvq_quasar_scores");
  return KVQ_OK;
}

extern "C" int64_t kvq_quasar_values_workspace(int64_t Hkv, int64_t rows, int64_t R, int64_t n_c) {
  if (Hkv <= 0 || rows <= 0 || R <= 0 || n_c < 0) return -1;
  return Hkv * rows * std::max<int64_t>(1, (n_c + kTokChunk - 1) / kTokChunk) * R;
}

extern "C" int kvq_quasar_values(const float* pv, int64_t Hkv, int64_t rows, int64_t n_c, const uint8_t* flat,
                                 int64_t flat_bytes, const int32_t* table, int n_steps, const float* levels,
                                 int64_t n_levels, int64_t R, float* out, float* workspace, int64_t workspace_floats,
                                 void* stream) {
  KVQ_REQUIRE(Hkv > 0 && Hkv < 65536 && rows > 0 && rows < 65536 && R > 0 && R <= 4096 && n_c >= 0 &&
              n_c < (1LL << 31), "kvq_quasar_values: bad sizes");
  StepTable tb;
  const int rc = load_table(table, n_steps, flat_bytes, n_levels, Hkv, R, n_c, &tb);
  if (rc != KVQ_OK) return rc;
  KVQ_REQUIRE(pv && out && workspace && (n_steps == 0 || (flat && levels)), "kvq_quasar_values: null pointer");
  const int64_t n_chunks = std::max<int64_t>(1, (n_c + kTokChunk - 1) / kTokChunk);
  KVQ_REQUIRE(n_chunks < 65536 && workspace_floats >= Hkv * rows * n_chunks * R,
              "kvq_quasar_values: workspace too small (%lld < %lld floats)", (long long)workspace_floats,
              (long long)(Hkv * rows * n_chunks * R));
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(quasar_values_partial_kernel, dim3(static_cast<unsigned>(Hkv), static_cast<unsigned>(rows),
                                                        static_cast<unsigned>(n_chunks)),
                     dim3(256), 0, s, pv, static_cast<int>(rows), static_cast<int>(n_c), flat, tb, levels,
                     static_cast<int>(R), static_cast<int>(n_chunks), workspace);
  KVQ_LAUNCH_CHECK("kvq_quasar_values(partials)");
  const int64_t total = Hkv * rows * R;
  hipLaunchKernelGGL(quasar_values_sum_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, s,
                     workspace, Hkv * rows, static_cast<int>(R), static_cast<int>(n_chunks), out);
  KVQ_LAUNCH_CHECK("kvq_quasar_values");
  return KVQ_OK;
}
