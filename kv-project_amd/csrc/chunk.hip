// Chunk-local selection and row gathers of the eviction families (gfx950).
//
//   kvq_gather_rows        exact rows of a (b, h) slice at given positions (SnapKV / StreamingLLM
//                          keep sets, MTLP's kept rows before their KIVI coding)
//   kvq_chunk_share        finalize_chunk's within-chunk attention share (STRATA_KV.py:581-583):
//                          share[c] = mean over the observed queries of softmax_c(q . k_c)
//   kvq_absmax_fake_quant  fake_quant_tokens / absmax_quant (STRATA_KV.py:549-563): what a reader of
//                          a kept token stored at `bits` sees, codes * fp16 scale
//
// All three are byte or elementwise work far below the decode's traffic; they run once per
// compression (prefill or chunk finalisation), so the kernels favour a fixed arithmetic order
// (results reproducible bit for bit) over the last microsecond.
#include "common.hpp"

namespace kvq {
namespace {

// ---- gather: 16-byte units, one thread each; an index outside [0, n_valid) writes a zero row ----
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint4* __restrict__ k, const uint4* __restrict__ v,
                                                          int64_t x_bh, int64_t n_valid, int row_u4,
                                                          const int32_t* __restrict__ idx, int64_t count,
                                                          int64_t idx_bh, uint4* __restrict__ k_out,
                                                          uint4* __restrict__ v_out, int64_t out_bh,
                                                          int64_t total) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (u >= total) return;
  const int64_t row = u / row_u4;                  // flat (bh, i)
  const int w = static_cast<int>(u % row_u4);
  const int64_t bh = row / count, i = row % count;
  const int64_t t = idx[bh * idx_bh + i];
  const bool ok = t >= 0 && t < n_valid;
  const int64_t src = bh * x_bh + (ok ? t : 0) * row_u4 + w;
  const int64_t dst = bh * out_bh + i * row_u4 + w;
  const uint4 zero = make_uint4(0u, 0u, 0u, 0u);
  k_out[dst] = ok ? k[src] : zero;
  if (v != nullptr) v_out[dst] = ok ? v[src] : zero;
}

// ---- chunk share ----------------------------------------------------------------------------
// logits[bh][q][c] = sum_e qref[bh][q][e] * k[bh][c][e] in increasing e (fp32 fma chain), one thread
// per (q, c); 64 keys x 4 queries per block.
__global__ __launch_bounds__(256) void chunk_logits_kernel(const float* __restrict__ qref, const float* __restrict__ k,
                                                           int nq, int C, int d, float* __restrict__ logits) {
  const int bh = blockIdx.x;
  const int c = blockIdx.y * 64 + threadIdx.x % 64;
  const int q = blockIdx.z * 4 + threadIdx.x / 64;
  if (c >= C || q >= nq) return;
  const float4* qr = reinterpret_cast<const float4*>(qref + (static_cast<int64_t>(bh) * nq + q) * d);
  const float4* kr = reinterpret_cast<const float4*>(k + (static_cast<int64_t>(bh) * C + c) * d);
  float s = 0.0f;
  for (int e = 0; e < d / 4; ++e) {
    const float4 a = qr[e], b = kr[e];
    s = __builtin_fmaf(a.x, b.x, s);
    s = __builtin_fmaf(a.y, b.y, s);
    s = __builtin_fmaf(a.z, b.z, s);
    s = __builtin_fmaf(a.w, b.w, s);
  }
  logits[(static_cast<int64_t>(bh) * nq + q) * C + c] = s;
}

// One block per bh.  Wave w takes query rows w, w + 4, ...: the row's max and sum of exp over the C
// keys (lanes own keys l, l + 64, ...; a fixed butterfly order), then p = exp(l - max) / sum into
// the wave's own LDS share row.  The four rows are summed in wave order and divided by nq.
constexpr int kShareMaxC = 2048;

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

__global__ __launch_bounds__(256) void chunk_share_kernel(const float* __restrict__ logits, int nq, int C,
                                                          float* __restrict__ share) {
  __shared__ float acc[4][kShareMaxC];
  const int bh = blockIdx.x;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  for (int c = lane; c < C; c += 64) acc[wave][c] = 0.0f;
  for (int q = wave; q < nq; q += 4) {
    const float* row = logits + (static_cast<int64_t>(bh) * nq + q) * C;
    float m = -INFINITY;
    for (int c = lane; c < C; c += 64) m = fmaxf(m, row[c]);
    m = wave_max(m);
    float s = 0.0f;
    for (int c = lane; c < C; c += 64) s += expf(row[c] - m);
    s = wave_sum(s);
    for (int c = lane; c < C; c += 64) acc[wave][c] += expf(row[c] - m) / s;
  }
  __syncthreads();
  for (int c = threadIdx.x; c < C; c += 256)
    share[static_cast<int64_t>(bh) * C + c] = (((acc[0][c] + acc[1][c]) + acc[2][c]) + acc[3][c]) / static_cast<float>(nq);
}

// ---- absmax fake quantisation: one wave per row of d elements --------------------------------
__global__ __launch_bounds__(256) void absmax_fake_quant_kernel(const float* __restrict__ x, int64_t rows, int d,
                                                                int bits, float* __restrict__ out) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  if (r >= rows) return;
  const float* xr = x + r * d;
  float a = 0.0f;
  for (int e = lane; e < d; e += 64) a = fmaxf(a, fabsf(xr[e]));
  a = wave_max(a);
  const float qmax = static_cast<float>((1 << (bits - 1)) - 1);
  // s = as_stored(amax / qmax): saturate to the fp16 range, round to fp16; then clamp_min(2^-24)
  const float ratio = fminf(fmaxf(a / qmax, -65504.0f), 65504.0f);
  const float s = fmaxf(f16_to_f32(f32_to_f16(ratio)), 0x1p-24f);
  for (int e = lane; e < d; e += 64) {
    const float c = fminf(fmaxf(rintf(xr[e] / s), -qmax), qmax);
    out[r * d + e] = c * s;
  }
}

}  // namespace
}  // namespace kvq

using namespace kvq;

extern "C" int kvq_gather_rows(const void* k, const void* v, int64_t BH, int64_t n_valid, int64_t x_bh,
                               int64_t row_bytes, const int32_t* idx, int64_t count, int64_t idx_bh, void* k_out,
                               void* v_out, int64_t out_bh, void* stream) {
  KVQ_REQUIRE(row_bytes > 0 && row_bytes % 16 == 0, "kvq_gather_rows: row_bytes must be a positive multiple of 16");
  KVQ_REQUIRE(BH >= 0 && count >= 0 && n_valid >= 0 && idx_bh >= count, "kvq_gather_rows: bad sizes");
  KVQ_REQUIRE(x_bh % 16 == 0 && out_bh % 16 == 0 && x_bh >= n_valid * row_bytes && out_bh >= count * row_bytes,
              "kvq_gather_rows: (b, h) strides must be multiples of 16 bytes covering the rows");
  const int64_t total = BH * count * (row_bytes / 16);
  if (total == 0) return KVQ_OK;
  KVQ_REQUIRE(k && idx && k_out && (v == nullptr) == (v_out == nullptr), "kvq_gather_rows: null pointer");
  KVQ_REQUIRE(reinterpret_cast<uintptr_t>(k) % 16 == 0 && reinterpret_cast<uintptr_t>(k_out) % 16 == 0 &&
              reinterpret_cast<uintptr_t>(v) % 16 == 0 && reinterpret_cast<uintptr_t>(v_out) % 16 == 0,
              "kvq_gather_rows: rows must be 16-byte aligned");
  const int64_t blocks = (total + 255) / 256;
  KVQ_REQUIRE(blocks < (1LL << 31) && row_bytes / 16 < (1 << 30), "kvq_gather_rows: too large");
  hipLaunchKernelGGL(gather_rows_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint4*>(k), static_cast<const uint4*>(v),
                     x_bh / 16, n_valid, static_cast<int>(row_bytes / 16), idx, count, idx_bh,
                     static_cast<uint4*>(k_out), static_cast<uint4*>(v_out), out_bh / 16, total);
  KVQ_LAUNCH_CHECK("kvq_gather_rows");
  return KVQ_OK;
}

extern "C" int64_t kvq_chunk_share_workspace(int64_t BH, int64_t nq, int64_t C) {
  if (BH <= 0 || nq <= 0 || C <= 0) return -1;
  return BH * nq * C;
}

extern "C" int kvq_chunk_share(const float* qref, const float* k, int64_t BH, int64_t nq, int64_t C, int64_t d,
                               float* share, float* workspace, int64_t workspace_floats, void* stream) {
  KVQ_REQUIRE(BH > 0 && nq > 0 && C > 0 && d > 0, "kvq_chunk_share: bad sizes");
  KVQ_REQUIRE(C <= kShareMaxC, "kvq_chunk_share: at most %d keys per chunk", kShareMaxC);
  KVQ_REQUIRE(d % 4 == 0 && nq < 65536 * 4 && BH < (1LL << 31), "kvq_chunk_share: d must be a multiple of 4");
  KVQ_REQUIRE(qref && k && share && workspace, "kvq_chunk_share: null pointer");
  KVQ_REQUIRE(workspace_floats >= BH * nq * C, "kvq_chunk_share: workspace too small (%lld < %lld floats)",
              (long long)workspace_floats, (long long)(BH * nq * C));
  KVQ_REQUIRE(reinterpret_cast<uintptr_t>(qref) % 16 == 0 && reinterpret_cast<uintptr_t>(k) % 16 == 0,
              "kvq_chunk_share: qref and k must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(chunk_logits_kernel, dim3(static_cast<unsigned>(BH), static_cast<unsigned>((C + 63) / 64),
                                               static_cast<unsigned>((nq + 3) / 4)),
                     dim3(256), 0, s, qref, k, static_cast<int>(nq), static_cast<int>(C), static_cast<int>(d),
                     workspace);
  KVQ_LAUNCH_CHECK("kvq_chunk_share(logits)");
  hipLaunchKernelGGL(chunk_share_kernel, dim3(static_cast<unsigned>(BH)), dim3(256), 0, s, workspace,
                     static_cast<int>(nq), static_cast<int>(C), share);
  KVQ_LAUNCH_CHECK("kvq_chunk_share");
  return KVQ_OK;
}

extern "C" int kvq_absmax_fake_quant(const float* x, int64_t rows, int64_t d, int bits, float* out, void* stream) {
  KVQ_REQUIRE(bits >= 2 && bits <= 15, "kvq_absmax_fake_quant: bits must be in 2..15 (16 and more keep the rows)");
  KVQ_REQUIRE(rows >= 0 && d > 0 && d < (1 << 24), "kvq_absmax_fake_quant: bad sizes");
  if (rows == 0) return KVQ_OK;
  KVQ_REQUIRE(x && out, "kvq_absmax_fake_quant: null pointer");
  const int64_t blocks = (rows + 3) / 4;
  KVQ_REQUIRE(blocks < (1LL << 31), "kvq_absmax_fake_quant: too many rows");
  hipLaunchKernelGGL(absmax_fake_quant_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, rows, static_cast<int>(d), bits, out);
  KVQ_LAUNCH_CHECK("kvq_absmax_fake_quant");
  return KVQ_OK;
}
