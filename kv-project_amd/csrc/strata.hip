// STRATA codec (A5), planar packing (A3) and the value-tile repack the STRATA tier decode reads.
//
// Reference (STRATA_KV.py): rotation_matrix 1110-1128 (R = H_d diag(s) / sqrt(d), Sylvester H),
// strata_quantize 1158-1168, pack_planar / unpack_planar 1171-1189, the centring and rotation of
// one side of a layer 1546-1548 (mu = fp16(mean over coded tokens), Y = (X - mu) R^T).
//
// Fixed arithmetic order (the CPU oracle restates exactly this, so codes and scales agree bit
// for bit):
//   mu:   per channel, float64 sum over the n tokens, / n, rounded to float32, then to fp16;
//   Y:    (x - mu) * s in float32, fast Walsh-Hadamard transform with butterfly stages
//         h = 1, 2, ..., d/2 (pairs (a, b) -> (a + b, a - b)), then * float32(1 / sqrt(d));
//   s:    rms = sqrt(float32(float64 sum of y^2 / d)); s = max(fp16(float32(step) * rms), 2^-24);
//   code: clamp(rint(y / s + (2^b - 1) / 2), 0, 2^b - 1) with IEEE float32 division and add.
#include "common.hpp"
#include "mfma_common.hpp"

namespace kvq {
namespace {

constexpr int kSD = 128;                          // head_dim of the STRATA kernels
constexpr float kMinScale = 5.9604644775390625e-08f;

__device__ __forceinline__ float as_stored16(float x) {
  x = fminf(fmaxf(x, -65504.0f), 65504.0f);
  return f16_to_f32(f32_to_f16(x));
}

// code of coordinate c of a planar row of `bits`-bit codes (d = kSD)
__device__ __forceinline__ int planar_code(const uint8_t* row, int c, int bits) {
  const int per = kSD * bits / 8;                 // bytes per row = coordinates per plane
  return (row[c % per] >> ((c / per) * bits)) & ((1 << bits) - 1);
}

__global__ void pack_planar_kernel(const uint8_t* __restrict__ codes, int64_t rows, int d, int bits,
                                   uint8_t* __restrict__ out) {
  const int64_t per = d * bits / 8;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * per) return;
  const int64_t r = i / per, b = i % per;
  const int P = 8 / bits;
  int v = 0;
  for (int p = 0; p < P; ++p) v |= static_cast<int>(codes[r * d + p * per + b]) << (p * bits);
  out[i] = static_cast<uint8_t>(v);
}

__global__ void unpack_planar_kernel(const uint8_t* __restrict__ packed, int64_t rows, int d, int bits,
                                     uint8_t* __restrict__ codes) {
  const int64_t per = d * bits / 8;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * d) return;
  const int64_t r = i / d;
  const int c = static_cast<int>(i % d);
  codes[i] = static_cast<uint8_t>((packed[r * per + c % per] >> ((c / per) * bits)) & ((1 << bits) - 1));
}

// mu[bh][c] = fp16(float32(sum_t x[bh][t][c] / n)): one block of 1024 threads per (b, h), 8 token
// strides per channel summed in float64, combined in a fixed order.
template <int DT>
__global__ __launch_bounds__(1024) void strata_mean_kernel(const void* __restrict__ x, int64_t n, int64_t x_bh,
                                                           uint16_t* __restrict__ mu) {
  __shared__ double part[8][kSD];
  const int c = threadIdx.x % kSD, j = threadIdx.x / kSD;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * x_bh;
  double acc = 0.0;
  for (int64_t t = j; t < n; t += 8) acc += static_cast<double>(load_as_f32<DT>(x, base + t * kSD + c));
  part[j][c] = acc;
  __syncthreads();
  if (j == 0) {
    double s = 0.0;
    for (int k = 0; k < 8; ++k) s += part[k][c];
    mu[static_cast<int64_t>(blockIdx.x) * kSD + c] = f32_to_f16(as_stored16(static_cast<float>(s / static_cast<double>(n))));
  }
}

// In-wave FWHT of a 128-vector held as (v0 = x[lane], v1 = x[lane + 64]), stages h = 1 .. 64.
__device__ __forceinline__ void fwht128(float& v0, float& v1, int lane) {
#pragma unroll
  for (int h = 1; h < 64; h <<= 1) {
    const float p0 = __shfl_xor(v0, h, 64), p1 = __shfl_xor(v1, h, 64);
    const bool upper = (lane & h) != 0;
    v0 = upper ? __fsub_rn(p0, v0) : __fadd_rn(v0, p0);
    v1 = upper ? __fsub_rn(p1, v1) : __fadd_rn(v1, p1);
  }
  const float a = v0, b = v1;
  v0 = __fadd_rn(a, b);
  v1 = __fsub_rn(a, b);
}

// Y[bh][t] = (x[bh][t] - mu[bh]) R^T: one wavefront per token.
template <int DT>
__global__ __launch_bounds__(256) void strata_rotate_kernel(const void* __restrict__ x, int64_t n, int64_t x_bh,
                                                            const uint16_t* __restrict__ mu,
                                                            const float* __restrict__ signs, float* __restrict__ y,
                                                            int64_t total) {
  const int lane = threadIdx.x % 64;
  const int64_t tok = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / 64;
  if (tok >= total) return;
  const int64_t bh = tok / n, t = tok % n;
  const int64_t xo = bh * x_bh + t * kSD;
  const float m0 = f16_to_f32(mu[bh * kSD + lane]), m1 = f16_to_f32(mu[bh * kSD + lane + 64]);
  float v0 = __fmul_rn(__fsub_rn(load_as_f32<DT>(x, xo + lane), m0), signs[lane]);
  float v1 = __fmul_rn(__fsub_rn(load_as_f32<DT>(x, xo + lane + 64), m1), signs[lane + 64]);
  fwht128(v0, v1, lane);
  const float inv = 0.08838834764831845f;         // float32(1 / sqrt(128))
  y[tok * kSD + lane] = __fmul_rn(v0, inv);
  y[tok * kSD + lane + 64] = __fmul_rn(v1, inv);
}

// Codes and scale of rotated vectors: one wavefront per output token i of (b, h); source token
// idx[bh][i] (or i when idx is null).  Writes planar rows and fp16 scales.
__global__ __launch_bounds__(256) void strata_quantize_kernel(const float* __restrict__ y, int64_t n,
                                                              const int32_t* __restrict__ idx, int64_t m,
                                                              int bits, float step, uint8_t* __restrict__ codes,
                                                              uint16_t* __restrict__ scales, int64_t total) {
  const int lane = threadIdx.x % 64;
  const int64_t oi = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / 64;
  if (oi >= total) return;
  const int64_t bh = oi / m, i = oi % m;
  const int64_t t = idx ? static_cast<int64_t>(idx[bh * m + i]) : i;
  if (t < 0 || t >= n) return;                    // rejected on the host for idx == null
  const float* row = y + (bh * n + t) * kSD;
  const float y0 = row[lane], y1 = row[lane + 64];
  double ss = static_cast<double>(y0) * y0 + static_cast<double>(y1) * y1;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
  const float rms = __fsqrt_rn(static_cast<float>(ss / kSD));
  const float s = fmaxf(as_stored16(__fmul_rn(step, rms)), kMinScale);
  const float half = static_cast<float>((1 << bits) - 1) * 0.5f;
  const float qmax = static_cast<float>((1 << bits) - 1);
  const int c0 = static_cast<int>(fminf(fmaxf(rintf(__fadd_rn(__fdiv_rn(y0, s), half)), 0.0f), qmax));
  const int c1 = static_cast<int>(fminf(fmaxf(rintf(__fadd_rn(__fdiv_rn(y1, s), half)), 0.0f), qmax));
  uint8_t* out = codes + oi * (kSD * bits / 8);
  if (bits == 8) {
    out[lane] = static_cast<uint8_t>(c0);
    out[lane + 64] = static_cast<uint8_t>(c1);
  } else if (bits == 4) {
    out[lane] = static_cast<uint8_t>(c0 | (c1 << 4));            // coordinates lane, lane + 64
  } else {
    const int u0 = __shfl_down(c0, 32, 64), u1 = __shfl_down(c1, 32, 64);   // coordinates +32, +96
    if (lane < 32) out[lane] = static_cast<uint8_t>(c0 | (u0 << 2) | (c1 << 4) | (u1 << 6));
  }
  if (lane == 0) scales[oi] = f32_to_f16(s);
}

// token of slot j of lane group g within a 32-token chunk (the order the decode's logits arrive in)
__device__ __forceinline__ int slot_token(int g, int j) { return 16 * (j >> 2) + 4 * g + (j & 3); }

__device__ __constant__ int kSlotOfNibble4[8] = {0, 2, 4, 6, 1, 3, 5, 7};
__device__ __constant__ int kSlotOfByte8[8] = {0, 2, 1, 3, 4, 6, 5, 7};

// Value tiles of one width from planar rows: one thread per 32-bit tile word.
//   4 bits: word (blk/4)*256 + l*4 + blk%4 of a 2 KiB chunk; nibble k holds slot kSlotOfNibble4[k]
//   8 bits: word (blk/2)*256 + l*4 + (blk%2)*2 + w of a 4 KiB chunk; byte k of the lane's 8 holds
//           slot kSlotOfByte8[k]
//   2 bits: word l*4 + blk/2 of a 1 KiB chunk; bits 2k: slot 2(k&3) + (k>>3) of blk 2(blk/2)+((k>>2)&1)
// with lane l = 16g + n, channel 16*blk + n, token slot_token(g, slot).  Tokens >= n read code 0.
__global__ void strata_vtile_kernel(const uint8_t* __restrict__ rows, int64_t n, int64_t rows_bh, int bits,
                                    int64_t cap_t, uint32_t* __restrict__ tiles, int64_t total_words) {
  const int64_t wi = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (wi >= total_words) return;
  const int words_per_chunk = 128 * bits;          // 512 * bits bytes
  const int64_t chunk_all = wi / words_per_chunk;
  const int w = static_cast<int>(wi % words_per_chunk);
  const int64_t nchunk = cap_t / 32;
  const int64_t bh = chunk_all / nchunk, chunk = chunk_all % nchunk;
  const int row_bytes = kSD * bits / 8;
  const uint8_t* base = rows + bh * rows_bh;
  uint32_t word = 0;
  auto code_at = [&](int slot, int g, int channel) -> uint32_t {
    const int64_t t = chunk * 32 + slot_token(g, slot);
    return t < n ? static_cast<uint32_t>(planar_code(base + t * row_bytes, channel, bits)) : 0u;
  };
  if (bits == 4) {
    const int blk = (w / 256) * 4 + (w % 4), l = (w % 256) / 4;
    const int g = l / 16, ch = 16 * blk + (l % 16);
    for (int k = 0; k < 8; ++k) word |= code_at(kSlotOfNibble4[k], g, ch) << (4 * k);
  } else if (bits == 8) {
    const int blk = (w / 256) * 2 + ((w % 4) / 2), l = (w % 256) / 4, half = w % 2;
    const int g = l / 16, ch = 16 * blk + (l % 16);
    for (int k = 0; k < 4; ++k) word |= code_at(kSlotOfByte8[4 * half + k], g, ch) << (8 * k);
  } else {
    const int l = w / 4, bp = w % 4;
    const int g = l / 16;
    for (int k = 0; k < 16; ++k) {
      const int blk = 2 * bp + ((k >> 2) & 1), slot = 2 * (k & 3) + (k >> 3);
      word |= code_at(slot, g, 16 * blk + (l % 16)) << (2 * k);
    }
  }
  tiles[wi] = word;
}

// Per-token scales in slot order: vsl[bh][chunk][8g + j] = vs[bh][token slot_token(g, j)].
__global__ void strata_vslot_kernel(const uint16_t* __restrict__ vs, int64_t n, int64_t vs_bh, int64_t cap_t,
                                    uint16_t* __restrict__ vsl, int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t nchunk = cap_t / 32;
  const int s = static_cast<int>(i % 32);
  const int64_t chunk = (i / 32) % nchunk, bh = i / 32 / nchunk;
  const int64_t t = chunk * 32 + slot_token(s / 8, s % 8);
  vsl[i] = t < n ? vs[bh * vs_bh + t] : static_cast<uint16_t>(0);
}

int blocks_for(int64_t items, int per) { return static_cast<int>((items + per - 1) / per); }

}  // namespace
}  // namespace kvq

using namespace kvq;

extern "C" int kvq_pack_planar(const uint8_t* codes, int64_t rows, int64_t d, int bits, uint8_t* out, void* stream) {
  KVQ_REQUIRE(bits == 2 || bits == 4 || bits == 8, "kvq_pack_planar: bits must be 2, 4 or 8");
  KVQ_REQUIRE(rows >= 0 && d > 0 && d % (8 / bits) == 0, "kvq_pack_planar: d must be a multiple of 8/bits");
  const int64_t total = rows * d * bits / 8;
  if (total == 0) return KVQ_OK;
  KVQ_REQUIRE(codes && out && total / 256 < (1LL << 31), "kvq_pack_planar: null pointer or too large");
  hipLaunchKernelGGL(pack_planar_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     codes, rows, static_cast<int>(d), bits, out);
  KVQ_LAUNCH_CHECK("kvq_pack_planar");
  return KVQ_OK;
}

extern "C" int kvq_unpack_planar(const uint8_t* packed, int64_t rows, int64_t d, int bits, uint8_t* codes, void* stream) {
  KVQ_REQUIRE(bits == 2 || bits == 4 || bits == 8, "kvq_unpack_planar: bits must be 2, 4 or 8");
  KVQ_REQUIRE(rows >= 0 && d > 0 && d % (8 / bits) == 0, "kvq_unpack_planar: d must be a multiple of 8/bits");
  const int64_t total = rows * d;
  if (total == 0) return KVQ_OK;
  KVQ_REQUIRE(packed && codes && total / 256 < (1LL << 31), "kvq_unpack_planar: null pointer or too large");
  hipLaunchKernelGGL(unpack_planar_kernel, dim3(blocks_for(total, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), packed, rows, static_cast<int>(d), bits, codes);
  KVQ_LAUNCH_CHECK("kvq_unpack_planar");
  return KVQ_OK;
}

extern "C" int kvq_strata_center_rotate(const void* x, int x_dtype, int64_t BH, int64_t n, int64_t d, int64_t x_bh,
                                        const float* signs, uint16_t* mu, float* y, void* stream) {
  KVQ_REQUIRE(valid_dtype(x_dtype), "kvq_strata_center_rotate: bad dtype");
  KVQ_REQUIRE(d == kSD, "kvq_strata_center_rotate: head_dim must be 128");
  KVQ_REQUIRE(BH >= 0 && n >= 0 && x_bh >= n * d, "kvq_strata_center_rotate: bad sizes");
  if (BH == 0 || n == 0) return KVQ_OK;
  KVQ_REQUIRE(x && signs && mu && y, "kvq_strata_center_rotate: null pointer");
  KVQ_REQUIRE(BH < (1LL << 31) && BH * n / 4 < (1LL << 31), "kvq_strata_center_rotate: too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  KVQ_DISPATCH_DTYPE(x_dtype, hipLaunchKernelGGL((strata_mean_kernel<DT_>), dim3(static_cast<unsigned>(BH)),
                                                dim3(1024), 0, s, x, n, x_bh, mu));
  KVQ_LAUNCH_CHECK("kvq_strata_center_rotate(mean)");
  KVQ_DISPATCH_DTYPE(x_dtype, hipLaunchKernelGGL((strata_rotate_kernel<DT_>), dim3(blocks_for(BH * n, 4)), dim3(256),
                                                0, s, x, n, x_bh, mu, signs, y, BH * n));
  KVQ_LAUNCH_CHECK("kvq_strata_center_rotate(rotate)");
  return KVQ_OK;
}

extern "C" int kvq_strata_quantize(const float* y, int64_t BH, int64_t n, int64_t d, const int32_t* idx, int64_t m,
                                   int bits, float step, uint8_t* codes, uint16_t* scales, void* stream) {
  KVQ_REQUIRE(bits == 2 || bits == 4 || bits == 8, "kvq_strata_quantize: bits must be 2, 4 or 8");
  KVQ_REQUIRE(d == kSD, "kvq_strata_quantize: head_dim must be 128");
  KVQ_REQUIRE(BH >= 0 && n >= 0 && m >= 0 && (idx != nullptr || m <= n), "kvq_strata_quantize: bad sizes");
  KVQ_REQUIRE(step > 0.0f, "kvq_strata_quantize: step must be positive");
  if (BH == 0 || m == 0) return KVQ_OK;
  KVQ_REQUIRE(y && codes && scales, "kvq_strata_quantize: null pointer");
  KVQ_REQUIRE(BH * m / 4 < (1LL << 31), "kvq_strata_quantize: too large");
  hipLaunchKernelGGL(strata_quantize_kernel, dim3(blocks_for(BH * m, 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), y, n, idx, m, bits, step, codes, scales, BH * m);
  KVQ_LAUNCH_CHECK("kvq_strata_quantize");
  return KVQ_OK;
}

extern "C" int kvq_strata_v_tile(const uint8_t* rows, int64_t BH, int64_t n, int64_t rows_bh, int bits,
                                 int64_t cap_t, uint8_t* tiles, const uint16_t* vs, int64_t vs_bh, uint16_t* vsl,
                                 void* stream) {
  KVQ_REQUIRE(bits == 2 || bits == 4 || bits == 8, "kvq_strata_v_tile: bits must be 2, 4 or 8");
  KVQ_REQUIRE(BH >= 0 && n >= 0 && cap_t % 32 == 0 && n <= cap_t && rows_bh >= n * kSD * bits / 8 && vs_bh >= n,
              "kvq_strata_v_tile: bad sizes");
  if (BH == 0 || cap_t == 0) return KVQ_OK;
  KVQ_REQUIRE((n == 0 || (rows && vs)) && tiles && vsl, "kvq_strata_v_tile: null pointer");
  const int64_t words = BH * (cap_t / 32) * 128 * bits;
  KVQ_REQUIRE(words / 256 < (1LL << 31), "kvq_strata_v_tile: too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(strata_vtile_kernel, dim3(blocks_for(words, 256)), dim3(256), 0, s, rows, n, rows_bh, bits,
                     cap_t, reinterpret_cast<uint32_t*>(tiles), words);
  KVQ_LAUNCH_CHECK("kvq_strata_v_tile(codes)");
  const int64_t slots = BH * cap_t;
  hipLaunchKernelGGL(strata_vslot_kernel, dim3(blocks_for(slots, 256)), dim3(256), 0, s, vs, n, vs_bh, cap_t, vsl,
                     slots);
  KVQ_LAUNCH_CHECK("kvq_strata_v_tile(scales)");
  return KVQ_OK;
}
