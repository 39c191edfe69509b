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
//   s:    rms = sqrt(float32(float64 sum of y^2 / d)) (correctly rounded sqrt);
//         s = max(fp16(float32(step) * rms), 2^-24);
//   code: clamp(rint(y / s + (2^b - 1) / 2), 0, 2^b - 1) with IEEE float32 division and add.
#include <algorithm>

#include "common.hpp"
#include "mfma_common.hpp"
#include "widths.hpp"
#include "partials.hpp"

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

// Long contexts: the same sums split over P token chunks (grid (BH, P), 8 strides per chunk in
// float64), the per-chunk partials then combined in chunk order by strata_mean_combine_kernel.
template <int DT>
__global__ __launch_bounds__(1024) void strata_mean_part_kernel(const void* __restrict__ x, int64_t n, int64_t x_bh,
                                                                int64_t chunk, double* __restrict__ part) {
  __shared__ double red[8][kSD];
  const int c = threadIdx.x % kSD, j = threadIdx.x / kSD;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * x_bh;
  const int64_t t0 = static_cast<int64_t>(blockIdx.y) * chunk, t1 = min(n, t0 + chunk);
  double acc = 0.0;
  for (int64_t t = t0 + j; t < t1; t += 8) acc += static_cast<double>(load_as_f32<DT>(x, base + t * kSD + c));
  red[j][c] = acc;
  __syncthreads();
  if (j == 0) {
    double sum = 0.0;
    for (int k = 0; k < 8; ++k) sum += red[k][c];
    part[(static_cast<int64_t>(blockIdx.x) * gridDim.y + blockIdx.y) * kSD + c] = sum;
  }
}

__global__ __launch_bounds__(kSD) void strata_mean_combine_kernel(const double* __restrict__ part, int P, int64_t n,
                                                                  uint16_t* __restrict__ mu) {
  const int c = threadIdx.x;
  double sum = 0.0;
  for (int p = 0; p < P; ++p) sum += part[(static_cast<int64_t>(blockIdx.x) * P + p) * kSD + c];
  mu[static_cast<int64_t>(blockIdx.x) * kSD + c] = f32_to_f16(as_stored16(static_cast<float>(sum / static_cast<double>(n))));
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
  const float rms = sqrt_rn(static_cast<float>(ss / kSD));
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
  auto code_at = [&](int slot, int g, int channel) -> uint32_t {
    const int64_t t = chunk * 32 + slot_token(g, slot);
    return t < n ? static_cast<uint32_t>(planar_code(base + t * row_bytes, channel, bits)) : 0u;
  };
  tiles[wi] = vtile_word(bits, w, code_at);
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

// ---- distortion table of the compression side (STRATA_KV.py:1543-1559) ----
// Metric in the code basis, written transposed: out[h] = (R (R S[h]^T)^T ... ) computed as
// rot(rows of (rot(rows of S))^T) = R S^T R^T, whose quadratic form equals that of R S R^T.
// One block per matrix; both passes through LDS.
__global__ __launch_bounds__(256) void strata_metric_kernel(const float* __restrict__ S, const float* __restrict__ signs,
                                                            float* __restrict__ out) {
  __shared__ float a[kSD][kSD + 1];
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const float* src = S + static_cast<int64_t>(blockIdx.x) * kSD * kSD;
  const float inv = 0.08838834764831845f;         // float32(1 / sqrt(128))
  for (int pass = 0; pass < 2; ++pass) {
    float r0[kSD / 4], r1[kSD / 4];
    for (int i = wave, u = 0; i < kSD; i += 4, ++u) {           // rows of the current matrix, rotated
      float v0 = pass == 0 ? src[i * kSD + lane] : a[i][lane];
      float v1 = pass == 0 ? src[i * kSD + lane + 64] : a[i][lane + 64];
      v0 = __fmul_rn(v0, signs[lane]);
      v1 = __fmul_rn(v1, signs[lane + 64]);
      fwht128(v0, v1, lane);
      r0[u] = __fmul_rn(v0, inv);
      r1[u] = __fmul_rn(v1, inv);
    }
    __syncthreads();
    for (int i = wave, u = 0; i < kSD; i += 4, ++u) {
      if (pass == 0) {                                            // transposed for the second pass
        a[lane][i] = r0[u];
        a[lane + 64][i] = r1[u];
      } else {
        out[static_cast<int64_t>(blockIdx.x) * kSD * kSD + i * kSD + lane] = r0[u];
        out[static_cast<int64_t>(blockIdx.x) * kSD * kSD + i * kSD + lane + 64] = r1[u];
      }
    }
    __syncthreads();
  }
}

// err[bh][t][b] = e^T M e with e = y_hat - y of token t quantised at width bits[b] (the codes of
// strata_quantize_kernel), M = Mt[bh] read as columns (M^T e gives the same form).
constexpr int kSMaxBits = 3;

struct ErrWidths {
  int n;
  int bits[kSMaxBits];
  float step[kSMaxBits];
};

// Computed on the matrix cores: a workgroup per (bh, kSErrTok tokens) stages M
// transposed in LDS as fp16 hi + lo parts of M x 2^(8 - em) (its largest entry brought to [128, 256));
// each wavefront takes tiles of 16 tokens.  Lane (g, n) holds token n's coordinates 32 ks + 8 g ..;
// per width it forms e with the codec's arithmetic (rms from the float64 sum of squares and the
// correctly rounded root, the fp16 scale, IEEE quotient and rint), scales e by a power of two
// (largest entry to [128, 256)), and y = e M comes from the products hi*hi + hi*lo + lo*hi in fp32
// (about 2^-22 relative); e . y is a row sum, e exchanged through the wavefront's LDS into the
// layout of the products' output.
constexpr int kSErrTok = 512;
constexpr int kSMtStride = kSD + 8;              // halves per LDS row of M^T (16-byte aligned rows)

__global__ __launch_bounds__(256) void strata_err_mfma(const float* __restrict__ y, int64_t n,
                                                       const float* __restrict__ Mt, ErrWidths w,
                                                       float* __restrict__ err) {
  __shared__ __align__(16) uint16_t mt[2][kSD * kSMtStride];  // [part][col][k]
  __shared__ __align__(16) float es[4][16][kSD + 4];
  __shared__ float red[4];
  __shared__ int eex[4][16];
  const int wave = threadIdx.x / 64, l = threadIdx.x % 64, g = l >> 4, nl = l & 15;
  const int64_t bh = blockIdx.y;
  // M's largest entry over the workgroup, then its transposed parts
  const float* mg = Mt + bh * kSD * kSD;
  constexpr int kPer = kSD * kSD / 256;
  float mv[kPer];
  float mx = 0.0f;
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    mv[e] = mg[threadIdx.x + 256 * e];
    mx = fmaxf(mx, fabsf(mv[e]));
  }
  mx = wave_max(mx);
  if (l == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int em = 0;
  if (mx > 0.0f) (void)frexpf(mx, &em);
  const float upm = ldexpf(1.0f, 8 - em);
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int idx = threadIdx.x + 256 * e, k = idx / kSD, c = idx % kSD;
    const float x = mv[e] * upm;
    const _Float16 hi = static_cast<_Float16>(x);
    const _Float16 lo = static_cast<_Float16>(x - static_cast<float>(hi));
    mt[0][c * kSMtStride + k] = __builtin_bit_cast(uint16_t, hi);
    mt[1][c * kSMtStride + k] = __builtin_bit_cast(uint16_t, lo);
  }
  __syncthreads();
  const int64_t t_end = min<int64_t>(n, static_cast<int64_t>(blockIdx.x + 1) * kSErrTok);
  for (int64_t t0 = static_cast<int64_t>(blockIdx.x) * kSErrTok + 16 * wave; t0 < t_end; t0 += 64) {
    const int64_t t = t0 + nl;                                  // this lane's token
    float yv[32];
    const bool ok = t < t_end;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const float* row = y + (bh * n + (ok ? t : t0)) * kSD + 32 * ks + 8 * g;
      const float4 a = *reinterpret_cast<const float4*>(row), b = *reinterpret_cast<const float4*>(row + 4);
      yv[8 * ks + 0] = a.x; yv[8 * ks + 1] = a.y; yv[8 * ks + 2] = a.z; yv[8 * ks + 3] = a.w;
      yv[8 * ks + 4] = b.x; yv[8 * ks + 5] = b.y; yv[8 * ks + 6] = b.z; yv[8 * ks + 7] = b.w;
    }
    // the sum of squares in the quantizer's order (leaf j = y[j]^2 + y[j + 64]^2, then pairs j, j ^ 32;
    // j, j ^ 16; ...; j, j ^ 1), so rms and the fp16 scale are the quantizer's to the bit.  This lane
    // holds leaves 8 g + e and 8 g + e + 32; leaves 16 apart sit in lanes 32 apart, 8 apart 16.
    double ps[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const double s0 = static_cast<double>(yv[e]) * yv[e] + static_cast<double>(yv[16 + e]) * yv[16 + e];
      const double s1 = static_cast<double>(yv[8 + e]) * yv[8 + e] + static_cast<double>(yv[24 + e]) * yv[24 + e];
      ps[e] = s0 + s1;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) ps[e] += __shfl_xor(ps[e], 32, 64);
#pragma unroll
    for (int e = 0; e < 8; ++e) ps[e] += __shfl_xor(ps[e], 16, 64);
#pragma unroll
    for (int e = 0; e < 4; ++e) ps[e] += ps[e + 4];
    const double ss = (ps[0] + ps[2]) + (ps[1] + ps[3]);
    const float rms = sqrt_rn(static_cast<float>(ss / kSD));
    float q[kSMaxBits][4];
#pragma unroll
    for (int b = 0; b < kSMaxBits; ++b) {
      if (b >= w.n) continue;                                   // uniform
      const int bits = w.bits[b];
      const float sc = fmaxf(as_stored16(__fmul_rn(w.step[b], rms)), kMinScale);
      const float half = static_cast<float>((1 << bits) - 1) * 0.5f;
      const float qmax = static_cast<float>((1 << bits) - 1);
      float ev[32], emx = 0.0f;
#pragma unroll
      for (int k = 0; k < 32; ++k) {
        const float c = fminf(fmaxf(rintf(__fadd_rn(__fdiv_rn(yv[k], sc), half)), 0.0f), qmax);
        ev[k] = __fsub_rn(__fmul_rn(__fsub_rn(c, half), sc), yv[k]);
        emx = fmaxf(emx, fabsf(ev[k]));
      }
      emx = xmax32(xmax16(emx));
      int ex = 0;
      if (emx > 0.0f) (void)frexpf(emx, &ex);
      const float upe = ldexpf(1.0f, 8 - ex);
      u32x4 eh[4], elo[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        float x8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x8[e] = ev[8 * ks + e] * upe;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const _Float16 h0 = static_cast<_Float16>(x8[2 * e]), h1 = static_cast<_Float16>(x8[2 * e + 1]);
          eh[ks][e] = pack_h2(h0, h1);
          elo[ks][e] = pack_h2(static_cast<_Float16>(x8[2 * e] - static_cast<float>(h0)),
                               static_cast<_Float16>(x8[2 * e + 1] - static_cast<float>(h1)));
        }
        *reinterpret_cast<float4*>(&es[wave][nl][32 * ks + 8 * g]) = make_float4(x8[0], x8[1], x8[2], x8[3]);
        *reinterpret_cast<float4*>(&es[wave][nl][32 * ks + 8 * g + 4]) = make_float4(x8[4], x8[5], x8[6], x8[7]);
      }
      if (g == 0) eex[wave][nl] = ex;
      wave_lds_fence();
      float dot[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int cb = 0; cb < 8; ++cb) {
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const int o = (16 * cb + nl) * kSMtStride + 32 * ks + 8 * g;
          const u32x4 bhi = *reinterpret_cast<const u32x4*>(&mt[0][o]);
          const u32x4 blo = *reinterpret_cast<const u32x4*>(&mt[1][o]);
          acc = mfma(as_half8(eh[ks]), as_half8(bhi), acc);
          acc = mfma(as_half8(eh[ks]), as_half8(blo), acc);
          acc = mfma(as_half8(elo[ks]), as_half8(bhi), acc);
        }
        // D lane (g, nl) register i: token 4g + i of the tile, column 16 cb + nl
#pragma unroll
        for (int i = 0; i < 4; ++i) dot[i] = __builtin_fmaf(acc[i], es[wave][4 * g + i][16 * cb + nl], dot[i]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) q[b][i] = ldexpf(row_sum16(dot[i]), 2 * eex[wave][4 * g + i] + em - 24);
      wave_lds_fence();                                         // es, eex of this width are read
    }
    // e^T M e = q x 2^(2 ex + em - 24): e and M entered as e 2^(8 - ex) and M 2^(8 - em)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t tt = t0 + 4 * g + i;
      if (nl == 0 && tt < t_end)
        for (int b = 0; b < w.n; ++b) err[(bh * n + tt) * w.n + b] = q[b][i];
    }
  }
}

// D[h][t] = [DD, A errK_b + W errV_b for each width, 0] (float32, products rounded before the sum)
__global__ __launch_bounds__(256) void strata_dtable_kernel(const float* __restrict__ ek, const float* __restrict__ ev,
                                                            const float* __restrict__ A, const float* __restrict__ W,
                                                            const float* __restrict__ DD, int nb, int64_t total,
                                                            float* __restrict__ D) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    float* row = D + i * (nb + 2);
    row[0] = DD[i];
    for (int b = 0; b < nb; ++b) row[1 + b] = __fadd_rn(__fmul_rn(A[i], ek[i * nb + b]), __fmul_rn(W[i], ev[i * nb + b]));
    row[nb + 1] = 0.0f;
  }
}

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
  if (n >= 1024) {
    // P chunks of >= 256 tokens; their float64 partials (BH P 128 doubles <= BH n 128 floats) sit
    // in y until the rotation overwrites it
    const int64_t P = std::min<int64_t>(64, n / 256);
    const int64_t chunk = (n + P - 1) / P;
    double* part = reinterpret_cast<double*>(y);
    KVQ_DISPATCH_DTYPE(x_dtype, hipLaunchKernelGGL((strata_mean_part_kernel<DT_>),
                                                  dim3(static_cast<unsigned>(BH), static_cast<unsigned>(P)), dim3(1024),
                                                  0, s, x, n, x_bh, chunk, part));
    hipLaunchKernelGGL(strata_mean_combine_kernel, dim3(static_cast<unsigned>(BH)), dim3(kSD), 0, s, part,
                       static_cast<int>(P), n, mu);
  } else {
    KVQ_DISPATCH_DTYPE(x_dtype, hipLaunchKernelGGL((strata_mean_kernel<DT_>), dim3(static_cast<unsigned>(BH)),
                                                  dim3(1024), 0, s, x, n, x_bh, mu));
  }
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

// =============================================================================================
// A6  STRATA tier decode: split-K flash-decoding partials of one stratum (STRATA_KV.py:1374-1469
// computes the same with a Triton kernel over planar rows; tier_reference 1751-1760), merged with
// the exact rows' partials and rotated back (StrataState.attend 1762-1795).
//
// Per (b, h, split): 4 wavefronts each stream an equal share of 32-token chunks.  Logit of token j
// for row r (base 2): s = ks_j * (q^ . c_j - half * sum(q^)) + qb, q^ = scaling*log2(e) * q R^T.
// The dot q^ . c_j runs on v_mfma_f32_16x16x32_f16 with the codes masked in place as fp16
// subnormals (a code at bit offset o within a 16-bit half is c * 2^o * 2^-24, exact) against the
// query operand q^ * Smax / 2^o split into fp16 hi / lo columns.  Values: p * vs as the B operand
// of the same product over value tiles; the offset -half * sum(p * vs) is added to every channel.
namespace kvq {
namespace {

constexpr int kSThreads = 256;
constexpr int kSWaves = 4;

constexpr int kMaxTiers = 16;

// One stratum of the launch: its codes, scales and split range [s_base, s_base + n_split).
// Dispatch-class weights of the strata's splits (see class_block_of): the mixed-width decode's
// (measured at the C3 shape: 29.6 us per step, against 30.0 with the KIVI decode's 141 : 98 : 68,
// 30.0 without classes and 30.2 with 125 : 100 : 80; steeper weights, 180 : 92 : 50 and
// 200 : 85 : 42, 0.6 and 1.2 us slower)
#ifndef KVQ_STRATA_CLASS_W
#define KVQ_STRATA_CLASS_W 165, 95, 55
#endif
#ifndef KVQ_STRATA_CLASSES
#define KVQ_STRATA_CLASSES 1
#endif
constexpr int kStrataClassW[3] = {KVQ_STRATA_CLASS_W};
constexpr int kStrataClassWSum = kStrataClassW[0] + kStrataClassW[1] + kStrataClassW[2];

struct StrataTierArg {
  const uint8_t* kc;            // (BH, n_t, d*bits/8) planar rows
  const uint16_t* ks;           // (BH, cap_t) fp16, zero past n_t
  const uint8_t* vt;            // (BH, cap_t/32, 512*bits) value tiles
  const uint16_t* vsl;          // (BH, cap_t/32, 32) fp16 slot-ordered value scales
  int64_t n_t, cap_t;           // tier tokens, tile capacity
  int n_split, s_base, bits;
};

struct StrataParams {
  const void* q;
  int64_t q_sb, q_sh, q_st;
  int Hq, Hkv, Tq, rep, R_real, BH;
  float qscale;                 // scaling * log2(e)
  const float* signs;           // (d) +-1
  const uint16_t* mu_k;         // (BH, d) fp16
  const uint16_t* mu_v;
  int n_tiers;                  // strata with tokens, in launch order
  StrataTierArg tiers[kMaxTiers];
  float* ws_o;                  // tier partials (BH * S_all partials)
  float* ws_m;
  float* ws_l;
  int S_all;
  int split_classes;            // 3: class-major blocks (split sa = 3 j + class), splits sized by class
  ExactArgs ex;                 // exact rows attended in the merge (ex.n > 0)
  const float* ex_o;            // exact-row partials (BH * S_ex partials)
  const float* ex_m;
  const float* ex_l;
  int S_ex;
  void* out;
  // pre-rotated query rows (kvq_strata_tier_partials): qr (BH, qr_rows, d) = scaling * q R^T and
  // qb (BH, qr_rows) = scaling * q . mu_K; the launch takes rows [qr_r0, qr_r0 + R_real).  Null: the
  // query is read from q and rotated here.
  const float* qr;
  const float* qb;
  int qr_rows, qr_r0;
  // partials in the reference's layout and units (natural exponent): m, l, z (BH, S_all, qr_rows),
  // acc (BH, S_all, qr_rows, d).  Null: partials go to the decode's workspace (base 2).
  float* t_m;
  float* t_l;
  float* t_acc;
  float* t_z;
};

constexpr float kStrataLog2e = 1.4426950408889634f;
constexpr float kStrataLn2 = 0.6931471805599453f;

__device__ __forceinline__ int64_t strata_q_offset(const StrataParams& p, int b, int h, int r) {
  const int hq = h * p.rep + r / p.Tq, t = r % p.Tq;
  return static_cast<int64_t>(b) * p.q_sb + static_cast<int64_t>(hq) * p.q_sh + static_cast<int64_t>(t) * p.q_st;
}

template <int BITS>
struct StrataChunk {
  static constexpr int KW = BITS;               // key words per tile per lane (4*BITS bytes)
  static constexpr int VW = 2 * BITS;           // value words per lane per chunk
  uint32_t kw[2][KW];
  uint32_t ksw[2][2];
  uint32_t vw[VW];
  u32x4 vsw;
};

template <int BITS, int R, int DT>
__device__ void strata_block(const StrataParams& p, const StrataTierArg& ta, int bh, int sidx, float* smem) {
  constexpr int NCLS = BITS == 2 ? 4 : (BITS == 4 ? 2 : 1);   // probability classes (code factors)
  constexpr int RB = 16 * BITS;                 // bytes per planar row
  const int b = bh / p.Hkv, h = bh % p.Hkv;
  float (*qs)[kSD] = reinterpret_cast<float (*)[kSD]>(smem);  // rotated, scaled query rows
  float* qsum = smem + R * kSD;
  float* qbias = qsum + R;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const int l = threadIdx.x % 64;
  const int g = l >> 4, n = l & 15;
  const int r_n = n % R;
  const int hl_qk = (n / R) & 1;
  const int v_pv = n / R;
  const int gcl = v_pv >> 1, hl_pv = v_pv & 1;

  // ---- query rows: q^ = FWHT(q * s) / sqrt(d) * qscale, sum(q^), qb = qscale * q . mu_K ----
  for (int r = wave; r < R; r += kSWaves) {
    float v0 = 0.0f, v1 = 0.0f, mk = 0.0f, qbv = 0.0f;
    if (r < p.R_real && p.qr != nullptr) {
      const int64_t qo = static_cast<int64_t>(bh) * p.qr_rows + p.qr_r0 + r;
      v0 = p.qr[qo * kSD + l] * kStrataLog2e;
      v1 = p.qr[qo * kSD + l + 64] * kStrataLog2e;
      qbv = p.qb[qo] * kStrataLog2e;
    } else if (r < p.R_real) {
      const int64_t qo = strata_q_offset(p, b, h, r);
      const float x0 = load_as_f32<DT>(p.q, qo + l), x1 = load_as_f32<DT>(p.q, qo + l + 64);
      mk = x0 * f16_to_f32(p.mu_k[static_cast<int64_t>(bh) * kSD + l]) +
           x1 * f16_to_f32(p.mu_k[static_cast<int64_t>(bh) * kSD + l + 64]);
      v0 = x0 * p.signs[l];
      v1 = x1 * p.signs[l + 64];
      fwht128(v0, v1, l);
      const float f = 0.08838834764831845f * p.qscale;
      v0 *= f;
      v1 *= f;
    }
    qs[r][l] = v0;
    qs[r][l + 64] = v1;
    const float su = wave_sum(v0 + v1);
    mk = wave_sum(mk);
    if (l == 0) {
      qsum[r] = su;
      qbias[r] = p.qr != nullptr ? qbv : mk * p.qscale;
    }
  }
  __syncthreads();
  // ---- query operand of the key product (fixed for the block) ----
  half8 bqk[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = qs[r_n][key_channel<BITS>(g, w, e)] *
                      static_cast<float>(1 << (smax_shift<BITS>() - code_shift<BITS>(e)));
      const _Float16 hi = static_cast<_Float16>(x);
      bqk[w][e] = hl_qk ? static_cast<_Float16>(x - static_cast<float>(hi)) : hi;
    }
  }
  const float half = static_cast<float>((1 << BITS) - 1) * 0.5f;
  const float hq = half * qsum[r_n];
  const float qbr = qbias[r_n];
  constexpr float kDotScale = static_cast<float>(1 << (24 - smax_shift<BITS>()));   // dot = D * this

  // ---- this wavefront's chunk range: the stratum's chunks over its splits' 4 wavefronts each, in
  // proportion to the splits' dispatch-class weights when the plan has classes (a stratum's splits
  // then cycle through the classes: split i is of class i % 3), else equally ----
  const int NC = static_cast<int>((ta.n_t + 31) / 32);
  int64_t wb0, wb1, wtot;
  if (p.split_classes > 0) {
    const int c = sidx % 3;
    const int64_t before = static_cast<int64_t>(sidx / 3) * kStrataClassWSum + (c > 0 ? kStrataClassW[0] : 0) +
                           (c > 1 ? kStrataClassW[1] : 0);
    wb0 = kSWaves * before + static_cast<int64_t>(wave) * kStrataClassW[c];
    wb1 = wb0 + kStrataClassW[c];
    wtot = static_cast<int64_t>(kSWaves) * (ta.n_split / 3) * kStrataClassWSum;
  } else {
    wb0 = sidx * kSWaves + wave;
    wb1 = wb0 + 1;
    wtot = static_cast<int64_t>(ta.n_split) * kSWaves;
  }
  const int t0 = 32 * static_cast<int>(wb0 * NC / wtot);
  const int t1 = min(32 * static_cast<int>(wb1 * NC / wtot), static_cast<int>(ta.n_t));
  const int t_last = t0 < t1 ? t0 + ((t1 - 1 - t0) & ~31) : t0;

  const __amdgpu_buffer_rsrc_t rk =
      make_rsrc(ta.kc + static_cast<int64_t>(bh) * ta.n_t * RB, static_cast<uint32_t>(ta.n_t * RB));
  // key scales padded to the tile capacity: a 4-token load never straddles the end of the row
  const __amdgpu_buffer_rsrc_t rks =
      make_rsrc(ta.ks + static_cast<int64_t>(bh) * ta.cap_t, static_cast<uint32_t>(ta.cap_t * 2));
  const __amdgpu_buffer_rsrc_t rv =
      make_rsrc(ta.vt + static_cast<int64_t>(bh) * (ta.cap_t / 32) * 512 * BITS,
                static_cast<uint32_t>((ta.cap_t / 32) * 512 * BITS));
  const __amdgpu_buffer_rsrc_t rvs =
      make_rsrc(ta.vsl + static_cast<int64_t>(bh) * ta.cap_t, static_cast<uint32_t>(ta.cap_t * 2));
  const int vo_k = n * RB + g * 4 * BITS;

  using Chunk = StrataChunk<BITS>;
  auto load_chunk = [&](int cb, Chunk& c) {
    cb = min(cb, t_last);
    const int so = __builtin_amdgcn_readfirstlane(cb * RB);
#pragma unroll
    for (int tau = 0; tau < 2; ++tau) {
      const int vo = vo_k + tau * 16 * RB;
      if constexpr (BITS == 2) {
        const auto x = __builtin_amdgcn_raw_buffer_load_b64(rk, vo, so, 2);
        c.kw[tau][0] = x[0];
        c.kw[tau][1] = x[1];
      } else {
#pragma unroll
        for (int i = 0; i < BITS / 4; ++i) {
          const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rk, vo + 16 * i, so, 2);
#pragma unroll
          for (int k = 0; k < 4; ++k) c.kw[tau][4 * i + k] = x[k];
        }
      }
      const auto kx = __builtin_amdgcn_raw_buffer_load_b64(rks, (16 * tau + 4 * g) * 2,
                                                           __builtin_amdgcn_readfirstlane(cb * 2), 0);
      c.ksw[tau][0] = kx[0];
      c.ksw[tau][1] = kx[1];
    }
    const int sv = __builtin_amdgcn_readfirstlane((cb / 32) * 512 * BITS);
#pragma unroll
    for (int i = 0; i < BITS / 2; ++i) {
      const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rv, l * 16 + 1024 * i, sv, 2);
#pragma unroll
      for (int k = 0; k < 4; ++k) c.vw[4 * i + k] = x[k];
    }
    c.vsw = __builtin_amdgcn_raw_buffer_load_b128(rvs, g * 16, __builtin_amdgcn_readfirstlane((cb / 32) * 64), 0);
  };

  f32x4 acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;
  float lc[NCLS], zc[NCLS];
#pragma unroll
  for (int k = 0; k < NCLS; ++k) lc[k] = zc[k] = 0.0f;
  const half2v hl_neg = hl_pv ? half2v{static_cast<_Float16>(-1.0f), static_cast<_Float16>(-1.0f)}
                              : half2v{static_cast<_Float16>(0.0f), static_cast<_Float16>(0.0f)};
  constexpr float kLazy = 4.0f;

  auto cls = [](int j) -> int { return BITS == 2 ? (j >> 1) : (BITS == 4 ? (((j & 3) >= 2) ? 1 : 0) : 0); };
  auto step = [&](int cb, const Chunk& c) {
    float s[8];
#pragma unroll
    for (int tau = 0; tau < 2; ++tau) {
      f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        half8 a;
        if constexpr (BITS == 4) a = unpack4(c.kw[tau][w]);
        else if constexpr (BITS == 8) a = unpack8(c.kw[tau][2 * w], c.kw[tau][2 * w + 1]);
        else a = unpack2((w & 1) ? (c.kw[tau][w >> 1] >> 8) : c.kw[tau][w >> 1]);
        d = mfma(a, bqk[w], d);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float dot = d[i] + dpp<kRowRor + R>(d[i]);                          // hi + lo columns
        const float ks = h2f(c.ksw[tau][i >> 1], i & 1);
        s[4 * tau + i] = __builtin_fmaf(ks, __builtin_fmaf(dot, kDotScale, -hq), qbr);
      }
    }
    if (cb + 32 > t1) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (cb + 16 * (j >> 2) + 4 * g + (j & 3) >= t1) s[j] = -INFINITY;
    }
    float lm = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
    if (__any(lm > m_run + kLazy)) {
      const float m_new = fmaxf(m_run, xmax32(xmax16(lm)));
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[k] *= alpha;
#pragma unroll
      for (int k = 0; k < NCLS; ++k) {
        lc[k] *= alpha;
        zc[k] *= alpha;
      }
      m_run = m_new;
    }
    float pr[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) pr[j] = __builtin_amdgcn_exp2f(s[j] - (m_run + static_cast<float>(code_shift<BITS>(j))));
    uint32_t words[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int j0 = 2 * jj, j1 = 2 * jj + 1;
      const float v0 = h2f(c.vsw[jj], 0), v1 = h2f(c.vsw[jj], 1);          // scales of slots j0, j1
      const half2v hi = half2v{static_cast<_Float16>(__builtin_fmaf(pr[j0], v0, 0.0f)),
                               static_cast<_Float16>(__builtin_fmaf(pr[j1], v1, 0.0f))};
      const half2v cn = hi * hl_neg;
      const half2v val = half2v{static_cast<_Float16>(__builtin_fmaf(pr[j0], v0, static_cast<float>(cn[0]))),
                                static_cast<_Float16>(__builtin_fmaf(pr[j1], v1, static_cast<float>(cn[1])))};
      words[jj] = w2(val);
      lc[cls(j0)] += pr[j0];
      lc[cls(j1)] += pr[j1];
      zc[cls(j0)] = __builtin_fmaf(pr[j0], v0, zc[cls(j0)]);
      zc[cls(j1)] = __builtin_fmaf(pr[j1], v1, zc[cls(j1)]);
    }
    const half8 bp = as_half8(u32x4{words[0], words[1], words[2], words[3]});
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
      half8 a;
      if constexpr (BITS == 4) a = unpack4(c.vw[blk]);
      else if constexpr (BITS == 8) a = unpack8(c.vw[(blk >> 1) * 4 + (blk & 1) * 2], c.vw[(blk >> 1) * 4 + (blk & 1) * 2 + 1]);
      else a = unpack2((blk & 1) ? (c.vw[blk >> 1] >> 8) : c.vw[blk >> 1]);
      acc[blk] = mfma(a, bp, acc[blk]);
    }
  };

  if (t0 < t1) {
    Chunk ca, cb_;
    load_chunk(t0, ca);
    for (int cb = t0;; cb += 64) {
      load_chunk(cb + 32, cb_);
      step(cb, ca);
      if (cb + 32 >= t1) break;
      load_chunk(cb + 64, ca);
      step(cb + 32, cb_);
      if (cb + 64 >= t1) break;
    }
  }

  // ---- wavefront epilogue ----
  float lsum = 0.0f, zsum = 0.0f;
#pragma unroll
  for (int k = 0; k < NCLS; ++k) {
    const float f = static_cast<float>(1 << (BITS == 2 ? 2 * k : 4 * k));
    lsum = __builtin_fmaf(lc[k], f, lsum);
    zsum = __builtin_fmaf(zc[k], f, zsum);
  }
  const float l_run = xsum32(xsum16(lsum));
  const float Z = -half * xsum32(xsum16(zsum));
  __syncthreads();
  float* red_o = smem;                           // [wave][R][d]
  float* red_ml = smem + kSWaves * R * kSD;      // [wave][2][R]
  constexpr float kTwo24 = 16777216.0f;
#pragma unroll
  for (int blk = 0; blk < 8; ++blk) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = acc[blk][i] + dpp<kRowShr + R>(acc[blk][i]);
      if (hl_pv == 1 && gcl == 0) red_o[(wave * R + r_n) * kSD + 16 * blk + 4 * g + i] = __builtin_fmaf(a, kTwo24, Z);
    }
  }
  if (g == 0 && n < R) {
    red_ml[(wave * 2 + 0) * R + n] = m_run;
    red_ml[(wave * 2 + 1) * R + n] = l_run;
  }
  __syncthreads();
  const int64_t po = static_cast<int64_t>(bh) * p.S_all + ta.s_base + sidx;
  for (int idx = threadIdx.x; idx < p.R_real * kSD; idx += kSThreads) {
    const int r = idx / kSD, c = idx % kSD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kSWaves; ++w) M = fmaxf(M, red_ml[(w * 2) * R + r]);
    float O = 0.0f, L = 0.0f;
#pragma unroll
    for (int w = 0; w < kSWaves; ++w) {
      const float mw_ = red_ml[(w * 2) * R + r];
      const float wgt = (mw_ == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw_ - M);
      O += wgt * red_o[(w * R + r) * kSD + c];
      L += wgt * red_ml[(w * 2 + 1) * R + r];
    }
    if (p.t_m != nullptr) {
      // the reference's partial (m, l, acc, z): natural exponent, the value offset folded into acc
      const int64_t to = po * p.qr_rows + p.qr_r0 + r;
      p.t_acc[to * kSD + c] = O;
      if (c == 0) {
        p.t_m[to] = M * kStrataLn2;
        p.t_l[to] = L;
        p.t_z[to] = 0.0f;
      }
    } else {
      p.ws_o[(po * R + r) * kSD + c] = O;
      if (c == 0) {
        p.ws_m[po * R + r] = M;
        p.ws_l[po * R + r] = L;
      }
    }
  }
}

// Every stratum in one launch: block id -> (XCD-aware) bh and split index over all strata; the
// stratum owning the split picks the width-specialised body.  W: waves per SIMD the registers
// target (3: every width's body fits 164 VGPRs).
template <int R, int DT, int W>
__global__ __launch_bounds__(kSThreads) __attribute__((amdgpu_waves_per_eu(W)))
void strata_split_all(StrataParams p) {
  extern __shared__ float smem[];
  int bh, sa;
  if (p.split_classes > 0) {
    // class-major (class_block_of), and the class's j-th split of a (b, h) is split 3 j + class
    int scm;
    class_block_of(blockIdx.x, p.S_all, 3, &bh, &scm);
    const int q = p.S_all / 3;
    sa = 3 * (scm % q) + scm / q;
  } else {
    const int k = blockIdx.x / 8;
    bh = blockIdx.x % 8 + 8 * (k / p.S_all);
    sa = k % p.S_all;
  }
  if (bh >= p.BH) return;
  int t = 0;
  while (t + 1 < p.n_tiers && sa >= p.tiers[t + 1].s_base) ++t;
  const StrataTierArg& ta = p.tiers[t];
  const int sidx = sa - ta.s_base;
  if (ta.bits == 8) strata_block<8, R, DT>(p, ta, bh, sidx, smem);
  else if (ta.bits == 4) strata_block<4, R, DT>(p, ta, bh, sidx, smem);
  else strata_block<2, R, DT>(p, ta, bh, sidx, smem);
}

// Merge of one (b, h, row): exact rows (unrotated; as partials of exact-row blocks, or attended
// here when the window fits the merge) and every tier partial (rotated basis):
// o = [sum_e w o_e + (sum_t w o_t) R + (sum_t w l_t) mu_V] / sum_all w l   (STRATA_KV.py:1784-1792).
// The partials are spread over the block's 256 threads (block reductions for the maximum and the
// sums, 128 channels x 2 partial halves for the output columns); one wavefront rotates the coded
// sum back to the channel basis (FWHT).
template <int R, int DT>
__global__ __launch_bounds__(kSThreads) void strata_merge(StrataParams p) {
  __shared__ float red[4];
  __shared__ float oc[2][kSD], oe[2][kSD];
  __shared__ float4 oi[8][kSD / 4];
  __shared__ float sl[kExactInMerge];
  const int bh = blockIdx.x / p.R_real, r = blockIdx.x % p.R_real;
  const int b = bh / p.Hkv, h = bh % p.Hkv;
  const int hq = h * p.rep + r / p.Tq, tq = r % p.Tq;
  const int tid = threadIdx.x, lane = tid % 64;
  auto reduce = [&](float v, bool is_max) -> float {
    v = is_max ? wave_max(v) : wave_sum(v);
    __syncthreads();
    if (lane == 0) red[tid / 64] = v;
    __syncthreads();
    return is_max ? fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])) : (red[0] + red[1]) + (red[2] + red[3]);
  };
  auto em = [&](int s) { return p.ex_m[(static_cast<int64_t>(bh) * p.S_ex + s) * R + r]; };
  auto cm = [&](int s) { return p.ws_m[(static_cast<int64_t>(bh) * p.S_all + s) * R + r]; };
  auto cl = [&](int s) { return p.ws_l[(static_cast<int64_t>(bh) * p.S_all + s) * R + r]; };
  // the first coded statistics are loaded before the exact pass so their latency overlaps it
  const float mc0 = tid < p.S_all ? cm(tid) : -INFINITY;
  const float lc0 = tid < p.S_all ? cl(tid) : 0.0f;
  // exact rows attended here (their partial: mi, li, and the value sums in channel-quad layout)
  float mi = -INFINITY, li = 0.0f;
  float4 o4 = make_float4(0.f, 0.f, 0.f, 0.f);
  if (p.ex.n > 0) exact_partial<DT, kSD>(p.ex, b, hq, tq, bh, sl, red, mi, li, o4, tid % 32, tid / 32);
  float m = fmaxf(mi, mc0);
  for (int s = tid; s < p.S_ex; s += kSThreads) m = fmaxf(m, em(s));
  for (int s = tid + kSThreads; s < p.S_all; s += kSThreads) m = fmaxf(m, cm(s));
  const float M = reduce(m, true);
  const float wi = mi == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mi - M);
  float le = 0.0f, lc = mc0 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mc0 - M) * lc0;
  for (int s = tid; s < p.S_ex; s += kSThreads) {
    const float x = em(s);
    if (x != -INFINITY) le += __builtin_amdgcn_exp2f(x - M) * p.ex_l[(static_cast<int64_t>(bh) * p.S_ex + s) * R + r];
  }
  for (int s = tid + kSThreads; s < p.S_all; s += kSThreads) {
    const float x = cm(s);
    if (x != -INFINITY) lc += __builtin_amdgcn_exp2f(x - M) * cl(s);
  }
  const float Le = reduce(le, false) + wi * li;
  const float Lc = reduce(lc, false);
  oi[tid / 32][tid % 32] = make_float4(wi * o4.x, wi * o4.y, wi * o4.z, wi * o4.w);
  const int c = tid % kSD, part = tid / kSD;
  float o_c = 0.0f, o_e = 0.0f;
#pragma unroll 4
  for (int s = part; s < p.S_all; s += 2) {
    const float x = cm(s);
    const float w = x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(x - M);
    o_c = __builtin_fmaf(w, p.ws_o[((static_cast<int64_t>(bh) * p.S_all + s) * R + r) * kSD + c], o_c);
  }
  for (int s = part; s < p.S_ex; s += 2) {
    const float x = em(s);
    const float w = x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(x - M);
    o_e = __builtin_fmaf(w, p.ex_o[((static_cast<int64_t>(bh) * p.S_ex + s) * R + r) * kSD + c], o_e);
  }
  oc[part][c] = o_c;
  oe[part][c] = o_e;
  __syncthreads();
  if (tid < 64) {                                 // coded sum back to the channel basis: x R
    float v0 = oc[0][tid] + oc[1][tid], v1 = oc[0][tid + 64] + oc[1][tid + 64];
    fwht128(v0, v1, tid);
    oc[0][tid] = v0 * 0.08838834764831845f * p.signs[tid];
    oc[0][tid + 64] = v1 * 0.08838834764831845f * p.signs[tid + 64];
  }
  __syncthreads();
  if (part == 0) {
    float O = oc[0][c] + Lc * f16_to_f32(p.mu_v[static_cast<int64_t>(bh) * kSD + c]) + oe[0][c] + oe[1][c];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float4 v = oi[k][c >> 2];
      O += (c & 3) == 0 ? v.x : (c & 3) == 1 ? v.y : (c & 3) == 2 ? v.z : v.w;
    }
    store_from_f32<DT>(p.out, ((static_cast<int64_t>(b) * p.Tq + tq) * p.Hq + hq) * kSD + c, O / (Le + Lc));
  }
}

// The merge of one (b, h, row) when no exact rows are attended here and the row has at most NS
// (<= 32) partials: one wavefront per row (four rows a workgroup, rows in strata_merge's grid order),
// lane s holding partial s's (m, l) (exact-row partials first, then the strata's) and lane l channels
// l and l + 64 of every partial's o, the FWHT's two coordinates; every load at once, wavefront
// reductions, the coded sum rotated back in registers; no LDS and no barrier.  Same formula as
// strata_merge: o = [sum_e w o_e + (sum_t w o_t) R + (sum_t w l_t) mu_V] / sum_all w l.
template <int R, int DT, int NS>
__global__ __launch_bounds__(kSThreads) void strata_merge_wave(StrataParams p, int n_rows) {
  const int row = static_cast<int>(blockIdx.x) * 4 + static_cast<int>(threadIdx.x >> 6);
  if (row >= n_rows) return;
  const int lane = threadIdx.x & 63;
  const int bh = row / p.R_real, r = row % p.R_real;
  const int S_ex = p.S_ex, S_all = p.S_ex + p.S_all;
  auto o_ptr = [&](int s) -> const float* {
    return s < S_ex ? p.ex_o + ((static_cast<int64_t>(bh) * S_ex + s) * R + r) * kSD
                    : p.ws_o + ((static_cast<int64_t>(bh) * p.S_all + (s - S_ex)) * R + r) * kSD;
  };
  float ms = -INFINITY, ls = 0.0f;
  if (lane < S_all) {
    ms = lane < S_ex ? p.ex_m[(static_cast<int64_t>(bh) * S_ex + lane) * R + r]
                     : p.ws_m[(static_cast<int64_t>(bh) * p.S_all + (lane - S_ex)) * R + r];
    ls = lane < S_ex ? p.ex_l[(static_cast<int64_t>(bh) * S_ex + lane) * R + r]
                     : p.ws_l[(static_cast<int64_t>(bh) * p.S_all + (lane - S_ex)) * R + r];
  }
  float2 ov[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const float* o = o_ptr(s < S_all ? s : S_all - 1);
    ov[s] = float2{o[lane], o[lane + 64]};
  }
  const float M = wave_max(ms);
  const float w = ms == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ms - M);   // 0 past S_all
  const float Le = wave_sum(lane < S_ex ? w * ls : 0.0f);
  const float Lc = wave_sum(lane >= S_ex ? w * ls : 0.0f);
  float c0 = 0.0f, c1 = 0.0f, e0 = 0.0f, e1 = 0.0f;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const float ws = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), s));
    const bool ex = s < S_ex;
    e0 = __builtin_fmaf(ex ? ws : 0.0f, ov[s].x, e0);
    e1 = __builtin_fmaf(ex ? ws : 0.0f, ov[s].y, e1);
    c0 = __builtin_fmaf(ex ? 0.0f : ws, ov[s].x, c0);
    c1 = __builtin_fmaf(ex ? 0.0f : ws, ov[s].y, c1);
  }
  fwht128(c0, c1, lane);                                   // coded sum back to the channel basis: x R
  c0 *= 0.08838834764831845f * p.signs[lane];
  c1 *= 0.08838834764831845f * p.signs[lane + 64];
  const int b = bh / p.Hkv, h = bh % p.Hkv;
  const int hq = h * p.rep + r / p.Tq, tq = r % p.Tq;
  const float L = Le + Lc;
  const int64_t o0 = ((static_cast<int64_t>(b) * p.Tq + tq) * p.Hq + hq) * kSD + lane;
  store_from_f32<DT>(p.out, o0, (c0 + Lc * f16_to_f32(p.mu_v[static_cast<int64_t>(bh) * kSD + lane]) + e0) / L);
  store_from_f32<DT>(p.out, o0 + 64,
                     (c1 + Lc * f16_to_f32(p.mu_v[static_cast<int64_t>(bh) * kSD + lane + 64]) + e1) / L);
}

inline int strata_pow2(int64_t r) {
  int R = 1;
  while (R < r) R <<= 1;
  return R;
}

// Splits per stratum: about one round of resident blocks (resident_per_cu x 256 CUs) shared in
// proportion to each stratum's bytes (tokens x (32 bits + 8) B: K and V codes and scales).  When a
// round of 3 blocks per CU holds 768 / BH splits per (b, h), a multiple of 3 of them per stratum
// (each stratum with enough chunks for its splits' wavefronts), the plan has dispatch classes:
// returns 3 (0 otherwise), with every stratum's split count a multiple of 3.
inline int strata_plan(int64_t BH, int n_tiers, const int* tier_bits, const int64_t* tier_n, int* ns) {
  double total = 0.0;
  for (int t = 0; t < n_tiers; ++t) total += static_cast<double>(tier_n[t]) * (32 * tier_bits[t] + 8);
  const double target = 256.0 * 3 / static_cast<double>(BH);             // splits per (b, h)
  for (int t = 0; t < n_tiers; ++t) {
    const int64_t nc = (tier_n[t] + 31) / 32;
    const double share = total > 0 ? target * static_cast<double>(tier_n[t]) * (32 * tier_bits[t] + 8) / total : 1.0;
    int64_t s = static_cast<int64_t>(share + 0.5);
    s = std::max<int64_t>(1, std::min<int64_t>(s, (nc + kSWaves - 1) / kSWaves));
    ns[t] = tier_n[t] > 0 ? static_cast<int>(s) : 0;
  }
  if (KVQ_STRATA_CLASSES == 0 || BH <= 0 || BH % 8 != 0 || 768 % BH != 0 || (768 / BH) % 3 != 0 || total <= 0) return 0;
  // units of 3 splits (one per class): one per stratum with tokens, the rest by largest deficit
  const int units = static_cast<int>(768 / BH / 3);
  int alloc[16] = {0}, cap[16] = {0}, used = 0;
  for (int t = 0; t < n_tiers; ++t) {
    if (tier_n[t] <= 0) continue;
    cap[t] = static_cast<int>(((tier_n[t] + 31) / 32 + kSWaves - 1) / kSWaves / 3);   // splits <= ceil(chunks / 4)
    if (cap[t] < 1) return 0;
    alloc[t] = 1;
    ++used;
  }
  if (used == 0 || used > units) return 0;
  for (; used < units; ++used) {
    int best = -1;
    double best_d = -1e300;
    for (int t = 0; t < n_tiers; ++t) {
      if (alloc[t] == 0 || alloc[t] >= cap[t]) continue;
      const double d = units * static_cast<double>(tier_n[t]) * (32 * tier_bits[t] + 8) / total - alloc[t];
      if (d > best_d) {
        best_d = d;
        best = t;
      }
    }
    if (best < 0) return 0;
    ++alloc[best];
  }
  for (int t = 0; t < n_tiers; ++t) ns[t] = 3 * alloc[t];
  return 3;
}

}  // namespace
}  // namespace kvq

extern "C" int64_t kvq_kivi_decode_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d, int64_t n_q,
                                             int64_t n_exact, int group_k, int group_v, int64_t split_tokens);
extern "C" int kvq_kivi_decode(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st, int64_t B,
                               int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d, float scaling, const uint8_t* kc,
                               const uint16_t* k_lo, const uint16_t* k_sc, const uint8_t* vc, const uint16_t* vmeta,
                               int64_t cap_t, int64_t n_q, int group_k, int group_v, const void* k_exact,
                               const void* v_exact, int exact_dtype, int64_t cap_e, int64_t n_exact,
                               const int64_t* exact_pos, const int64_t* q_pos, void* out, int out_dtype,
                               float* workspace, int64_t workspace_floats, float* scores, int64_t scores_bh,
                               float score_weight, int64_t split_tokens, int phases, void* stream);

namespace {
int64_t strata_ws_parts(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t n_exact, int n_tiers,
                        const int* tier_bits, const int64_t* tier_n, int64_t* ex_floats, int* S_all) {
  int ns[16];
  kvq::strata_plan(B * Hkv, n_tiers, tier_bits, tier_n, ns);
  int S = 0;
  for (int t = 0; t < n_tiers; ++t) S += ns[t];
  *S_all = S;
  *ex_floats = (n_exact > 0 && !kvq::exact_in_merge(n_exact))
                   ? kvq_kivi_decode_workspace(B, Hq, Hkv, Tq, 128, 0, n_exact, 32, 32, 0) : 0;
  const int64_t R = kvq::strata_pow2((Hq / Hkv) * Tq);
  return *ex_floats + B * Hkv * static_cast<int64_t>(S) * R * (128 + 2);
}
}  // namespace

extern "C" int64_t kvq_strata_decode_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d,
                                               int64_t n_exact, int n_tiers, const int* tier_bits,
                                               const int64_t* tier_n) {
  if (d != 128 || B <= 0 || Hkv <= 0 || Hq % Hkv != 0 || Tq <= 0 || n_tiers < 0 || n_tiers > 16) return -1;
  if (n_tiers > 0 && (tier_n == nullptr || tier_bits == nullptr)) return -1;
  for (int t = 0; t < n_tiers; ++t)
    if (tier_bits[t] != 2 && tier_bits[t] != 4 && tier_bits[t] != 8) return -1;
  int64_t ex;
  int S;
  return strata_ws_parts(B, Hq, Hkv, Tq, n_exact, n_tiers, tier_bits, tier_n, &ex, &S);
}

extern "C" int kvq_strata_decode(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st, int64_t B,
                                 int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d, float scaling, const float* signs,
                                 const uint16_t* mu_k, const uint16_t* mu_v, int n_tiers, const int* tier_bits,
                                 const int64_t* tier_n, const int64_t* tier_cap, const uint8_t* const* tier_kc,
                                 const uint16_t* const* tier_ks, const uint8_t* const* tier_vt,
                                 const uint16_t* const* tier_vsl, const void* k_exact, const void* v_exact,
                                 int64_t cap_e, int64_t n_exact, const int64_t* exact_pos, const int64_t* q_pos,
                                 void* out, float* workspace, int64_t workspace_floats, void* stream) {
  using namespace kvq;
  KVQ_REQUIRE(d == 128, "kvq_strata_decode: head_dim must be 128");
  KVQ_REQUIRE(valid_dtype(q_dtype), "kvq_strata_decode: bad dtype");
  KVQ_REQUIRE(B > 0 && Hkv > 0 && Hq % Hkv == 0 && Tq > 0, "kvq_strata_decode: bad head counts");
  const int64_t R_real = (Hq / Hkv) * Tq;
  KVQ_REQUIRE(R_real <= 8, "kvq_strata_decode: rep*Tq must be <= 8");
  KVQ_REQUIRE(n_tiers >= 0 && n_tiers <= 16, "kvq_strata_decode: at most 16 tiers");
  KVQ_REQUIRE(n_tiers == 0 || (tier_bits && tier_n && tier_cap && tier_kc && tier_ks && tier_vt && tier_vsl),
              "kvq_strata_decode: null tier arrays");
  int64_t coded = 0;
  for (int t = 0; t < n_tiers; ++t) {
    KVQ_REQUIRE(tier_bits[t] == 2 || tier_bits[t] == 4 || tier_bits[t] == 8, "kvq_strata_decode: tier bits in {2,4,8}");
    KVQ_REQUIRE(tier_n[t] >= 0 && tier_cap[t] % 32 == 0 && tier_n[t] <= tier_cap[t] && tier_n[t] < (1LL << 30),
                "kvq_strata_decode: tier capacity must be a multiple of 32 holding n");
    KVQ_REQUIRE(tier_n[t] == 0 || (tier_kc[t] && tier_ks[t] && tier_vt[t] && tier_vsl[t]), "kvq_strata_decode: null tier");
    coded += tier_n[t];
  }
  KVQ_REQUIRE(coded == 0 || (signs && mu_k && mu_v), "kvq_strata_decode: null rotation / means");
  KVQ_REQUIRE(coded + n_exact > 0, "kvq_strata_decode: empty cache");
  KVQ_REQUIRE(q && out && workspace, "kvq_strata_decode: null q / out / workspace");
  int64_t ex_floats;
  int S_all;
  const int64_t need = strata_ws_parts(B, Hq, Hkv, Tq, n_exact, n_tiers, tier_bits, tier_n, &ex_floats, &S_all);
  KVQ_REQUIRE(workspace_floats >= need, "kvq_strata_decode: workspace too small (%lld < %lld floats)",
              (long long)workspace_floats, (long long)need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int R = strata_pow2(R_real);
  StrataParams p{};
  p.q = q; p.q_sb = q_sb; p.q_sh = q_sh; p.q_st = q_st;
  p.Hq = (int)Hq; p.Hkv = (int)Hkv; p.Tq = (int)Tq; p.rep = (int)(Hq / Hkv); p.R_real = (int)R_real;
  p.BH = (int)(B * Hkv);
  p.qscale = scaling * 1.4426950408889634f;
  p.signs = signs; p.mu_k = mu_k; p.mu_v = mu_v;
  p.out = out;
  // exact rows: partials of the KIVI exact-row blocks (no packed rows), into the first region
  const bool ex_merge = exact_in_merge(n_exact);
  int ex_rows = 0;
  const int64_t S_ex = (ex_merge || n_exact == 0) ? 0 : plan_exact_blocks(B * Hkv, n_exact, &ex_rows);
  if (ex_merge) {
    p.ex = ExactArgs{q, q_sb, q_sh, q_st, p.qscale, k_exact, v_exact, cap_e, static_cast<int>(n_exact), exact_pos, q_pos};
  } else if (n_exact > 0) {
    const int rc = kvq_kivi_decode(q, q_dtype, q_sb, q_sh, q_st, B, Hq, Hkv, Tq, d, scaling, nullptr, nullptr, nullptr,
                                   nullptr, nullptr, 0, 0, 32, 32, k_exact, v_exact, q_dtype, cap_e, n_exact, exact_pos,
                                   q_pos, out, q_dtype, workspace, ex_floats, nullptr, 0, 0.0f, 0, 1, stream);
    if (rc != KVQ_OK) return rc;
    const int64_t nrow = B * Hkv * S_ex * R;
    p.ex_o = workspace;
    p.ex_m = workspace + nrow * 128;
    p.ex_l = p.ex_m + nrow;
    p.S_ex = (int)S_ex;
  }
  float* tw = workspace + ex_floats;
  const int64_t trow = B * Hkv * static_cast<int64_t>(S_all) * R;
  p.ws_o = tw;
  p.ws_m = tw + trow * 128;
  p.ws_l = p.ws_m + trow;
  p.S_all = S_all;
  int ns[16];
  p.split_classes = strata_plan(B * Hkv, n_tiers, tier_bits, tier_n, ns);
  // strata with tokens, widest first (their blocks carry the most bytes: dispatched first)
  int base = 0;
  for (int pass_bits : {8, 4, 2}) {
    for (int t = 0; t < n_tiers; ++t) {
      if (ns[t] == 0 || tier_bits[t] != pass_bits) continue;
      StrataTierArg& ta = p.tiers[p.n_tiers++];
      ta.kc = tier_kc[t]; ta.ks = tier_ks[t]; ta.vt = tier_vt[t]; ta.vsl = tier_vsl[t];
      ta.n_t = tier_n[t]; ta.cap_t = tier_cap[t];
      ta.n_split = ns[t]; ta.s_base = base; ta.bits = tier_bits[t];
      base += ns[t];
    }
  }
  const int bh_pad = (p.BH + 7) / 8 * 8;
  const size_t split_smem = std::max<size_t>((R * kSD + 2 * R) * sizeof(float),
                                             (kSWaves * R * kSD + kSWaves * 2 * R) * sizeof(float));
  if (S_all > 0) {
    const dim3 grid(static_cast<unsigned>(S_all) * bh_pad);
#define KVQ_STRATA_LAUNCH(R_, DT_) \
    hipLaunchKernelGGL((strata_split_all<R_, DT_, 3>), grid, dim3(kSThreads), split_smem, s, p)
#define KVQ_STRATA_R(DT_)                                                \
    switch (R) {                                                         \
      case 1: KVQ_STRATA_LAUNCH(1, DT_); break;                          \
      case 2: KVQ_STRATA_LAUNCH(2, DT_); break;                          \
      case 4: KVQ_STRATA_LAUNCH(4, DT_); break;                          \
      default: KVQ_STRATA_LAUNCH(8, DT_); break;                         \
    }
    switch (q_dtype) {
      case KVQ_F32: KVQ_STRATA_R(KVQ_F32) break;
      case KVQ_F16: KVQ_STRATA_R(KVQ_F16) break;
      default: KVQ_STRATA_R(KVQ_BF16) break;
    }
#undef KVQ_STRATA_R
#undef KVQ_STRATA_LAUNCH
    KVQ_LAUNCH_CHECK("kvq_strata_decode(tiers)");
  }
  const int n_rows = p.BH * p.R_real;
  const int S_merge = p.S_ex + p.S_all;
  if (p.ex.n == 0 && S_merge >= 1 && S_merge <= 32) {            // one wavefront per row
    const dim3 wgrid(static_cast<unsigned>((n_rows + 3) / 4));
#define KVQ_SMW_N(R_, DT_, N_) hipLaunchKernelGGL((strata_merge_wave<R_, DT_, N_>), wgrid, dim3(kSThreads), 0, s, p, n_rows)
#define KVQ_SMW_L(R_, DT_)                                        \
    do {                                                          \
      if (S_merge <= 8) KVQ_SMW_N(R_, DT_, 8);                    \
      else if (S_merge <= 16) KVQ_SMW_N(R_, DT_, 16);             \
      else KVQ_SMW_N(R_, DT_, 32);                                \
    } while (0)
#define KVQ_SMW_R(DT_)                                            \
    switch (R) {                                                  \
      case 1: KVQ_SMW_L(1, DT_); break;                           \
      case 2: KVQ_SMW_L(2, DT_); break;                           \
      case 4: KVQ_SMW_L(4, DT_); break;                           \
      default: KVQ_SMW_L(8, DT_); break;                          \
    }
    switch (q_dtype) {
      case KVQ_F32: KVQ_SMW_R(KVQ_F32) break;
      case KVQ_F16: KVQ_SMW_R(KVQ_F16) break;
      default: KVQ_SMW_R(KVQ_BF16) break;
    }
#undef KVQ_SMW_R
#undef KVQ_SMW_L
#undef KVQ_SMW_N
    KVQ_LAUNCH_CHECK("kvq_strata_decode(merge)");
    return KVQ_OK;
  }
  const dim3 mgrid(static_cast<unsigned>(n_rows));
#define KVQ_STRATA_MERGE(R_, DT_) hipLaunchKernelGGL((strata_merge<R_, DT_>), mgrid, dim3(kSThreads), 0, s, p)
#define KVQ_STRATA_MR(DT_)                                               \
  switch (R) {                                                           \
    case 1: KVQ_STRATA_MERGE(1, DT_); break;                             \
    case 2: KVQ_STRATA_MERGE(2, DT_); break;                             \
    case 4: KVQ_STRATA_MERGE(4, DT_); break;                             \
    default: KVQ_STRATA_MERGE(8, DT_); break;                            \
  }
  switch (q_dtype) {
    case KVQ_F32: KVQ_STRATA_MR(KVQ_F32) break;
    case KVQ_F16: KVQ_STRATA_MR(KVQ_F16) break;
    default: KVQ_STRATA_MR(KVQ_BF16) break;
  }
#undef KVQ_STRATA_MR
#undef KVQ_STRATA_MERGE
  KVQ_LAUNCH_CHECK("kvq_strata_decode(merge)");
  return KVQ_OK;
}

extern "C" int kvq_strata_tier_partials(const float* qr, const float* qb, int64_t BH, int64_t rows, int64_t d,
                                        int bits, int64_t n, const uint8_t* kc, const uint16_t* ks,
                                        const uint8_t* vt, const uint16_t* vsl, int64_t cap, int64_t n_split,
                                        float* m, float* l, float* acc, float* z, void* stream) {
  using namespace kvq;
  KVQ_REQUIRE(d == 128, "kvq_strata_tier_partials: head_dim must be 128");
  KVQ_REQUIRE(bits == 2 || bits == 4 || bits == 8, "kvq_strata_tier_partials: bits in {2,4,8}");
  KVQ_REQUIRE(BH > 0 && BH < 65536 && rows > 0 && rows < (1 << 20), "kvq_strata_tier_partials: bad head / row counts");
  KVQ_REQUIRE(n > 0 && n < (1LL << 30) && cap % 32 == 0 && n <= cap,
              "kvq_strata_tier_partials: need 0 < n <= cap, cap a multiple of 32");
  KVQ_REQUIRE(n_split > 0 && n_split <= (n + 31) / 32 && n_split * BH < (1LL << 31),
              "kvq_strata_tier_partials: n_split must be in [1, ceil(n / 32)]");
  KVQ_REQUIRE(qr && qb && kc && ks && vt && vsl && m && l && acc && z, "kvq_strata_tier_partials: null pointer");
  StrataParams p{};
  p.BH = static_cast<int>(BH);
  p.Hkv = static_cast<int>(BH);
  p.qr = qr;
  p.qb = qb;
  p.qr_rows = static_cast<int>(rows);
  p.t_m = m; p.t_l = l; p.t_acc = acc; p.t_z = z;
  p.n_tiers = 1;
  StrataTierArg& ta = p.tiers[0];
  ta.kc = kc; ta.ks = ks; ta.vt = vt; ta.vsl = vsl;
  ta.n_t = n; ta.cap_t = cap; ta.n_split = static_cast<int>(n_split); ta.s_base = 0; ta.bits = bits;
  p.S_all = static_cast<int>(n_split);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int bh_pad = (p.BH + 7) / 8 * 8;
  const dim3 grid(static_cast<unsigned>(n_split) * bh_pad);
  // the split kernel holds at most 8 query rows per KV head: rows go in launches of 8
  for (int64_t r0 = 0; r0 < rows; r0 += 8) {
    p.qr_r0 = static_cast<int>(r0);
    p.R_real = static_cast<int>(std::min<int64_t>(8, rows - r0));
    const int R = strata_pow2(p.R_real);
    const size_t smem = std::max<size_t>((R * kSD + 2 * R) * sizeof(float),
                                         (kSWaves * R * kSD + kSWaves * 2 * R) * sizeof(float));
    switch (R) {
      case 1: hipLaunchKernelGGL((strata_split_all<1, KVQ_F32, 3>), grid, dim3(kSThreads), smem, s, p); break;
      case 2: hipLaunchKernelGGL((strata_split_all<2, KVQ_F32, 3>), grid, dim3(kSThreads), smem, s, p); break;
      case 4: hipLaunchKernelGGL((strata_split_all<4, KVQ_F32, 3>), grid, dim3(kSThreads), smem, s, p); break;
      default: hipLaunchKernelGGL((strata_split_all<8, KVQ_F32, 3>), grid, dim3(kSThreads), smem, s, p); break;
    }
    KVQ_LAUNCH_CHECK("kvq_strata_tier_partials");
  }
  return KVQ_OK;
}

extern "C" int64_t kvq_strata_distortion_workspace(int64_t Hkv, int64_t n, int nbits) {
  if (Hkv <= 0 || n <= 0 || nbits < 1 || nbits > kSMaxBits) return -1;
  return 4 * (2 * Hkv * kSD * kSD + 2 * Hkv * n * nbits);
}

extern "C" int kvq_strata_distortion(const float* yk, const float* yv, int64_t Hkv, int64_t n, int64_t d,
                                     const float* S, const float* Mbar, const float* signs, const float* A,
                                     const float* W, const float* DD, int nbits, const int* bits, const float* steps,
                                     float* D, float* workspace, int64_t workspace_bytes, void* stream) {
  KVQ_REQUIRE(d == kSD, "kvq_strata_distortion: head_dim must be 128");
  KVQ_REQUIRE(Hkv > 0 && n > 0 && Hkv < 65536 && Hkv * n < (1LL << 31), "kvq_strata_distortion: bad sizes");
  KVQ_REQUIRE(nbits >= 1 && nbits <= kSMaxBits && bits && steps, "kvq_strata_distortion: 1 to %d widths", kSMaxBits);
  KVQ_REQUIRE(yk && yv && S && Mbar && signs && A && W && DD && D && workspace, "kvq_strata_distortion: null pointer");
  KVQ_REQUIRE(workspace_bytes >= kvq_strata_distortion_workspace(Hkv, n, nbits),
              "kvq_strata_distortion: workspace too small");
  ErrWidths w{};
  w.n = nbits;
  for (int b = 0; b < nbits; ++b) {
    KVQ_REQUIRE(bits[b] == 2 || bits[b] == 4 || bits[b] == 8, "kvq_strata_distortion: widths must be 2, 4 or 8");
    KVQ_REQUIRE(steps[b] > 0.0f, "kvq_strata_distortion: steps must be positive");
    w.bits[b] = bits[b];
    w.step[b] = steps[b];
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* mk = workspace;
  float* mv = mk + Hkv * kSD * kSD;
  float* ek = mv + Hkv * kSD * kSD;
  float* ev = ek + Hkv * n * nbits;
  hipLaunchKernelGGL(strata_metric_kernel, dim3(static_cast<unsigned>(Hkv)), dim3(256), 0, st, S, signs, mk);
  hipLaunchKernelGGL(strata_metric_kernel, dim3(static_cast<unsigned>(Hkv)), dim3(256), 0, st, Mbar, signs, mv);
  const dim3 eg(static_cast<unsigned>((n + kSErrTok - 1) / kSErrTok), static_cast<unsigned>(Hkv));
  hipLaunchKernelGGL(strata_err_mfma, eg, dim3(256), 0, st, yk, n, mk, w, ek);
  hipLaunchKernelGGL(strata_err_mfma, eg, dim3(256), 0, st, yv, n, mv, w, ev);
  const int64_t total = Hkv * n;
  hipLaunchKernelGGL(strata_dtable_kernel, dim3(static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 4096))),
                     dim3(256), 0, st, ek, ev, A, W, DD, nbits, total, D);
  KVQ_LAUNCH_CHECK("kvq_strata_distortion");
  return KVQ_OK;
}
