// KIVI group quantisation, MSB-first packing and the value-tile decode layout (gfx950).
//
// kivi_quant semantics follow STRATA_KV.py:826-856 bit for bit:
//   lo    = fp16(clamp(min, +-65504))                           (as_stored, 539-542)
//   scale = max(fp16(clamp((max - lo) / qmax)), 2^-24)          (IEEE fp32 subtract and divide)
//   code  = clamp(rint((x - lo) / scale), 0, qmax)               (round half to even)
//   xhat  = code * scale + lo                                   (two roundings, never fused)
// All arithmetic that feeds a code or a metadata value uses the explicitly rounded intrinsics so
// that no multiply-add contraction can change a bit.
#include <algorithm>

#include "common.hpp"
#include "mfma_common.hpp"

// Build-time switch: blocks of the vectorised quantisers (grid-stride loops over their items);
// 0 = one block per item.
#ifndef KVQ_QUANT_GRID
#define KVQ_QUANT_GRID 0
#endif

namespace kvq {
namespace {

constexpr float kF16Max = 65504.0f;
constexpr float kMinScale = 5.9604644775390625e-08f;  // 2^-24, the smallest fp16 subnormal

__device__ __forceinline__ float as_stored(float x) {
  x = fminf(fmaxf(x, -kF16Max), kF16Max);
  return f16_to_f32(f32_to_f16(x));
}

__device__ __forceinline__ int quant_code(float x, float lo, float sc, int qmax) {
  float t = rintf(__fdiv_rn(__fsub_rn(x, lo), sc));
  t = fminf(fmaxf(t, 0.0f), static_cast<float>(qmax));
  return static_cast<int>(t);
}

// quant_code with the division replaced by a multiply with r = RN(1 / sc), exact by a bound:
// |RN(d r) - RN(d / sc)| <= 1.5 * 2^-23 * |d / sc| <= 5.4e-5 for quotients up to 300 (codes are at
// most 255 and d / sc exceeds qmax by at most a rounding of sc), so when RN(d r) is more than
// 1e-4 from a half-integer both round to the same integer; otherwise the IEEE quotient is taken.
// The IEEE division runs only in wavefronts where some lane needs it (a wave-uniform branch).
__device__ __forceinline__ int quant_code_r(float x, float lo, float sc, float r, int qmax) {
  const float d = __fsub_rn(x, lo);
  float t = rintf(__fmul_rn(d, r));
  const bool near = fabsf(__fmul_rn(d, r) - t) > 0.4999f;
  if (__builtin_expect(__any(near), 0)) {
    if (near) t = rintf(__fdiv_rn(d, sc));
  }
  t = fminf(fmaxf(t, 0.0f), static_cast<float>(qmax));
  return static_cast<int>(t);
}

__device__ __forceinline__ float dequant(int code, float lo, float sc) {
  return __fadd_rn(__fmul_rn(static_cast<float>(code), sc), lo);
}

// Combine the codes of `per` consecutive lanes (8/bits of them) into one MSB-first byte, returned
// in the first lane of the run.  All lanes of the wavefront must call it.
__device__ __forceinline__ uint32_t pack_lanes(int code, int bits) {
  uint32_t v = static_cast<uint32_t>(code);
  const int per = 8 / bits;
  uint32_t byte = v << (8 - bits);
  for (int k = 1; k < per; ++k) {
    uint32_t o = static_cast<uint32_t>(__shfl_down(static_cast<int>(v), k, 64));
    byte |= o << (8 - bits * (k + 1));
  }
  return byte & 0xffu;
}

// Keys: one block per (group, b*h); one thread per channel (blockDim.x == d).
template <int DT>
__global__ void kivi_quant_keys(const void* __restrict__ x, int H, int64_t sb, int64_t sh,
                                int64_t st, int n_sink, int n, int d, int bits, int group,
                                uint8_t* __restrict__ codes, int64_t codes_bh,
                                uint8_t* __restrict__ packed, int64_t packed_bh,
                                uint16_t* __restrict__ lo_out, uint16_t* __restrict__ sc_out,
                                int64_t meta_bh, float* __restrict__ xhat, int T) {
  const int gi = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / H, h = bh % H;
  const int c = threadIdx.x;
  const int qmax = (1 << bits) - 1;
  const int t0 = gi * group;
  const int t1 = min(t0 + group, n);
  const int64_t base = static_cast<int64_t>(b) * sb + static_cast<int64_t>(h) * sh + c;
  float mn = INFINITY, mx = -INFINITY;
  for (int t = t0; t < t1; ++t) {
    float v = load_as_f32<DT>(x, base + static_cast<int64_t>(n_sink + t) * st);
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
  const float lo = as_stored(mn);
  const float sc = fmaxf(as_stored(__fdiv_rn(__fsub_rn(mx, lo), static_cast<float>(qmax))), kMinScale);
  const int64_t mo = static_cast<int64_t>(bh) * meta_bh + static_cast<int64_t>(gi) * d + c;
  lo_out[mo] = f32_to_f16(lo);
  sc_out[mo] = f32_to_f16(sc);
  const int per = 8 / bits;
  for (int t = t0; t < t0 + group; ++t) {       // every lane runs the full loop (shuffles inside)
    const bool valid = t < t1;
    float v = valid ? load_as_f32<DT>(x, base + static_cast<int64_t>(n_sink + t) * st) : 0.0f;
    int code = valid ? quant_code(v, lo, sc, qmax) : 0;
    if (packed != nullptr) {
      uint32_t byte = pack_lanes(code, bits);
      if (valid && (c % per) == 0)
        packed[static_cast<int64_t>(bh) * packed_bh + static_cast<int64_t>(t) * (d * bits / 8) +
               c / per] = static_cast<uint8_t>(byte);
    }
    if (!valid) continue;
    if (codes != nullptr)
      codes[static_cast<int64_t>(bh) * codes_bh + static_cast<int64_t>(t) * d + c] =
          static_cast<uint8_t>(code);
    if (xhat != nullptr)
      xhat[(static_cast<int64_t>(bh) * T + n_sink + t) * d + c] = dequant(code, lo, sc);
  }
}

// Values: one thread per (token, 8-channel slab); lanes of one channel group reduce with
// butterfly shuffles.  blockDim.x == 256, d % 8 == 0, (width / 8) a power of two <= 64.
template <int DT>
__global__ void kivi_quant_values(const void* __restrict__ x, int H, int64_t sb, int64_t sh,
                                  int64_t st, int n_sink, int n, int d, int bits, int width,
                                  uint8_t* __restrict__ codes, int64_t codes_bh,
                                  uint8_t* __restrict__ packed, int64_t packed_bh,
                                  uint16_t* __restrict__ lo_out, uint16_t* __restrict__ sc_out,
                                  int64_t meta_bh, float* __restrict__ xhat, int T) {
  const int slabs = d / 8;
  const int tok_per_block = blockDim.x / slabs;
  const int bh = blockIdx.y;
  const int b = bh / H, h = bh % H;
  const int t = blockIdx.x * tok_per_block + threadIdx.x / slabs;
  const int s = threadIdx.x % slabs;
  const int lanes = width / 8;
  const bool valid = t < n && static_cast<int>(threadIdx.x) < tok_per_block * slabs;
  const int qmax = (1 << bits) - 1;
  float v[8];
  float mn = INFINITY, mx = -INFINITY;
  const int64_t row = static_cast<int64_t>(b) * sb + static_cast<int64_t>(h) * sh +
                      static_cast<int64_t>(n_sink + (valid ? t : 0)) * st + s * 8;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    v[k] = valid ? load_as_f32<DT>(x, row + k) : 0.0f;
    mn = fminf(mn, v[k]);
    mx = fmaxf(mx, v[k]);
  }
  for (int off = 1; off < lanes; off <<= 1) {
    mn = fminf(mn, __shfl_xor(mn, off, 64));
    mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  }
  if (!valid) return;
  const float lo = as_stored(mn);
  const float sc = fmaxf(as_stored(__fdiv_rn(__fsub_rn(mx, lo), static_cast<float>(qmax))), kMinScale);
  const int gc = (s * 8) / width;
  if ((s * 8) % width == 0) {
    const int64_t mo = static_cast<int64_t>(bh) * meta_bh + static_cast<int64_t>(t) * (d / width) + gc;
    lo_out[mo] = f32_to_f16(lo);
    sc_out[mo] = f32_to_f16(sc);
  }
  int cd[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) cd[k] = quant_code(v[k], lo, sc, qmax);
  if (codes != nullptr) {
    uint8_t* dst = codes + static_cast<int64_t>(bh) * codes_bh + static_cast<int64_t>(t) * d + s * 8;
#pragma unroll
    for (int k = 0; k < 8; ++k) dst[k] = static_cast<uint8_t>(cd[k]);
  }
  if (packed != nullptr) {
    uint8_t* dst = packed + static_cast<int64_t>(bh) * packed_bh +
                   static_cast<int64_t>(t) * (d * bits / 8) + s * bits;   // 8 codes = `bits` bytes
    const int per = 8 / bits;
    for (int byte = 0; byte < bits; ++byte) {
      uint32_t acc = 0;
      for (int k = 0; k < per; ++k) acc |= static_cast<uint32_t>(cd[byte * per + k]) << (8 - bits * (k + 1));
      dst[byte] = static_cast<uint8_t>(acc);
    }
  }
  if (xhat != nullptr) {
    float* dst = xhat + (static_cast<int64_t>(bh) * T + n_sink + t) * d + s * 8;
#pragma unroll
    for (int k = 0; k < 8; ++k) dst[k] = dequant(cd[k], lo, sc);
  }
}

// ---------------------------------------------------------------------------------------------
// Vectorised variants for d == 128 and 16-byte aligned rows (the common case): the same
// arithmetic as the kernels above (as_stored, quant_code, dequant), so the results are identical
// bit for bit; only the memory access changes.  A thread owns 8 consecutive channels ("slab")
// of a row: one 16-byte load per row (two for fp32), one word store per row for the packed codes.

template <int DT>
__device__ __forceinline__ void load_slab(const void* base, int64_t i, float (&v)[8]) {
  if constexpr (DT == KVQ_F32) {
    const float4* p4 = reinterpret_cast<const float4*>(static_cast<const float*>(base) + i);
    const float4 a = p4[0], c = p4[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = c.x; v[5] = c.y; v[6] = c.z; v[7] = c.w;
  } else {
    const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + i);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint16_t a = static_cast<uint16_t>(ws[k] & 0xffffu), c = static_cast<uint16_t>(ws[k] >> 16);
      v[2 * k] = DT == KVQ_F16 ? f16_to_f32(a) : bf16_to_f32(a);
      v[2 * k + 1] = DT == KVQ_F16 ? f16_to_f32(c) : bf16_to_f32(c);
    }
  }
}

// codes of one slab: MSB-first packed bytes (`bits` of them), raw codes, dequantised values
__device__ __forceinline__ void store_slab(const int (&cd)[8], int bits, uint8_t* packed_dst, uint8_t* codes_dst,
                                           float* xhat_dst, const float (&lo)[8], const float (&sc)[8]) {
  if (packed_dst != nullptr) {
    if (bits == 4) {
      uint32_t w = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) w |= static_cast<uint32_t>((cd[2 * k] << 4) | cd[2 * k + 1]) << (8 * k);
      *reinterpret_cast<uint32_t*>(packed_dst) = w;
    } else if (bits == 2) {
      uint32_t w = 0;
#pragma unroll
      for (int k = 0; k < 2; ++k)
        w |= static_cast<uint32_t>((cd[4 * k] << 6) | (cd[4 * k + 1] << 4) | (cd[4 * k + 2] << 2) | cd[4 * k + 3]) << (8 * k);
      *reinterpret_cast<uint16_t*>(packed_dst) = static_cast<uint16_t>(w);
    } else {
      uint2 w;
      w.x = cd[0] | (cd[1] << 8) | (cd[2] << 16) | (static_cast<uint32_t>(cd[3]) << 24);
      w.y = cd[4] | (cd[5] << 8) | (cd[6] << 16) | (static_cast<uint32_t>(cd[7]) << 24);
      *reinterpret_cast<uint2*>(packed_dst) = w;
    }
  }
  if (codes_dst != nullptr) {
    uint2 w;
    w.x = cd[0] | (cd[1] << 8) | (cd[2] << 16) | (static_cast<uint32_t>(cd[3]) << 24);
    w.y = cd[4] | (cd[5] << 8) | (cd[6] << 16) | (static_cast<uint32_t>(cd[7]) << 24);
    *reinterpret_cast<uint2*>(codes_dst) = w;
  }
  if (xhat_dst != nullptr) {
    float4 a, c;
    a.x = dequant(cd[0], lo[0], sc[0]); a.y = dequant(cd[1], lo[1], sc[1]);
    a.z = dequant(cd[2], lo[2], sc[2]); a.w = dequant(cd[3], lo[3], sc[3]);
    c.x = dequant(cd[4], lo[4], sc[4]); c.y = dequant(cd[5], lo[5], sc[5]);
    c.z = dequant(cd[6], lo[6], sc[6]); c.w = dequant(cd[7], lo[7], sc[7]);
    reinterpret_cast<float4*>(xhat_dst)[0] = a;
    reinterpret_cast<float4*>(xhat_dst)[1] = c;
  }
}

// Raw 16-byte slab (8 elements; fp32 needs two) and its conversion: loads are issued one work
// item ahead and converted when the item is processed.
template <int DT>
struct Slab {
  uint4 a, b;
};
template <int DT>
__device__ __forceinline__ void slab_load(const void* base, int64_t i, Slab<DT>& r) {
  if constexpr (DT == KVQ_F32) {
    const uint4* p = reinterpret_cast<const uint4*>(static_cast<const float*>(base) + i);
    r.a = p[0];
    r.b = p[1];
  } else {
    r.a = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + i);
  }
}
template <int DT>
__device__ __forceinline__ void slab_values(const Slab<DT>& r, float (&v)[8]) {
  if constexpr (DT == KVQ_F32) {
    v[0] = __uint_as_float(r.a.x); v[1] = __uint_as_float(r.a.y); v[2] = __uint_as_float(r.a.z); v[3] = __uint_as_float(r.a.w);
    v[4] = __uint_as_float(r.b.x); v[5] = __uint_as_float(r.b.y); v[6] = __uint_as_float(r.b.z); v[7] = __uint_as_float(r.b.w);
  } else {
    const uint32_t ws[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint16_t a = static_cast<uint16_t>(ws[k] & 0xffffu), c = static_cast<uint16_t>(ws[k] >> 16);
      v[2 * k] = DT == KVQ_F16 ? f16_to_f32(a) : bf16_to_f32(a);
      v[2 * k + 1] = DT == KVQ_F16 ? f16_to_f32(c) : bf16_to_f32(c);
    }
  }
}

// Keys, d == 128: a 256-thread block walks the (group, b*h) items with a grid stride, loading the
// next item while it reduces and codes the current one.  Thread t owns slab s = t % 16 of rows
// t / 16 + 16 j (j < RPT, RPT = ceil(group / 16)); per-channel min / max reduce over the rows of
// the thread, then over the 16 row lanes (shuffles inside a wavefront, LDS across the four).
template <int DT, int RPT>
__global__ __launch_bounds__(256) void kivi_quant_keys_v(const void* __restrict__ x, int H, int64_t sb, int64_t sh,
                                                          int64_t st, int n_sink, int n, int bits, int group,
                                                          uint8_t* __restrict__ codes, int64_t codes_bh,
                                                          uint8_t* __restrict__ packed, int64_t packed_bh,
                                                          uint16_t* __restrict__ lo_out, uint16_t* __restrict__ sc_out,
                                                          int64_t meta_bh, float* __restrict__ xhat, int T,
                                                          int n_g, int64_t n_items) {
  constexpr int D = 128;
  __shared__ float red_mn[4][D], red_mx[4][D];
  __shared__ float meta_l[D], meta_s[D], meta_r[D];
  const int s = threadIdx.x & 15, rl = threadIdx.x >> 4, wave = threadIdx.x >> 6;
  const int qmax = (1 << bits) - 1;
  Slab<DT> cur[RPT], nxt[RPT];
  auto row_ok = [&](int64_t item, int j) -> bool {
    const int gi = static_cast<int>(item % n_g);
    return rl + 16 * j < group && gi * group + rl + 16 * j < n;
  };
  auto issue = [&](int64_t item, Slab<DT> (&r)[RPT]) {
    if (item >= n_items) return;
    const int gi = static_cast<int>(item % n_g), bh = static_cast<int>(item / n_g);
    const int b = bh / H, h = bh % H;
    const int64_t base = static_cast<int64_t>(b) * sb + static_cast<int64_t>(h) * sh + s * 8;
#pragma unroll
    for (int j = 0; j < RPT; ++j)
      if (row_ok(item, j)) slab_load<DT>(x, base + static_cast<int64_t>(n_sink + gi * group + rl + 16 * j) * st, r[j]);
  };
  int64_t item = blockIdx.x;
  issue(item, cur);
  for (; item < n_items; item += gridDim.x) {
    issue(item + gridDim.x, nxt);
    const int gi = static_cast<int>(item % n_g), bh = static_cast<int>(item / n_g);
    const int t0 = gi * group;
    float v[RPT][8];
    float mn[8], mx[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      mn[k] = INFINITY;
      mx[k] = -INFINITY;
    }
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      if (row_ok(item, j)) {
        slab_values<DT>(cur[j], v[j]);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          mn[k] = fminf(mn[k], v[j][k]);
          mx[k] = fmaxf(mx[k], v[j][k]);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
#pragma unroll
      for (int o = 16; o < 64; o <<= 1) {
        mn[k] = fminf(mn[k], __shfl_xor(mn[k], o, 64));
        mx[k] = fmaxf(mx[k], __shfl_xor(mx[k], o, 64));
      }
    }
    __syncthreads();                              // the previous item's reads of red_* / meta are done
    if ((threadIdx.x & 63) < 16) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        red_mn[wave][s * 8 + k] = mn[k];
        red_mx[wave][s * 8 + k] = mx[k];
      }
    }
    __syncthreads();
    if (threadIdx.x < D) {                        // one thread per channel: lo, scale, 1 / scale
      const int c = threadIdx.x;
      const float a = fminf(fminf(red_mn[0][c], red_mn[1][c]), fminf(red_mn[2][c], red_mn[3][c]));
      const float z = fmaxf(fmaxf(red_mx[0][c], red_mx[1][c]), fmaxf(red_mx[2][c], red_mx[3][c]));
      const float l = as_stored(a);
      const float q = fmaxf(as_stored(__fdiv_rn(__fsub_rn(z, l), static_cast<float>(qmax))), kMinScale);
      meta_l[c] = l;
      meta_s[c] = q;
      meta_r[c] = __fdiv_rn(1.0f, q);
    }
    __syncthreads();
    float lo[8], sc[8], rc[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      lo[k] = meta_l[s * 8 + k];
      sc[k] = meta_s[s * 8 + k];
      rc[k] = meta_r[s * 8 + k];
    }
    if (rl == 0) {
      const int64_t mo = static_cast<int64_t>(bh) * meta_bh + static_cast<int64_t>(gi) * D + s * 8;
      uint4 wl, ws_;
      wl.x = f32_to_f16(lo[0]) | (static_cast<uint32_t>(f32_to_f16(lo[1])) << 16);
      wl.y = f32_to_f16(lo[2]) | (static_cast<uint32_t>(f32_to_f16(lo[3])) << 16);
      wl.z = f32_to_f16(lo[4]) | (static_cast<uint32_t>(f32_to_f16(lo[5])) << 16);
      wl.w = f32_to_f16(lo[6]) | (static_cast<uint32_t>(f32_to_f16(lo[7])) << 16);
      ws_.x = f32_to_f16(sc[0]) | (static_cast<uint32_t>(f32_to_f16(sc[1])) << 16);
      ws_.y = f32_to_f16(sc[2]) | (static_cast<uint32_t>(f32_to_f16(sc[3])) << 16);
      ws_.z = f32_to_f16(sc[4]) | (static_cast<uint32_t>(f32_to_f16(sc[5])) << 16);
      ws_.w = f32_to_f16(sc[6]) | (static_cast<uint32_t>(f32_to_f16(sc[7])) << 16);
      *reinterpret_cast<uint4*>(lo_out + mo) = wl;
      *reinterpret_cast<uint4*>(sc_out + mo) = ws_;
    }
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      if (!row_ok(item, j)) continue;
      const int t = t0 + rl + 16 * j;
      int cd[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) cd[k] = quant_code_r(v[j][k], lo[k], sc[k], rc[k], qmax);
      store_slab(cd, bits,
                 packed ? packed + static_cast<int64_t>(bh) * packed_bh + static_cast<int64_t>(t) * (D * bits / 8) + s * bits
                        : nullptr,
                 codes ? codes + static_cast<int64_t>(bh) * codes_bh + static_cast<int64_t>(t) * D + s * 8 : nullptr,
                 xhat ? xhat + (static_cast<int64_t>(bh) * T + n_sink + t) * D + s * 8 : nullptr, lo, sc);
    }
#pragma unroll
    for (int j = 0; j < RPT; ++j) cur[j] = nxt[j];
  }
}

// Values, d == 128: a 256-thread block walks items of 16 x VR rows with a grid stride (thread:
// slab s = t % 16 of rows 16 r + t / 16, r < VR), loading the next item while coding the current
// one; a channel group of `width` channels is width / 8 consecutive lanes (butterfly shuffles).
template <int DT, int VR>
__global__ __launch_bounds__(256) void kivi_quant_values_v(const void* __restrict__ x, int H, int64_t sb, int64_t sh,
                                                            int64_t st, int n_sink, int n, int bits, int width,
                                                            uint8_t* __restrict__ codes, int64_t codes_bh,
                                                            uint8_t* __restrict__ packed, int64_t packed_bh,
                                                            uint16_t* __restrict__ lo_out, uint16_t* __restrict__ sc_out,
                                                            int64_t meta_bh, float* __restrict__ xhat, int T,
                                                            int n_rb, int64_t n_items) {
  constexpr int D = 128;
  const int s = threadIdx.x & 15, rl = threadIdx.x >> 4;
  const int lanes = width / 8;
  const int qmax = (1 << bits) - 1;
  Slab<DT> cur[VR], nxt[VR];
  auto issue = [&](int64_t item, Slab<DT> (&r)[VR]) {
    if (item >= n_items) return;
    const int rb = static_cast<int>(item % n_rb), bh = static_cast<int>(item / n_rb);
    const int b = bh / H, h = bh % H;
    const int64_t base = static_cast<int64_t>(b) * sb + static_cast<int64_t>(h) * sh + s * 8;
#pragma unroll
    for (int j = 0; j < VR; ++j) {
      const int t = rb * 16 * VR + 16 * j + rl;
      if (t < n) slab_load<DT>(x, base + static_cast<int64_t>(n_sink + t) * st, r[j]);
    }
  };
  int64_t item = blockIdx.x;
  issue(item, cur);
  for (; item < n_items; item += gridDim.x) {
    issue(item + gridDim.x, nxt);
    const int rb = static_cast<int>(item % n_rb), bh = static_cast<int>(item / n_rb);
#pragma unroll
    for (int j = 0; j < VR; ++j) {
      const int t = rb * 16 * VR + 16 * j + rl;
      const bool valid = t < n;
      float v[8];
      float mn = INFINITY, mx = -INFINITY;
      if (valid) {
        slab_values<DT>(cur[j], v);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          mn = fminf(mn, v[k]);
          mx = fmaxf(mx, v[k]);
        }
      }
      for (int off = 1; off < lanes; off <<= 1) {
        mn = fminf(mn, __shfl_xor(mn, off, 64));
        mx = fmaxf(mx, __shfl_xor(mx, off, 64));
      }
      if (!valid) continue;
      const float l1 = as_stored(mn);
      const float s1 = fmaxf(as_stored(__fdiv_rn(__fsub_rn(mx, l1), static_cast<float>(qmax))), kMinScale);
      if ((s * 8) % width == 0) {
        const int64_t mo = static_cast<int64_t>(bh) * meta_bh + static_cast<int64_t>(t) * (D / width) + (s * 8) / width;
        lo_out[mo] = f32_to_f16(l1);
        sc_out[mo] = f32_to_f16(s1);
      }
      float lo[8], sc[8];
      int cd[8];
      const float r1 = __fdiv_rn(1.0f, s1);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        lo[k] = l1;
        sc[k] = s1;
        cd[k] = quant_code_r(v[k], l1, s1, r1, qmax);
      }
      store_slab(cd, bits,
                 packed ? packed + static_cast<int64_t>(bh) * packed_bh + static_cast<int64_t>(t) * (D * bits / 8) + s * bits
                        : nullptr,
                 codes ? codes + static_cast<int64_t>(bh) * codes_bh + static_cast<int64_t>(t) * D + s * 8 : nullptr,
                 xhat ? xhat + (static_cast<int64_t>(bh) * T + n_sink + t) * D + s * 8 : nullptr, lo, sc);
    }
#pragma unroll
    for (int j = 0; j < VR; ++j) cur[j] = nxt[j];
  }
}

// ---------------------------------------------------------------------------------------------
// Packed-only 4-bit variants (16-bit input, d == 128, no unpacked codes or xhat: the prefill
// path of the decode cache).  One wavefront per item, no barriers: lane (s = lane % 16, rq =
// lane / 16) owns the 8-channel slab s of rows rq + 4 j.  Every row of the item is loaded at
// once through a buffer resource that ends at the item's last valid row (rows past it read
// zero and are masked), so the load path has no branches.  The arithmetic is that of
// quant_code_r; the check for quotients near a half-integer is taken once per row and the IEEE
// division redone only where a lane needs it.  Results are bit-identical to the kernels above.

template <int DT>
__device__ __forceinline__ void cvt_slab(const u32x4 w, float (&v)[8]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint16_t a = static_cast<uint16_t>(w[k] & 0xffffu), c = static_cast<uint16_t>(w[k] >> 16);
    v[2 * k] = DT == KVQ_F16 ? f16_to_f32(a) : bf16_to_f32(a);
    v[2 * k + 1] = DT == KVQ_F16 ? f16_to_f32(c) : bf16_to_f32(c);
  }
}

// 4-bit codes of 8 values: t = rint(RN(RN(x - lo) * r)) with r = v_rcp_f32(sc), and where some
// lane's product is within 1e-4 of a half-integer, rint(RN(RN(x - lo) / sc)).  Exact: r is within
// 1 ulp of 1 / sc (the instruction's documented accuracy; sc is a normal fp16 value >= 2^-24), so
// |RN(d r) - RN(d / sc)| <= (2^-23 + 2^-24 + 2^-24) |d / sc| = 2^-22 |d / sc|, under 1e-4 while
// |d / sc| <= 400, so a product more than 1e-4 from a half-integer rounds to the same integer as
// the IEEE quotient; larger quotients (inputs beyond the fp16 range that lo and sc clamp to) give
// the same clamped code 0 or 15 either way.
__device__ __forceinline__ uint32_t code_word4(const float (&v)[8], const float (&lo)[8], const float (&sc)[8],
                                               const float (&rc)[8]) {
  float t[8];
  bool near = false;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float p = __fmul_rn(__fsub_rn(v[k], lo[k]), rc[k]);
    t[k] = rintf(p);
    near |= fabsf(p - t[k]) > 0.4999f;
  }
  if (__builtin_expect(__any(near), 0)) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float dd = __fsub_rn(v[k], lo[k]);
      if (fabsf(__fmul_rn(dd, rc[k]) - t[k]) > 0.4999f) t[k] = rintf(__fdiv_rn(dd, sc[k]));
    }
  }
  uint32_t w = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t c = static_cast<uint32_t>(fminf(fmaxf(t[k], 0.0f), 15.0f));
    w |= c << ((k & 1) ? 8 * (k / 2) : 8 * (k / 2) + 4);       // MSB-first: even channel high nibble
  }
  return w;
}

// Keys: item = (group gi, b*h), group <= 4 RPL rows; per-channel min / max over the rows of the
// lane, then over the four row lanes (permlane swaps).
template <int DT, int RPL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void kivi_quant_keys_p4(
    const void* __restrict__ x, int H, int64_t sb, int64_t sh, int64_t st, int n_sink, int n, int group,
    uint8_t* __restrict__ packed, int64_t packed_bh, uint16_t* __restrict__ lo_out, uint16_t* __restrict__ sc_out,
    int64_t meta_bh, int n_g, int64_t n_items) {
  constexpr int D = 128;
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (item >= n_items) return;
  const int s = lane & 15, rq = lane >> 4;
  const int gi = static_cast<int>(item % n_g), bh = static_cast<int>(item / n_g);
  const int b = bh / H, h = bh % H;
  const int t0 = gi * group;
  const int rv = min(group, n - t0);                          // valid rows of the item (>= 1)
  const uint16_t* src = static_cast<const uint16_t*>(x) + static_cast<int64_t>(b) * sb + static_cast<int64_t>(h) * sh +
                        static_cast<int64_t>(n_sink + t0) * st;
  const uint32_t rstride = static_cast<uint32_t>(st * 2);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(src, static_cast<uint32_t>(rv) * rstride);
  u32x4 raw[RPL];                                   // rows read once: non-temporal loads
#pragma unroll
  for (int j = 0; j < RPL; ++j) raw[j] = __builtin_amdgcn_raw_buffer_load_b128(rs, (rq + 4 * j) * rstride + s * 16, 0, 2);
  float mn[8], mx[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    mn[k] = INFINITY;
    mx[k] = -INFINITY;
  }
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    const bool ok = rq + 4 * j < rv;
    float v[8];
    cvt_slab<DT>(raw[j], v);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      mn[k] = fminf(mn[k], ok ? v[k] : INFINITY);
      mx[k] = fmaxf(mx[k], ok ? v[k] : -INFINITY);
    }
  }
  // the rows are converted again when coded: only the raw words stay live across the reduction
#pragma unroll
  for (int j = 0; j < RPL; ++j) asm volatile("" : "+v"(raw[j]));
  float lo[8], sc[8], rc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float a = xmin32(xmin16(mn[k])), z = xmax32(xmax16(mx[k]));
    const float l = as_stored(a);
    const float q = fmaxf(as_stored(__fdiv_rn(__fsub_rn(z, l), 15.0f)), kMinScale);
    lo[k] = l;
    sc[k] = q;
    rc[k] = __builtin_amdgcn_rcpf(q);
  }
  if (rq == 0) {
    const int64_t mo = static_cast<int64_t>(bh) * meta_bh + static_cast<int64_t>(gi) * D + s * 8;
    u32x4 wl, ws;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      wl[k] = f32_to_f16(lo[2 * k]) | (static_cast<uint32_t>(f32_to_f16(lo[2 * k + 1])) << 16);
      ws[k] = f32_to_f16(sc[2 * k]) | (static_cast<uint32_t>(f32_to_f16(sc[2 * k + 1])) << 16);
    }
    *reinterpret_cast<u32x4*>(lo_out + mo) = wl;
    *reinterpret_cast<u32x4*>(sc_out + mo) = ws;
  }
  uint32_t* dst = reinterpret_cast<uint32_t*>(packed + static_cast<int64_t>(bh) * packed_bh + static_cast<int64_t>(t0) * (D / 2)) + s;
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    float v[8];
    cvt_slab<DT>(raw[j], v);
    const uint32_t w = code_word4(v, lo, sc, rc);
    if (rq + 4 * j < rv) __builtin_nontemporal_store(w, &dst[(rq + 4 * j) * (D / 8)]);   // written once
  }
}

// min / max over runs of L lanes (L = 1, 2, 4, 8, 16) inside a row of 16, every lane of a run
// receiving the result (quad swaps, then the half-row and row mirrors)
template <int L>
__device__ __forceinline__ void run_minmax(float& mn, float& mx) {
  if constexpr (L >= 2) { mn = fminf(mn, dpp<kQuadSwap1>(mn)); mx = fmaxf(mx, dpp<kQuadSwap1>(mx)); }
  if constexpr (L >= 4) { mn = fminf(mn, dpp<kQuadSwap2>(mn)); mx = fmaxf(mx, dpp<kQuadSwap2>(mx)); }
  if constexpr (L >= 8) { mn = fminf(mn, dpp<0x141>(mn)); mx = fmaxf(mx, dpp<0x141>(mx)); }    // row_half_mirror
  if constexpr (L >= 16) { mn = fminf(mn, dpp<0x140>(mn)); mx = fmaxf(mx, dpp<0x140>(mx)); }   // row_mirror
}

// Values: item = 64 consecutive rows of one b*h; a channel group of 8 L channels is L lanes.
template <int DT, int L>
__global__ __launch_bounds__(256) void kivi_quant_values_p4(
    const void* __restrict__ x, int H, int64_t sb, int64_t sh, int64_t st, int n_sink, int n,
    uint8_t* __restrict__ packed, int64_t packed_bh, uint16_t* __restrict__ lo_out, uint16_t* __restrict__ sc_out,
    int64_t meta_bh, int n_rb, int64_t n_items) {
  constexpr int D = 128, RPL = 16, NG = D / (8 * L);
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (item >= n_items) return;
  const int s = lane & 15, rq = lane >> 4;
  const int rb = static_cast<int>(item % n_rb), bh = static_cast<int>(item / n_rb);
  const int b = bh / H, h = bh % H;
  const int t0 = rb * 4 * RPL;
  const int rv = min(4 * RPL, n - t0);
  const uint16_t* src = static_cast<const uint16_t*>(x) + static_cast<int64_t>(b) * sb + static_cast<int64_t>(h) * sh +
                        static_cast<int64_t>(n_sink + t0) * st;
  const uint32_t rstride = static_cast<uint32_t>(st * 2);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(src, static_cast<uint32_t>(rv) * rstride);
  u32x4 raw[RPL];                                   // rows read once: non-temporal loads
#pragma unroll
  for (int j = 0; j < RPL; ++j) raw[j] = __builtin_amdgcn_raw_buffer_load_b128(rs, (rq + 4 * j) * rstride + s * 16, 0, 2);
  uint32_t* dst = reinterpret_cast<uint32_t*>(packed + static_cast<int64_t>(bh) * packed_bh + static_cast<int64_t>(t0) * (D / 2)) + s;
  const int64_t mrow = static_cast<int64_t>(bh) * meta_bh + static_cast<int64_t>(t0) * NG + s / L;
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    const int r = rq + 4 * j;
    float v[8];
    cvt_slab<DT>(raw[j], v);
    float mn = INFINITY, mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      mn = fminf(mn, v[k]);
      mx = fmaxf(mx, v[k]);
    }
    run_minmax<L>(mn, mx);
    const float l1 = as_stored(mn);
    const float s1 = fmaxf(as_stored(__fdiv_rn(__fsub_rn(mx, l1), 15.0f)), kMinScale);
    const float r1 = __builtin_amdgcn_rcpf(s1);
    const float lo[8] = {l1, l1, l1, l1, l1, l1, l1, l1}, sc[8] = {s1, s1, s1, s1, s1, s1, s1, s1};
    const float rc[8] = {r1, r1, r1, r1, r1, r1, r1, r1};
    const uint32_t w = code_word4(v, lo, sc, rc);
    if (r < rv) {
      __builtin_nontemporal_store(w, &dst[r * (D / 8)]);                                 // written once
      if (s % L == 0) {
        lo_out[mrow + static_cast<int64_t>(r) * NG] = f32_to_f16(l1);
        sc_out[mrow + static_cast<int64_t>(r) * NG] = f32_to_f16(s1);
      }
    }
  }
}

template <int DT>
__global__ void copy_sinks(const void* __restrict__ x, int H, int64_t sb, int64_t sh, int64_t st,
                           int n_sink, int d, int T, float* __restrict__ xhat) {
  const int bh = blockIdx.y;
  const int b = bh / H, h = bh % H;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<int64_t>(n_sink) * d) return;
  const int t = static_cast<int>(i / d), c = static_cast<int>(i % d);
  xhat[(static_cast<int64_t>(bh) * T + t) * d + c] =
      load_as_f32<DT>(x, static_cast<int64_t>(b) * sb + static_cast<int64_t>(h) * sh +
                             static_cast<int64_t>(t) * st + c);
}

__global__ void pack_codes_kernel(const uint8_t* __restrict__ codes, int64_t count, int bits,
                                  uint8_t* __restrict__ out, int64_t nbytes) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= nbytes) return;
  const int per = 8 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  uint32_t acc = 0;
  for (int k = 0; k < per; ++k) {
    const int64_t j = i * per + k;
    const uint32_t c = j < count ? (static_cast<uint32_t>(codes[j]) & mask) : 0u;
    acc |= c << (8 - bits * (k + 1));
  }
  out[i] = static_cast<uint8_t>(acc);
}

__global__ void unpack_codes_kernel(const uint8_t* __restrict__ packed, int64_t count, int bits,
                                    uint8_t* __restrict__ out) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j >= count) return;
  const int per = 8 / bits;
  const uint32_t byte = packed[j / per];
  const int k = static_cast<int>(j % per);
  out[j] = static_cast<uint8_t>((byte >> (8 - bits * (k + 1))) & ((1u << bits) - 1u));
}

// ---- value tiles --------------------------------------------------------------------------
// A 32-token chunk of 4-bit value codes is 16*d bytes: word (q, lane, b4) with q < d/64,
// lane < 64, b4 < 4 holds channel 16*(4q+b4) + lane%16 for the 8 tokens of "slot" j = 0..7 of
// lane group g = lane/16, token(g, j) = 16*(j/4) + 4g + j%4.  Nibble k (bits 4k..4k+3) of the
// word holds slot kSlotOfNibble[k]; this is the order in which the decode kernel's magic-number
// conversion produces the matrix-core operand (nibbles 0,4 | 1,5 | 2,6 | 3,7 per register).
__device__ __constant__ int kSlotOfNibble[8] = {0, 2, 4, 6, 1, 3, 5, 7};

__device__ __forceinline__ int slot_token(int g, int j) { return 16 * (j >> 2) + 4 * g + (j & 3); }

__device__ __forceinline__ uint32_t row_nibble(const uint8_t* rows_bh, int64_t tok, int ch, int d) {
  const uint8_t byte = rows_bh[tok * (d / 2) + ch / 2];
  return (ch & 1) ? (byte & 0xfu) : (byte >> 4);        // even channel in the high nibble
}

__global__ void v_tile_kernel(const uint8_t* __restrict__ rows, int64_t n, int64_t rows_bh, int d,
                              int64_t cap_t, uint8_t* __restrict__ tiles) {
  const int64_t bh = blockIdx.y;
  const int64_t words_per_chunk = 4 * d;                 // 16*d bytes
  const int64_t w = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (w >= (cap_t / 32) * words_per_chunk) return;
  const int64_t chunk = w / words_per_chunk;
  const int r = static_cast<int>(w % words_per_chunk);
  const int q = r / 256, lane = (r / 4) % 64, b4 = r % 4;
  const int ch = 16 * (4 * q + b4) + lane % 16;
  const int g = lane / 16;
  const uint8_t* src = rows + bh * rows_bh;
  uint32_t word = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int64_t tok = chunk * 32 + slot_token(g, kSlotOfNibble[k]);
    const uint32_t c = tok < n ? row_nibble(src, tok, ch, d) : 0u;
    word |= c << (4 * k);
  }
  reinterpret_cast<uint32_t*>(tiles + bh * (cap_t * d / 2))[w] = word;
}

__global__ void v_untile_kernel(const uint8_t* __restrict__ tiles, int64_t n, int d, int64_t cap_t,
                                uint8_t* __restrict__ rows, int64_t rows_bh) {
  const int64_t bh = blockIdx.y;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;  // output byte
  if (i >= n * (d / 2)) return;
  const int64_t tok = i / (d / 2);
  const int ch0 = static_cast<int>(i % (d / 2)) * 2;
  const int64_t chunk = tok / 32;
  const int u = static_cast<int>(tok % 32);
  const int g = (u % 16) / 4;
  const int j = 4 * (u / 16) + (u % 4);
  int nib = 0;
  for (int k = 0; k < 8; ++k)
    if (kSlotOfNibble[k] == j) nib = k;
  const uint32_t* tw = reinterpret_cast<const uint32_t*>(tiles + bh * (cap_t * d / 2) + chunk * 16 * d);
  uint32_t out = 0;
  for (int e = 0; e < 2; ++e) {
    const int ch = ch0 + e;
    const int blk = ch / 16;
    const int lane = 16 * g + ch % 16;
    const uint32_t word = tw[(blk / 4) * 256 + lane * 4 + (blk % 4)];
    const uint32_t c = (word >> (4 * nib)) & 0xfu;
    out |= e == 0 ? (c << 4) : c;
  }
  rows[bh * rows_bh + i] = static_cast<uint8_t>(out);
}

// vmeta (BH, cap_t/32, ngv, 32 slots, 2): slot p = 8g + j holds token(g, j) of the chunk as the
// fp16 pair (scale, lo); tokens past n hold (0, 0).
__global__ void vmeta_tile_kernel(const uint16_t* __restrict__ lo, const uint16_t* __restrict__ sc,
                                  int64_t n, int64_t ngv, int64_t meta_bh, int64_t cap_t,
                                  uint16_t* __restrict__ vmeta) {
  const int64_t bh = blockIdx.y;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t per_chunk = ngv * 32;
  if (i >= (cap_t / 32) * per_chunk) return;
  const int64_t chunk = i / per_chunk;
  const int64_t gc = (i % per_chunk) / 32;
  const int p = static_cast<int>(i % 32);
  const int64_t tok = chunk * 32 + slot_token(p / 8, p % 8);
  uint16_t s = 0, l = 0;
  if (tok < n) {
    s = sc[bh * meta_bh + tok * ngv + gc];
    l = lo[bh * meta_bh + tok * ngv + gc];
  }
  uint16_t* dst = vmeta + bh * (cap_t / 32) * per_chunk * 2 + i * 2;
  dst[0] = s;
  dst[1] = l;
}

inline dim3 grid1d(int64_t n, int block, int64_t y = 1) {
  return dim3(static_cast<unsigned>((n + block - 1) / block), static_cast<unsigned>(y));
}

}  // namespace
}  // namespace kvq

using namespace kvq;

extern "C" int kvq_kivi_quant(const void* x, int x_dtype, int64_t B, int64_t H, int64_t T,
                              int64_t d, int64_t sb, int64_t sh, int64_t st, int bits, int group,
                              int along_tokens, int n_sink, uint8_t* codes, int64_t codes_bh,
                              uint8_t* packed, int64_t packed_bh, uint16_t* lo, uint16_t* scale,
                              int64_t meta_bh, float* xhat, void* stream) {
  KVQ_REQUIRE(x != nullptr && lo != nullptr && scale != nullptr, "kvq_kivi_quant: null pointer");
  KVQ_REQUIRE(valid_dtype(x_dtype), "kvq_kivi_quant: bad dtype %d", x_dtype);
  KVQ_REQUIRE(bits >= 1 && bits <= 8, "kvq_kivi_quant: bits must be in [1, 8], got %d", bits);
  KVQ_REQUIRE(packed == nullptr || bits == 2 || bits == 4 || bits == 8,
              "kvq_kivi_quant: packed output needs bits in {2, 4, 8}");
  KVQ_REQUIRE(B >= 0 && H >= 0 && T >= 0 && d > 0 && group > 0, "kvq_kivi_quant: bad sizes");
  KVQ_REQUIRE(n_sink >= 0 && n_sink <= T, "kvq_kivi_quant: n_sink out of range");
  KVQ_REQUIRE(B * H < (1LL << 31), "kvq_kivi_quant: too many (b,h) rows");
  const int n = static_cast<int>(T - n_sink);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (B * H == 0) return KVQ_OK;
  if (xhat != nullptr && n_sink > 0) {
    KVQ_DISPATCH_DTYPE(x_dtype, hipLaunchKernelGGL((copy_sinks<DT_>), grid1d(n_sink * d, 256, B * H),
                                                   dim3(256), 0, s, x, (int)H, sb, sh, st, n_sink,
                                                   (int)d, (int)T, xhat));
    KVQ_LAUNCH_CHECK("kvq_kivi_quant(sinks)");
  }
  if (n == 0) return KVQ_OK;
  auto al = [](const void* p, uintptr_t a) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % a == 0; };
  const bool vec = d == 128 && al(x, 16) && sb % 8 == 0 && sh % 8 == 0 && st % 8 == 0 && al(packed, 16) &&
                   packed_bh % 8 == 0 && al(codes, 16) && codes_bh % 8 == 0 && al(xhat, 16) && al(lo, 16) &&
                   al(scale, 16) && meta_bh % 8 == 0;
  // packed-only 4-bit output of 16-bit input: one wavefront per item (the decode cache's prefill)
  const bool p4 = vec && bits == 4 && packed != nullptr && codes == nullptr && xhat == nullptr &&
                  x_dtype != KVQ_F32 && st < (1LL << 25);
  if (p4 && along_tokens && group <= 64) {
    const int n_g = (n + group - 1) / group;
    const int64_t n_items = static_cast<int64_t>(n_g) * B * H;
    KVQ_REQUIRE(n_items < (1LL << 33), "kvq_kivi_quant: too many key groups");
    const dim3 grid(static_cast<unsigned>((n_items + 3) / 4));
#define KVQ_KEYS_P4(RPL_)                                                                                      \
    KVQ_DISPATCH_DTYPE(x_dtype, if constexpr (DT_ != KVQ_F32) hipLaunchKernelGGL((kivi_quant_keys_p4<DT_, RPL_>), grid, \
                       dim3(256), 0, s, x, (int)H, sb, sh, st, n_sink, n, group, packed, packed_bh, lo, scale,      \
                       meta_bh, n_g, n_items))
    if (group <= 16) { KVQ_KEYS_P4(4); }
    else if (group <= 32) { KVQ_KEYS_P4(8); }
    else { KVQ_KEYS_P4(16); }
#undef KVQ_KEYS_P4
    KVQ_LAUNCH_CHECK("kvq_kivi_quant(keys)");
    return KVQ_OK;
  }
  if (p4 && !along_tokens) {
    const int64_t width = (d % group == 0) ? group : d;
    if (width % 8 == 0 && ((width / 8) & (width / 8 - 1)) == 0) {
      const int n_rb = (n + 63) / 64;
      const int64_t n_items = static_cast<int64_t>(n_rb) * B * H;
      KVQ_REQUIRE(n_items < (1LL << 33), "kvq_kivi_quant: too many value rows");
      const dim3 grid(static_cast<unsigned>((n_items + 3) / 4));
#define KVQ_VALUES_P4(L_)                                                                                      \
      KVQ_DISPATCH_DTYPE(x_dtype, if constexpr (DT_ != KVQ_F32) hipLaunchKernelGGL((kivi_quant_values_p4<DT_, L_>), grid, \
                         dim3(256), 0, s, x, (int)H, sb, sh, st, n_sink, n, packed, packed_bh, lo, scale, meta_bh,  \
                         n_rb, n_items))
      switch (width / 8) {
        case 1: KVQ_VALUES_P4(1); break;
        case 2: KVQ_VALUES_P4(2); break;
        case 4: KVQ_VALUES_P4(4); break;
        case 8: KVQ_VALUES_P4(8); break;
        default: KVQ_VALUES_P4(16); break;
      }
#undef KVQ_VALUES_P4
      KVQ_LAUNCH_CHECK("kvq_kivi_quant(values)");
      return KVQ_OK;
    }
  }
  if (along_tokens && vec && group <= 128) {
    const int n_g = (n + group - 1) / group;
    const int rpt = (group + 15) / 16;
    // one resident round of blocks (256 CUs x 4 blocks at these kernels' register use)
    const int64_t n_items = static_cast<int64_t>(n_g) * B * H;
    const unsigned grid = static_cast<unsigned>(KVQ_QUANT_GRID > 0 ? std::min<int64_t>(n_items, KVQ_QUANT_GRID) : n_items);
#define KVQ_KEYS_V(RPT_)                                                                                     \
    KVQ_DISPATCH_DTYPE(x_dtype, hipLaunchKernelGGL((kivi_quant_keys_v<DT_, RPT_>), dim3(grid), dim3(256), 0, s,  \
                                                   x, (int)H, sb, sh, st, n_sink, n, bits, group, codes, codes_bh,      \
                                                   packed, packed_bh, lo, scale, meta_bh, xhat, (int)T, n_g, n_items))
    if (rpt <= 1) { KVQ_KEYS_V(1); }
    else if (rpt <= 2) { KVQ_KEYS_V(2); }
    else if (rpt <= 4) { KVQ_KEYS_V(4); }
    else { KVQ_KEYS_V(8); }
#undef KVQ_KEYS_V
    KVQ_LAUNCH_CHECK("kvq_kivi_quant(keys)");
    return KVQ_OK;
  }
  if (!along_tokens && vec) {
    const int64_t width = (d % group == 0) ? group : d;
    if (width % 8 == 0 && ((width / 8) & (width / 8 - 1)) == 0) {
      constexpr int kVR = 4;
      const int n_rb = (n + 16 * kVR - 1) / (16 * kVR);
      const int64_t n_items = static_cast<int64_t>(n_rb) * B * H;
      const unsigned grid = static_cast<unsigned>(KVQ_QUANT_GRID > 0 ? std::min<int64_t>(n_items, KVQ_QUANT_GRID) : n_items);
      KVQ_DISPATCH_DTYPE(x_dtype, hipLaunchKernelGGL((kivi_quant_values_v<DT_, kVR>), dim3(grid), dim3(256), 0, s,
                                                     x, (int)H, sb, sh, st, n_sink, n, bits, (int)width, codes,
                                                     codes_bh, packed, packed_bh, lo, scale, meta_bh, xhat, (int)T,
                                                     n_rb, n_items));
      KVQ_LAUNCH_CHECK("kvq_kivi_quant(values)");
      return KVQ_OK;
    }
  }
  if (along_tokens) {
    KVQ_REQUIRE(d <= 1024 && d % 64 == 0, "kvq_kivi_quant(keys): d must be a multiple of 64 <= 1024");
    const int n_g = (n + group - 1) / group;
    KVQ_DISPATCH_DTYPE(x_dtype, hipLaunchKernelGGL((kivi_quant_keys<DT_>), dim3(n_g, B * H), dim3(d), 0, s,
                                                   x, (int)H, sb, sh, st, n_sink, n, (int)d, bits, group,
                                                   codes, codes_bh, packed, packed_bh, lo, scale,
                                                   meta_bh, xhat, (int)T));
  } else {
    const int64_t width = (d % group == 0) ? group : d;
    const int64_t lanes = width / 8;
    KVQ_REQUIRE(d % 8 == 0 && width % 8 == 0 && lanes <= 64 && (lanes & (lanes - 1)) == 0 &&
                    d / 8 <= 256,
                "kvq_kivi_quant(values): need d %% 8 == 0 and width/8 a power of two <= 64");
    const int slabs = static_cast<int>(d / 8);
    const int tpb = 256 / slabs;
    KVQ_DISPATCH_DTYPE(x_dtype, hipLaunchKernelGGL((kivi_quant_values<DT_>), grid1d(n, tpb, B * H), dim3(256),
                                                   0, s, x, (int)H, sb, sh, st, n_sink, n, (int)d, bits,
                                                   (int)width, codes, codes_bh, packed, packed_bh, lo,
                                                   scale, meta_bh, xhat, (int)T));
  }
  KVQ_LAUNCH_CHECK("kvq_kivi_quant");
  return KVQ_OK;
}

namespace kvq {
namespace {
// Decode of pack_rows bytes through a byte table (QUASAR_KV.py:1185-1202): byte i holds 8/bits
// codes, the first in the most significant bits; each code becomes levels[code].  One thread per
// byte; the 2^bits levels sit in LDS, so a byte costs one load and 8/bits table reads.
__global__ __launch_bounds__(256) void unpack_rows_lut_kernel(const uint8_t* __restrict__ packed, int64_t n_bytes,
                                                              int bits, const float* __restrict__ levels,
                                                              float* __restrict__ out) {
  __shared__ float lv[256];
  const int nl = 1 << bits;
  for (int i = threadIdx.x; i < nl; i += blockDim.x) lv[i] = levels[i];
  __syncthreads();
  const int per = 8 / bits;
  const uint32_t mask = static_cast<uint32_t>(nl - 1);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n_bytes;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const uint32_t byte = packed[i];
    for (int s = 0; s < per; ++s) out[i * per + s] = lv[(byte >> (bits * (per - 1 - s))) & mask];
  }
}
}  // namespace
}  // namespace kvq

extern "C" int kvq_pack_codes(const uint8_t* codes, int64_t count, int bits, uint8_t* out, void* stream) {
  KVQ_REQUIRE(bits == 1 || bits == 2 || bits == 4 || bits == 8, "kvq_pack_codes: bits in {1,2,4,8}");
  KVQ_REQUIRE(count >= 0 && (count == 0 || (codes && out)), "kvq_pack_codes: bad arguments");
  const int64_t nbytes = (count * bits + 7) / 8;
  if (nbytes == 0) return KVQ_OK;
  hipLaunchKernelGGL(pack_codes_kernel, grid1d(nbytes, 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), codes, count, bits, out, nbytes);
  KVQ_LAUNCH_CHECK("kvq_pack_codes");
  return KVQ_OK;
}

extern "C" int kvq_unpack_codes(const uint8_t* packed, int64_t count, int bits, uint8_t* out, void* stream) {
  KVQ_REQUIRE(bits == 1 || bits == 2 || bits == 4 || bits == 8, "kvq_unpack_codes: bits in {1,2,4,8}");
  KVQ_REQUIRE(count >= 0 && (count == 0 || (packed && out)), "kvq_unpack_codes: bad arguments");
  if (count == 0) return KVQ_OK;
  hipLaunchKernelGGL(unpack_codes_kernel, grid1d(count, 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), packed, count, bits, out);
  KVQ_LAUNCH_CHECK("kvq_unpack_codes");
  return KVQ_OK;
}

extern "C" int kvq_unpack_rows_lut(const uint8_t* packed, int64_t n_bytes, int bits, const float* levels,
                                   float* out, void* stream) {
  KVQ_REQUIRE(bits == 1 || bits == 2 || bits == 4 || bits == 8, "kvq_unpack_rows_lut: bits in {1,2,4,8}");
  KVQ_REQUIRE(n_bytes >= 0 && (n_bytes == 0 || (packed && levels && out)), "kvq_unpack_rows_lut: bad arguments");
  if (n_bytes == 0) return KVQ_OK;
  const int64_t blocks = std::min<int64_t>((n_bytes + 255) / 256, 65536);
  hipLaunchKernelGGL(unpack_rows_lut_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), packed, n_bytes, bits, levels, out);
  KVQ_LAUNCH_CHECK("kvq_unpack_rows_lut");
  return KVQ_OK;
}

extern "C" int kvq_v_tile(const uint8_t* rows, int64_t BH, int64_t n, int64_t rows_bh, int64_t d,
                          int64_t cap_t, uint8_t* tiles, void* stream) {
  KVQ_REQUIRE((n == 0 || rows) && tiles, "kvq_v_tile: null pointer");
  KVQ_REQUIRE(d % 64 == 0 && d > 0 && cap_t % 32 == 0 && n >= 0 && n <= cap_t && BH >= 0,
              "kvq_v_tile: need d %% 64 == 0, cap_t %% 32 == 0, 0 <= n <= cap_t");
  if (BH == 0 || cap_t == 0) return KVQ_OK;
  hipLaunchKernelGGL(v_tile_kernel, grid1d((cap_t / 32) * 4 * d, 256, BH), dim3(256), 0,
                     static_cast<hipStream_t>(stream), rows, n, rows_bh, (int)d, cap_t, tiles);
  KVQ_LAUNCH_CHECK("kvq_v_tile");
  return KVQ_OK;
}

extern "C" int kvq_v_untile(const uint8_t* tiles, int64_t BH, int64_t n, int64_t d, int64_t cap_t,
                            uint8_t* rows, int64_t rows_bh, void* stream) {
  KVQ_REQUIRE(rows && tiles, "kvq_v_untile: null pointer");
  KVQ_REQUIRE(d % 64 == 0 && d > 0 && cap_t % 32 == 0 && n >= 0 && n <= cap_t && BH >= 0,
              "kvq_v_untile: need d %% 64 == 0, cap_t %% 32 == 0, 0 <= n <= cap_t");
  if (BH == 0 || n == 0) return KVQ_OK;
  hipLaunchKernelGGL(v_untile_kernel, grid1d(n * (d / 2), 256, BH), dim3(256), 0,
                     static_cast<hipStream_t>(stream), tiles, n, (int)d, cap_t, rows, rows_bh);
  KVQ_LAUNCH_CHECK("kvq_v_untile");
  return KVQ_OK;
}

extern "C" int kvq_vmeta_tile(const uint16_t* lo, const uint16_t* scale, int64_t BH, int64_t n,
                              int64_t ngv, int64_t meta_bh, int64_t cap_t, uint16_t* vmeta, void* stream) {
  KVQ_REQUIRE((n == 0 || (lo && scale)) && vmeta, "kvq_vmeta_tile: null pointer");
  KVQ_REQUIRE(cap_t % 32 == 0 && n >= 0 && n <= cap_t && ngv > 0 && BH >= 0,
              "kvq_vmeta_tile: need cap_t %% 32 == 0, 0 <= n <= cap_t");
  if (BH == 0 || cap_t == 0) return KVQ_OK;
  hipLaunchKernelGGL(vmeta_tile_kernel, grid1d((cap_t / 32) * ngv * 32, 256, BH), dim3(256), 0,
                     static_cast<hipStream_t>(stream), lo, scale, n, ngv, meta_bh, cap_t, vmeta);
  KVQ_LAUNCH_CHECK("kvq_vmeta_tile");
  return KVQ_OK;
}
