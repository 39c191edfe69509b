// KIVI group quantisation, MSB-first packing and the value-tile decode layout (gfx950).
//
// kivi_quant semantics follow STRATA_KV.py:826-856 bit for bit:
//   lo    = fp16(clamp(min, +-65504))                           (as_stored, 539-542)
//   scale = max(fp16(clamp((max - lo) / qmax)), 2^-24)          (IEEE fp32 subtract and divide)
//   code  = clamp(rint((x - lo) / scale), 0, qmax)               (round half to even)
//   xhat  = code * scale + lo                                   (two roundings, never fused)
// All arithmetic that feeds a code or a metadata value uses the explicitly rounded intrinsics so
// that no multiply-add contraction can change a bit.
#include "common.hpp"

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
  const bool valid = t < n && threadIdx.x < tok_per_block * slabs;
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
