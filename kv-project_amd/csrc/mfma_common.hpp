// Matrix-core and cross-lane helpers shared by the decode kernels (gfx950, wave64).
//
// v_mfma_f32_16x16x32_f16 operand layout (checked on the hardware by kvq_selftest_mfma_layout):
//   A (16x32): lane l holds A[l%16][8*(l/16) + k], k = 0..7
//   B (32x16): lane l holds B[8*(l/16) + k][l%16]
//   D (16x16): lane l register i holds D[4*(l/16) + i][l%16]
#pragma once
#include "common.hpp"

namespace kvq {
namespace {

// Row stride (dwords) of the per-wavefront staging rows of the query B operand: 64 + 4, so that
// the rows (one per (query row, hi/lo) column pair) start in different LDS banks and the 16-byte
// operand reads of one lane group do not all collide in the same four banks.
constexpr int kBqStride = 68;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  // raw buffer: loads past `bytes` return zero instead of touching memory
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), 0x00020000);
}

__device__ __forceinline__ half2v h2(uint32_t w) { return __builtin_bit_cast(half2v, w); }
__device__ __forceinline__ uint32_t w2(half2v h) { return __builtin_bit_cast(uint32_t, h); }

__device__ __forceinline__ half8 as_half8(u32x4 v) { return __builtin_bit_cast(half8, v); }

__device__ __forceinline__ f32x4 mfma(half8 a, half8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}
constexpr int kRowShr = 0x110;     // row_shr:k  (lane i reads lane i-k of its row of 16)
constexpr int kRowRor = 0x120;     // row_ror:k
constexpr int kQuadSwap1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kQuadSwap2 = 0x4E;   // quad_perm [2,3,0,1]

// max / sum with the xor-16 and xor-32 lane partners (gfx950 permlane swaps: VALU, no LDS trip)
__device__ __forceinline__ float xmax16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xmax32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xmin16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fminf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xmin32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fminf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xsum16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xsum32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// sum / max over the 16 lanes of a row, every lane receiving the same value (DPP row rotations by
// 8, 4, 2, 1: each step adds a commutative pair, so all lanes round alike; no LDS trip)
__device__ __forceinline__ float row_sum16(float x) {
  x += dpp<kRowRor + 8>(x);
  x += dpp<kRowRor + 4>(x);
  x += dpp<kRowRor + 2>(x);
  x += dpp<kRowRor + 1>(x);
  return x;
}
__device__ __forceinline__ float row_max16(float x) {
  x = fmaxf(x, dpp<kRowRor + 8>(x));
  x = fmaxf(x, dpp<kRowRor + 4>(x));
  x = fmaxf(x, dpp<kRowRor + 2>(x));
  x = fmaxf(x, dpp<kRowRor + 1>(x));
  return x;
}
// over the whole wavefront (rows, then the xor-16 and xor-32 partners)
__device__ __forceinline__ float wave_sum(float x) { return xsum32(xsum16(row_sum16(x))); }
__device__ __forceinline__ float wave_max(float x) { return xmax32(xmax16(row_max16(x))); }

__device__ __forceinline__ uint32_t pack_h2(_Float16 a, _Float16 b) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, a)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b)) << 16);
}

__device__ __forceinline__ float h2f(uint32_t w, int hi) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(hi ? (w >> 16) : (w & 0xffffu))));
}

__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Workgroup barrier ordering LDS only: each wavefront waits for its own LDS operations, not for
// its outstanding global / buffer loads (a plain __syncthreads waits for those too).
__device__ __forceinline__ void block_lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace
}  // namespace kvq
