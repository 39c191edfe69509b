// Dense products of query-like rows with 16-token tiles on the matrix cores (gfx950), shared by the
// SnapKV scores and the STRATA coverage statistics.
//
// v_mfma_f32_16x16x32_{bf16,f16} (layout in mfma_common.hpp): A = 16 tokens x 32 channels of one
// k-step (lane l: token l%16, channels 8(l/16)..+7), B = 32 channels x 16 rows, D lane l register i =
// (token 4(l/16) + i, row l%16).  16-bit inputs are exact operands of their own type; fp32 values
// enter as two parts of the operand type (hi + lo, ~2^-22 relative for fp16 parts, ~2^-17 for bf16
// parts), and the products hi*hi + hi*lo + lo*hi are accumulated in fp32.
#pragma once
#include "mfma_common.hpp"

namespace kvq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <int DT>
struct TileOps {
  static constexpr int NH = DT == KVQ_F32 ? 2 : 1;          // operand parts of a DT value
  static constexpr int ESZ = DT == KVQ_F32 ? 4 : 2;
};

// the matrix-core product of DT's operand type: bf16 for bf16 data, fp16 otherwise
template <int DT>
__device__ __forceinline__ f32x4 tile_mfma(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == KVQ_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0,
                                                  0, 0);
}

__device__ __forceinline__ uint32_t pack_bf2(float a, float b) {
  return static_cast<uint32_t>(f32_to_bf16(a)) | (static_cast<uint32_t>(f32_to_bf16(b)) << 16);
}

// fp32 x[8] -> hi and lo parts in DT's operand type (bf16 parts for bf16, fp16 parts otherwise)
template <int DT>
__device__ __forceinline__ void f32_parts(const float (&x)[8], u32x4& hi, u32x4& lo) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if constexpr (DT == KVQ_BF16) {
      const float h0 = bf16_to_f32(f32_to_bf16(x[2 * k])), h1 = bf16_to_f32(f32_to_bf16(x[2 * k + 1]));
      hi[k] = pack_bf2(h0, h1);
      lo[k] = pack_bf2(x[2 * k] - h0, x[2 * k + 1] - h1);
    } else {
      const _Float16 h0 = static_cast<_Float16>(x[2 * k]), h1 = static_cast<_Float16>(x[2 * k + 1]);
      hi[k] = pack_h2(h0, h1);
      lo[k] = pack_h2(static_cast<_Float16>(x[2 * k] - static_cast<float>(h0)),
                      static_cast<_Float16>(x[2 * k + 1] - static_cast<float>(h1)));
    }
  }
}

// the operand parts of 8 consecutive DT channels at element i of a row (plain loads, in bounds)
template <int DT>
__device__ __forceinline__ void load_op(const void* base, int64_t i, u32x4 (&op)[TileOps<DT>::NH]) {
  if constexpr (DT == KVQ_F32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + i);
    const float4 a = p[0], c = p[1];
    const float x[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
    f32_parts<DT>(x, op[0], op[1]);
  } else {
    op[0] = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + i);
  }
}

// the same through a buffer resource (reads past the resource return zero)
template <int DT>
__device__ __forceinline__ void load_op_buf(__amdgpu_buffer_rsrc_t rs, int byte_off, u32x4 (&op)[TileOps<DT>::NH]) {
  if constexpr (DT == KVQ_F32) {
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rs, byte_off, 0, 0);
    const u32x4 c = __builtin_amdgcn_raw_buffer_load_b128(rs, byte_off + 16, 0, 0);
    const float x[8] = {__uint_as_float(a[0]), __uint_as_float(a[1]), __uint_as_float(a[2]), __uint_as_float(a[3]),
                        __uint_as_float(c[0]), __uint_as_float(c[1]), __uint_as_float(c[2]), __uint_as_float(c[3])};
    f32_parts<DT>(x, op[0], op[1]);
  } else {
    op[0] = __builtin_amdgcn_raw_buffer_load_b128(rs, byte_off, 0, 0);
  }
}

// dot products over 128 channels of one 16-token tile (A, NA parts per k-step) with one 16-row block
// (B, NB parts): hi*hi, then hi*lo and lo*hi where the parts exist
template <int DT, int NA, int NB>
__device__ __forceinline__ f32x4 tile_dots(const u32x4 (&a)[4][NA], const u32x4 (&b)[4][NB]) {
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    acc = tile_mfma<DT>(a[ks][0], b[ks][0], acc);
    if constexpr (NB > 1) acc = tile_mfma<DT>(a[ks][0], b[ks][1], acc);
    if constexpr (NA > 1) acc = tile_mfma<DT>(a[ks][1], b[ks][0], acc);
  }
  return acc;
}

}  // namespace
}  // namespace kvq
