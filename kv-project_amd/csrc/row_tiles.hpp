// Dense products of query-like rows with 16-token tiles on the matrix cores (gfx950), shared by the
// SnapKV scores and the STRATA coverage statistics.
//
// v_mfma_f32_16x16x32_{bf16,f16} (layout in mfma_common.hpp): A = 16 tokens x 32 channels of one
// k-step (lane l: token l%16, channels 8(l/16)..+7), B = 32 channels x 16 rows, D lane l register i =
// (token 4(l/16) + i, row l%16).  16-bit inputs are exact operands of their own type; fp32 values
// enter as two parts of the operand type (hi + lo, ~2^-22 relative for fp16 parts, ~2^-17 for bf16
// parts), each fp32 tensor first brought into the parts' range by a power of two (rows_scale_kernel),
// and the products hi*hi + hi*lo + lo*hi are accumulated in fp32.
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

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// two fp32 values rounded to nearest even as one packed bf16 pair (one v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack_bf2(float a, float b) {
  return __builtin_bit_cast(uint32_t, bf16x2{static_cast<__bf16>(a), static_cast<__bf16>(b)});
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

// the operand parts of 8 consecutive DT channels at element i of a row (plain loads, in bounds);
// fp32 values are multiplied by sc (the tensor's power of two, rows_scale_kernel) before the split
template <int DT>
__device__ __forceinline__ void load_op(const void* base, int64_t i, u32x4 (&op)[TileOps<DT>::NH], float sc = 1.0f) {
  if constexpr (DT == KVQ_F32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + i);
    const float4 a = p[0], c = p[1];
    const float x[8] = {a.x * sc, a.y * sc, a.z * sc, a.w * sc, c.x * sc, c.y * sc, c.z * sc, c.w * sc};
    f32_parts<DT>(x, op[0], op[1]);
  } else {
    op[0] = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + i);
  }
}

// the same through a buffer resource (reads past the resource return zero)
template <int DT>
__device__ __forceinline__ void load_op_buf(__amdgpu_buffer_rsrc_t rs, int byte_off, u32x4 (&op)[TileOps<DT>::NH],
                                            float sc = 1.0f) {
  if constexpr (DT == KVQ_F32) {
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rs, byte_off, 0, 0);
    const u32x4 c = __builtin_amdgcn_raw_buffer_load_b128(rs, byte_off + 16, 0, 0);
    float x[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      x[k] = __uint_as_float(a[k]) * sc;
      x[4 + k] = __uint_as_float(c[k]) * sc;
    }
    f32_parts<DT>(x, op[0], op[1]);
  } else {
    op[0] = __builtin_amdgcn_raw_buffer_load_b128(rs, byte_off, 0, 0);
  }
}

// fp32 rows enter the products as fp16 hi + lo parts, whose range ends at 65504 (and whose lo part
// turns subnormal for values below about 2^-2), so each fp32 tensor is first multiplied by a power of
// two (exact) that brings its largest finite |x| to [2^12, 2^13); the products are scaled back by the
// inverse powers.  The power is at most 2^63, so that the product of two of them stays finite: a
// tensor whose largest |x| is below 2^-50 comes out smaller than 2^13 (full precision down to a
// largest |x| of about 2^-66; below that its products lose relative precision, and they are zero
// below about 2^-87, never NaN).  A view of rows of 128 floats: row (i0, i1, i2) at base + i0 s0 + i1 s1 + i2 s2.
struct RowView {
  const float* base;
  int n0, n1, n2;
  int64_t s0, s1, s2;
};
constexpr int kAmaxBlocks = 128;                         // workgroups per view of the magnitude pass
constexpr int kAmaxViews = 3;                            // views of one pass at most
constexpr int64_t kAmaxFloats = kAmaxViews * kAmaxBlocks + kAmaxViews;   // partial maxima + scales

// per (view blockIdx.y, workgroup): the largest finite |x| of its share of the view's rows (NaN and
// infinities skipped: they cannot be scaled into range, and masked rows may hold them)
__global__ __launch_bounds__(256) void rows_absmax_kernel(RowView v0, RowView v1, RowView v2, float* part) {
  __shared__ float red[4];
  const RowView v = blockIdx.y == 0 ? v0 : (blockIdx.y == 1 ? v1 : v2);
  const int64_t units = static_cast<int64_t>(v.n0) * v.n1 * v.n2 * 32;   // float4 units
  float m = 0.0f;
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; u < units;
       u += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t row = u / 32;
    const int64_t i2 = row % v.n2, r1 = row / v.n2;
    const int64_t i1 = r1 % v.n1, i0 = r1 / v.n1;
    const float4 x = *reinterpret_cast<const float4*>(v.base + i0 * v.s0 + i1 * v.s1 + i2 * v.s2 + 4 * (u % 32));
    const float a[4] = {fabsf(x.x), fabsf(x.y), fabsf(x.z), fabsf(x.w)};
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (a[k] < INFINITY) m = fmaxf(m, a[k]);
  }
  m = wave_max(m);
  if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = m;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.y * gridDim.x + blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// one wavefront per view: scale[v] = 2^min(13 - e, 63) for a largest |x| of f 2^e (f in [0.5, 1)),
// 1 when the view is all zeros
__global__ __launch_bounds__(64 * kAmaxViews) void rows_scale_kernel(const float* part, int n_part, float* scale) {
  const int vi = threadIdx.x / 64, lane = threadIdx.x % 64;
  float m = 0.0f;
  for (int i = lane; i < n_part; i += 64) m = fmaxf(m, part[vi * n_part + i]);
  m = wave_max(m);
  if (lane == 0) {
    int e = 0;
    if (m > 0.0f) (void)frexpf(m, &e);
    scale[vi] = m > 0.0f ? ldexpf(1.0f, min(13 - e, 63)) : 1.0f;
  }
}

// the scales of n_views (1..3) fp32 views into scale[0 .. n_views), partial maxima in part
inline void launch_rows_scales(const RowView* views, int n_views, float* part, float* scale, hipStream_t s) {
  hipLaunchKernelGGL(rows_absmax_kernel, dim3(kAmaxBlocks, n_views), dim3(256), 0, s, views[0],
                     views[n_views > 1 ? 1 : 0], views[n_views > 2 ? 2 : 0], part);
  hipLaunchKernelGGL(rows_scale_kernel, dim3(1), dim3(64 * n_views), 0, s, part, kAmaxBlocks, scale);
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
