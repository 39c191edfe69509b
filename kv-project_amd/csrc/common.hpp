// Shared helpers of libkvq: error reporting, dtype codes, fp16 / bf16 conversion.
// Every entry point returns 0 (KVQ_OK) or a nonzero status and records a message that
// kvq_last_error() returns; nothing here allocates device memory or synchronises.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/kvq.h"

namespace kvq {

void set_error(const char* fmt, ...);

#define KVQ_REQUIRE(cond, ...)                 \
  do {                                         \
    if (!(cond)) {                             \
      ::kvq::set_error(__VA_ARGS__);           \
      return KVQ_EINVAL;                       \
    }                                          \
  } while (0)

#define KVQ_LAUNCH_CHECK(what)                                               \
  do {                                                                       \
    hipError_t e_ = hipGetLastError();                                       \
    if (e_ != hipSuccess) {                                                  \
      ::kvq::set_error("%s: %s", what, hipGetErrorString(e_));               \
      return KVQ_EHIP;                                                       \
    }                                                                        \
  } while (0)

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (gfx950's v_cvt_pk_bf16_f32; NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}

// fp32 -> fp16, round to nearest even (hardware conversion under the default rounding mode).
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __half_as_ushort(__float2half_rn(f));
}

template <int DT>
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i) {
  if constexpr (DT == KVQ_F32) return static_cast<const float*>(p)[i];
  else if constexpr (DT == KVQ_F16) return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
  else return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

template <int DT>
__device__ __forceinline__ void store_from_f32(void* p, int64_t i, float v) {
  if constexpr (DT == KVQ_F32) static_cast<float*>(p)[i] = v;
  else if constexpr (DT == KVQ_F16) static_cast<uint16_t*>(p)[i] = f32_to_f16(v);
  else static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
}

// 8 consecutive elements (16-byte aligned) as floats: one 16-byte load for 16-bit types, two for fp32
template <int DT>
__device__ __forceinline__ void load8(const void* base, int64_t i, float (&x)[8]) {
  if constexpr (DT == KVQ_F32) {
    const float4* p4 = reinterpret_cast<const float4*>(static_cast<const float*>(base) + i);
    const float4 a = p4[0], c = p4[1];
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = c.x; x[5] = c.y; x[6] = c.z; x[7] = c.w;
  } else {
    const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + i);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint16_t lo = static_cast<uint16_t>(ws[k] & 0xffffu), hi = static_cast<uint16_t>(ws[k] >> 16);
      x[2 * k] = DT == KVQ_F16 ? f16_to_f32(lo) : bf16_to_f32(lo);
      x[2 * k + 1] = DT == KVQ_F16 ? f16_to_f32(hi) : bf16_to_f32(hi);
    }
  }
}

// 4 consecutive elements (8-byte aligned for 16-bit types, 16-byte for fp32) as floats: one load
template <int DT>
__device__ __forceinline__ void load4(const void* base, int64_t i, float (&x)[4]) {
  if constexpr (DT == KVQ_F32) {
    const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + i);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
  } else {
    const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + i);
    const uint32_t ws[2] = {w.x, w.y};
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const uint16_t lo = static_cast<uint16_t>(ws[k] & 0xffffu), hi = static_cast<uint16_t>(ws[k] >> 16);
      x[2 * k] = DT == KVQ_F16 ? f16_to_f32(lo) : bf16_to_f32(lo);
      x[2 * k + 1] = DT == KVQ_F16 ? f16_to_f32(hi) : bf16_to_f32(hi);
    }
  }
}

// Correctly rounded float32 square root (IEEE round to nearest, what numpy and torch compute on the
// host).  The hardware root (v_sqrt_f32) is accurate to about one ulp, not correctly rounded, so
// its result y is moved to the nearest root by Tuckerman's test (Markstein, "IA-64 and Elementary
// Functions", 2000, section 9.3): with y- and y+ the neighbours of y, RN(sqrt(x)) is y- when
// x <= y y-, y+ when x > y y+, else y; the sign of x - y y± is exact through one fma.  Arguments
// below 2^-96 are scaled by 2^32 first (the root by 2^-16 after: exact), so the neighbours stay
// normal numbers.
__device__ __forceinline__ float sqrt_rn(float x) {
  const bool small = x < 0x1p-96f;
  const float xs = small ? x * 0x1p32f : x;
  float y = __builtin_amdgcn_sqrtf(xs);
  if (xs > 0.0f && xs < INFINITY) {
    const float yd = __uint_as_float(__float_as_uint(y) - 1u);
    const float yu = __uint_as_float(__float_as_uint(y) + 1u);
    if (__builtin_fmaf(-yd, y, xs) <= 0.0f) y = yd;
    else if (__builtin_fmaf(-yu, y, xs) > 0.0f) y = yu;
  }
  return small ? y * 0x1p-16f : y;
}

inline bool valid_dtype(int dt) { return dt == KVQ_F32 || dt == KVQ_F16 || dt == KVQ_BF16; }

}  // namespace kvq

// Dispatch a runtime dtype code to a compile-time template parameter named DT_.
#define KVQ_DISPATCH_DTYPE(dt, ...)                          \
  switch (dt) {                                              \
    case KVQ_F32: { constexpr int DT_ = KVQ_F32; __VA_ARGS__; break; }   \
    case KVQ_F16: { constexpr int DT_ = KVQ_F16; __VA_ARGS__; break; }   \
    case KVQ_BF16: { constexpr int DT_ = KVQ_BF16; __VA_ARGS__; break; } \
    default: ::kvq::set_error("unknown dtype code %d", (int)(dt)); return KVQ_EINVAL; \
  }
