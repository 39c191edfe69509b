// Library-wide entry points: error reporting, ABI version, and the operand-layout self-test the
// decode kernel's lane mapping is written against.
#include <cstdarg>

#include "common.hpp"

namespace kvq {

namespace {
thread_local char g_last_error[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// One wavefront: lane l feeds a[l*8..l*8+7] / b[l*8..] as its A / B operand registers and writes
// the four accumulator registers it receives, then the lane index it reads through row_shr:4 and
// row_ror:4 (DPP within rows of 16 lanes).
__global__ void mfma_layout_probe(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,
                                  float* __restrict__ out) {
  const int l = threadIdx.x;
  half8 av, bv;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    av[k] = __builtin_bit_cast(_Float16, a[l * 8 + k]);
    bv[k] = __builtin_bit_cast(_Float16, b[l * 8 + k]);
  }
  f32x4 c = {0.f, 0.f, 0.f, 0.f};
  c = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, c, 0, 0, 0);
#pragma unroll
  for (int i = 0; i < 4; ++i) out[l * 4 + i] = c[i];
  const int shr = __builtin_amdgcn_update_dpp(-1, l, 0x114, 0xF, 0xF, false);
  const int ror = __builtin_amdgcn_update_dpp(-1, l, 0x124, 0xF, 0xF, false);
  out[256 + l] = static_cast<float>(shr);
  out[320 + l] = static_cast<float>(ror);
  // gfx950 cross-row swaps: the lane each lane receives in the second result of
  // v_permlane32_swap / v_permlane16_swap with both operands holding the lane index
  const auto s32 = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(l), static_cast<unsigned>(l), false, false);
  const auto s16 = __builtin_amdgcn_permlane16_swap(static_cast<unsigned>(l), static_cast<unsigned>(l), false, false);
  out[384 + l] = static_cast<float>(s32[0]);
  out[448 + l] = static_cast<float>(s32[1]);
  out[512 + l] = static_cast<float>(s16[0]);
  out[576 + l] = static_cast<float>(s16[1]);
}

}  // namespace
}  // namespace kvq

extern "C" const char* kvq_last_error(void) { return kvq::g_last_error; }

extern "C" int kvq_abi_version(void) { return 18; }

extern "C" int kvq_selftest_mfma_layout(const uint16_t* a, const uint16_t* b, float* out, void* stream) {
  KVQ_REQUIRE(a && b && out, "kvq_selftest_mfma_layout: null pointer");
  hipLaunchKernelGGL(kvq::mfma_layout_probe, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), a, b, out);
  KVQ_LAUNCH_CHECK("kvq_selftest_mfma_layout");
  return KVQ_OK;
}
