// Exact merge of flash-decoding partials (m, l, o) in base 2 and the output write, shared by the
// decode kernels whose partials need no post-processing (DCT blocks, mixed-width KIVI blocks).
// Two partial sets per (b, h): S_ex exact-row partials and S coded partials, each (m, l, o[d]) per
// row r of the R padded rows; o = sum_j exp2(s_j - m) v_j, l = sum_j exp2(s_j - m).  The result
// out[b, t, hq, :] = sum_s exp2(m_s - M) o_s / sum_s exp2(m_s - M) l_s, M = max_s m_s (the
// combination StrataState.attend performs in base e, STRATA_KV.py:1784-1792).
#pragma once
#include "common.hpp"

namespace kvq {
namespace {

struct MergeArgs {
  const float* ws_o;
  const float* ws_m;
  const float* ws_l;
  int S;
  const float* ex_o;
  const float* ex_m;
  const float* ex_l;
  int S_ex;
  int Hq, Hkv, Tq, rep, R_real;
  void* out;
};

// One workgroup per (b, h); `stat` holds 2R floats of shared memory.
template <int R, int DT, int D>
__device__ void merge_partials(const MergeArgs& a, int bh, float* stat) {
  const int b = bh / a.Hkv, h = bh % a.Hkv;
  if (threadIdx.x < R) {
    const int r = threadIdx.x;
    float M = -INFINITY, L = 0.0f;
    for (int s = 0; s < a.S_ex; ++s) M = fmaxf(M, a.ex_m[(static_cast<int64_t>(bh) * a.S_ex + s) * R + r]);
    for (int s = 0; s < a.S; ++s) M = fmaxf(M, a.ws_m[(static_cast<int64_t>(bh) * a.S + s) * R + r]);
    for (int s = 0; s < a.S_ex; ++s) {
      const int64_t po = static_cast<int64_t>(bh) * a.S_ex + s;
      if (a.ex_m[po * R + r] != -INFINITY) L += __builtin_amdgcn_exp2f(a.ex_m[po * R + r] - M) * a.ex_l[po * R + r];
    }
    for (int s = 0; s < a.S; ++s) {
      const int64_t po = static_cast<int64_t>(bh) * a.S + s;
      if (a.ws_m[po * R + r] != -INFINITY) L += __builtin_amdgcn_exp2f(a.ws_m[po * R + r] - M) * a.ws_l[po * R + r];
    }
    stat[r] = M;
    stat[R + r] = L;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < a.R_real * D; idx += blockDim.x) {
    const int r = idx / D, c = idx % D;
    const float M = stat[r];
    float O = 0.0f;
    for (int s = 0; s < a.S_ex; ++s) {
      const int64_t po = static_cast<int64_t>(bh) * a.S_ex + s;
      if (a.ex_m[po * R + r] != -INFINITY) O += __builtin_amdgcn_exp2f(a.ex_m[po * R + r] - M) * a.ex_o[(po * R + r) * D + c];
    }
    for (int s = 0; s < a.S; ++s) {
      const int64_t po = static_cast<int64_t>(bh) * a.S + s;
      if (a.ws_m[po * R + r] != -INFINITY) O += __builtin_amdgcn_exp2f(a.ws_m[po * R + r] - M) * a.ws_o[(po * R + r) * D + c];
    }
    const int hq = h * a.rep + r / a.Tq, t = r % a.Tq;
    store_from_f32<DT>(a.out, ((static_cast<int64_t>(b) * a.Tq + t) * a.Hq + hq) * D + c, O / stat[R + r]);
  }
}

inline int pow2_rows(int64_t r) {
  int R = 1;
  while (R < r) R <<= 1;
  return R;
}

}  // namespace
}  // namespace kvq
