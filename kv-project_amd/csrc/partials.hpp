// Exact merge of flash-decoding partials (m, l, o) in base 2 and the output write, shared by every
// decode kernel whose partials need no post-processing (packed KIVI, DCT blocks, mixed-width
// blocks).  Two partial sets per (b, h): S_ex partials of exact rows and S coded partials, each
// (m, l, o[D]) per row r of the R padded rows; o = sum_j exp2(s_j - m) v_j, l = sum_j exp2(s_j - m).
// The result out[b, t, hq, :] = sum_s exp2(m_s - M) o_s / sum_s exp2(m_s - M) l_s, M = max_s m_s
// (the combination StrataState.attend performs in base e, STRATA_KV.py:1784-1792).
//
// One workgroup per (b, h, row): the partials are spread over all 256 threads (max and sum by
// block reduction; the output columns by 128 channels x 2 partial halves), so the merge costs a
// few dependent loads whatever the split count.
#pragma once
#include <algorithm>

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
  float* row_ml;                  // optional (BH, R, 2): the row's M and L
};

constexpr int kMergeThreads = 256;

__device__ __forceinline__ float block_reduce_256(float v, bool is_max, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float u = __shfl_xor(v, o, 64);
    v = is_max ? fmaxf(v, u) : v + u;
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float a = red[0], b = red[1], c = red[2], d = red[3];
  return is_max ? fmaxf(fmaxf(a, b), fmaxf(c, d)) : (a + b) + (c + d);
}

// grid = BH * R_real workgroups of kMergeThreads
template <int R, int DT, int D>
__global__ __launch_bounds__(kMergeThreads) void merge_rows_kernel(MergeArgs a) {
  static_assert(kMergeThreads % D == 0, "channels must divide the workgroup");
  constexpr int PARTS = kMergeThreads / D;
  __shared__ float red[4];
  __shared__ float part_o[PARTS][D];
  const int bh = blockIdx.x / a.R_real, r = blockIdx.x % a.R_real;
  const int tid = threadIdx.x;
  const int S_all = a.S_ex + a.S;
  // partial s: exact-row partials first, then the coded ones
  auto m_of = [&](int s) -> float {
    return s < a.S_ex ? a.ex_m[(static_cast<int64_t>(bh) * a.S_ex + s) * R + r]
                      : a.ws_m[(static_cast<int64_t>(bh) * a.S + (s - a.S_ex)) * R + r];
  };
  auto l_of = [&](int s) -> float {
    return s < a.S_ex ? a.ex_l[(static_cast<int64_t>(bh) * a.S_ex + s) * R + r]
                      : a.ws_l[(static_cast<int64_t>(bh) * a.S + (s - a.S_ex)) * R + r];
  };
  auto o_of = [&](int s, int c) -> float {
    return s < a.S_ex ? a.ex_o[((static_cast<int64_t>(bh) * a.S_ex + s) * R + r) * D + c]
                      : a.ws_o[((static_cast<int64_t>(bh) * a.S + (s - a.S_ex)) * R + r) * D + c];
  };
  float m = -INFINITY;
  for (int s = tid; s < S_all; s += kMergeThreads) m = fmaxf(m, m_of(s));
  const float M = block_reduce_256(m, true, red);
  float l = 0.0f;
  for (int s = tid; s < S_all; s += kMergeThreads) {
    const float ms = m_of(s);
    if (ms != -INFINITY) l += __builtin_amdgcn_exp2f(ms - M) * l_of(s);
  }
  const float L = block_reduce_256(l, false, red);
  const int c = tid % D, part = tid / D;
  float o = 0.0f;
#pragma unroll 4
  for (int s = part; s < S_all; s += PARTS) {
    const float ms = m_of(s);
    const float w = ms == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ms - M);
    o = __builtin_fmaf(w, o_of(s, c), o);
  }
  part_o[part][c] = o;
  __syncthreads();
  if (part == 0) {
    float O = 0.0f;
#pragma unroll
    for (int k = 0; k < PARTS; ++k) O += part_o[k][c];
    const int b = bh / a.Hkv, h = bh % a.Hkv;
    const int hq = h * a.rep + r / a.Tq, t = r % a.Tq;
    store_from_f32<DT>(a.out, ((static_cast<int64_t>(b) * a.Tq + t) * a.Hq + hq) * D + c, O / L);
  }
  if (tid == 0 && a.row_ml != nullptr) {
    a.row_ml[(static_cast<int64_t>(bh) * R + r) * 2] = M;
    a.row_ml[(static_cast<int64_t>(bh) * R + r) * 2 + 1] = L;
  }
}

// Splits per (b, h) of a block-streaming decode launch: BH * S workgroups of 4 wavefronts, each
// wavefront taking about nb / (4 S) blocks.  Workgroups run in rounds of `slots` resident ones
// (256 CUs x resident_per_cu); the count minimises rounds x (blocks of one wavefront + a fixed
// per-workgroup cost of `overhead` blocks), ties to fewer splits.
inline int plan_block_splits(int64_t BH, int64_t nb, int resident_per_cu, int64_t overhead) {
  if (nb <= 0 || BH <= 0) return 0;
  const int64_t slots = 256LL * resident_per_cu;
  const int64_t max_s = std::max<int64_t>(1, std::min<int64_t>((nb + 3) / 4, 1024));
  int64_t best = 1, best_cost = -1;
  for (int64_t s = 1; s <= max_s; ++s) {
    const int64_t rounds = (BH * s + slots - 1) / slots;
    const int64_t cost = rounds * ((nb + 4 * s - 1) / (4 * s) + overhead);
    if (best_cost < 0 || cost < best_cost) {
      best = s;
      best_cost = cost;
    }
  }
  return static_cast<int>(best);
}

inline int pow2_rows(int64_t r) {
  int R = 1;
  while (R < r) R <<= 1;
  return R;
}

// launch merge_rows_kernel for a runtime row count R (power of two <= 8) and output dtype
inline int launch_merge_rows(const MergeArgs& a, int R, int BH, int out_dtype, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(BH) * a.R_real);
#define KVQ_MERGE_L(R_, DT_) hipLaunchKernelGGL((merge_rows_kernel<R_, DT_, 128>), grid, dim3(kMergeThreads), 0, s, a)
#define KVQ_MERGE_R(DT_)                           \
  switch (R) {                                     \
    case 1: KVQ_MERGE_L(1, DT_); break;            \
    case 2: KVQ_MERGE_L(2, DT_); break;            \
    case 4: KVQ_MERGE_L(4, DT_); break;            \
    default: KVQ_MERGE_L(8, DT_); break;           \
  }
  switch (out_dtype) {
    case KVQ_F32: KVQ_MERGE_R(KVQ_F32) break;
    case KVQ_F16: KVQ_MERGE_R(KVQ_F16) break;
    default: KVQ_MERGE_R(KVQ_BF16) break;
  }
#undef KVQ_MERGE_R
#undef KVQ_MERGE_L
  KVQ_LAUNCH_CHECK("merge_rows");
  return KVQ_OK;
}

}  // namespace
}  // namespace kvq
