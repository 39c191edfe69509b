// Exact merge of flash-decoding partials (m, l, o) in base 2 and the output write, shared by every
// decode kernel whose partials need no post-processing (packed KIVI, DCT blocks, mixed-width
// blocks).  Two partial sets per (b, h): S_ex partials of exact rows and S coded partials, each
// (m, l, o[D]) per row r of the R padded rows; o = sum_j exp2(s_j - m) v_j, l = sum_j exp2(s_j - m).
// The result out[b, t, hq, :] = sum_s exp2(m_s - M) o_s / sum_s exp2(m_s - M) l_s, M = max_s m_s
// (the combination StrataState.attend performs in base e, STRATA_KV.py:1784-1792).
//
// One workgroup per (b, h, row): the partials are spread over all 256 threads (max and sum by
// block reduction; the output columns by 32 channel quads x 8 partial slices), so the merge
// costs a few dependent loads whatever the split count.  Rows with at most 32 partials and no
// exact rows to attend take one wavefront each instead (merge_rows_wave_kernel).
#pragma once
#include <algorithm>

#include "common.hpp"
#include "mfma_common.hpp"

namespace kvq {
namespace {

constexpr int kMergeThreadsEx = 256;              // threads of the merge blocks

// Exact rows (the residual window, appended tokens) a merge may attend itself instead of reading
// their partials: rows [0, n) of k_exact / v_exact (BH, cap_e, D) in the output dtype, visible to
// query t when exact_pos[i] <= q_pos[t] (both null: all visible).  The query row is read from q.
struct ExactArgs {
  const void* q;
  int64_t q_sb, q_sh, q_st;
  float qscale;                   // scaling * log2(e)
  const void* k_exact;
  const void* v_exact;
  int64_t cap_e;
  int n;                          // 0: no exact rows in the merge
  const int64_t* exact_pos;
  const int64_t* q_pos;
};

// Exact windows up to this many rows are attended inside the merge (one pass over them per query
// row, overlapping nothing but also adding no tail blocks to the split launch); longer ones are
// split into blocks of kExactRowsPerBlock rows of the split launch.
constexpr int64_t kExactInMerge = 1024;
constexpr int kExactRowsPerBlock = 64;
inline bool exact_in_merge(int64_t n_exact) { return n_exact > 0 && n_exact <= kExactInMerge; }

// Exact-row blocks of a window attended neither by packed splits nor by the merge: about one round
// of 768 workgroups over the BH (b, h) pairs, at least kExactRowsPerBlock rows each, rows per block
// a multiple of 16.  Returns the blocks per (b, h); *rows receives the rows of each block.
inline int plan_exact_blocks(int64_t BH, int64_t n_exact, int* rows) {
  const int64_t per_bh = std::max<int64_t>(1, 768 / std::max<int64_t>(BH, 1));
  const int64_t most = (n_exact + kExactRowsPerBlock - 1) / kExactRowsPerBlock;
  const int64_t nb = std::max<int64_t>(1, std::min(per_bh, most));
  const int64_t r = ((n_exact + nb - 1) / nb + 15) / 16 * 16;
  *rows = static_cast<int>(r);
  return static_cast<int>((n_exact + r - 1) / r);
}

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
  ExactArgs ex;                   // exact rows attended here (ex.n > 0)
};

// The exact-row partial of query row (b, hq, t) over the rows of (b, h) = bh, computed by the 256
// threads of a merge block: logits by 16-lane dot products (8 channels a lane), base-2 softmax
// statistics by block reductions, and the value sum of channel quad c4 over rows part, part + 8,
// ... (the merge's output layout).  Loads go out in batches with row indices clamped to n - 1 (a
// clamped row is loaded, never used), so a window of up to 128 rows costs one key and one value
// round trip.  sl: LDS for kExactInMerge logits.
template <int DT, int D>
__device__ void exact_partial(const ExactArgs& e, int b, int hq, int t, int bh, float* sl, float* red, float& me,
                              float& le, float4& oe, int c4, int part) {
  constexpr int kRowsPerPass = kMergeThreadsEx / 16;   // key rows one pass of the block covers
  constexpr int kKeyBatch = 8;                         // passes whose key loads are in flight together
  constexpr int kParts = kMergeThreadsEx / (D / 4);    // value row slices
  constexpr int kValBatch = 16;                        // value rows in flight per thread
  const int tid = threadIdx.x, lane = tid % 64;
  const int j = tid >> 4, pt = tid & 15;
  const int n = e.n;
  const int64_t qo = static_cast<int64_t>(b) * e.q_sb + static_cast<int64_t>(hq) * e.q_sh +
                     static_cast<int64_t>(t) * e.q_st + 8 * pt;
  float qv[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) qv[k] = load_as_f32<DT>(e.q, qo + k) * e.qscale;
  const int64_t base = static_cast<int64_t>(bh) * e.cap_e * D;
  const bool masked = e.exact_pos != nullptr && e.q_pos != nullptr;
  const int64_t qp = masked ? e.q_pos[t] : 0;
  for (int i0 = 0; i0 < n; i0 += kRowsPerPass * kKeyBatch) {
    float kx[kKeyBatch][8];
    bool vis[kKeyBatch];
#pragma unroll
    for (int u = 0; u < kKeyBatch; ++u) {
      const int i = min(i0 + u * kRowsPerPass + j, n - 1);
      load8<DT>(e.k_exact, base + static_cast<int64_t>(i) * D + 8 * pt, kx[u]);
      vis[u] = !masked || e.exact_pos[i] <= qp;
    }
#pragma unroll
    for (int u = 0; u < kKeyBatch; ++u) {
      float s = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) s = __builtin_fmaf(qv[k], kx[u][k], s);
      s = row_sum16(s);
      const int i = i0 + u * kRowsPerPass + j;
      if (pt == 0 && i < n) sl[i] = vis[u] ? s : -INFINITY;
    }
  }
  __syncthreads();
  float m = -INFINITY;
  for (int i = tid; i < n; i += kMergeThreadsEx) m = fmaxf(m, sl[i]);
  m = wave_max(m);
  if (lane == 0) red[tid / 64] = m;
  __syncthreads();
  me = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float l = 0.0f;
  for (int i = tid; i < n; i += kMergeThreadsEx) {
    const float pr = me == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sl[i] - me);
    sl[i] = pr;
    l += pr;
  }
  l = wave_sum(l);
  __syncthreads();                                  // red[] reads of the maximum are done
  if (lane == 0) red[tid / 64] = l;
  __syncthreads();
  le = (red[0] + red[1]) + (red[2] + red[3]);
  oe = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int i0 = part; i0 < n; i0 += kParts * kValBatch) {
    float vx[kValBatch][4];
#pragma unroll
    for (int u = 0; u < kValBatch; ++u) {
      const int i = min(i0 + u * kParts, n - 1);
      load4<DT>(e.v_exact, base + static_cast<int64_t>(i) * D + 4 * c4, vx[u]);
    }
#pragma unroll
    for (int u = 0; u < kValBatch; ++u) {
      const int i = i0 + u * kParts;
      const float pr = i < n ? sl[i] : 0.0f;
      oe.x = __builtin_fmaf(pr, vx[u][0], oe.x);
      oe.y = __builtin_fmaf(pr, vx[u][1], oe.y);
      oe.z = __builtin_fmaf(pr, vx[u][2], oe.z);
      oe.w = __builtin_fmaf(pr, vx[u][3], oe.w);
    }
  }
  __syncthreads();                                  // red[] free for the caller
}

constexpr int kMergeThreads = 256;

// barriers ordering LDS only: global loads issued before the reduction stay in flight across it
__device__ __forceinline__ float block_reduce_256(float v, bool is_max, float* red) {
  v = is_max ? wave_max(v) : wave_sum(v);
  block_lds_barrier();                              // earlier reads of red[] are done
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  block_lds_barrier();
  const float a = red[0], b = red[1], c = red[2], d = red[3];
  return is_max ? fmaxf(fmaxf(a, b), fmaxf(c, d)) : (a + b) + (c + d);
}

// grid = BH * R_real workgroups of kMergeThreads; thread t sums channels 4 (t % (D/4)) .. +3 of
// the partials s = t / (D/4) (mod PARTS) with 16-byte loads, the PARTS slices meet in LDS.  The
// first NPRE partials of every slice are loaded before anything else, so a merge of up to
// NPRE x PARTS partials waits for one round of loads.
template <int R, int DT, int D, int NPRE>
__global__ __launch_bounds__(kMergeThreads) void merge_rows_kernel(MergeArgs a) {
  static_assert(kMergeThreads % (D / 4) == 0, "channel quads must divide the workgroup");
  constexpr int PARTS = kMergeThreads / (D / 4);
  __shared__ float red[4];
  __shared__ float4 part_o[PARTS][D / 4];
  __shared__ float sl[kExactInMerge];
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
  auto o_of = [&](int s, int c4) -> float4 {
    const float* base = s < a.S_ex ? a.ex_o + ((static_cast<int64_t>(bh) * a.S_ex + s) * R + r) * D
                                   : a.ws_o + ((static_cast<int64_t>(bh) * a.S + (s - a.S_ex)) * R + r) * D;
    return reinterpret_cast<const float4*>(base)[c4];
  };
  const int c4 = tid % (D / 4), part = tid / (D / 4);
  const int b = bh / a.Hkv, h = bh % a.Hkv;
  const int hq = h * a.rep + r / a.Tq, t = r % a.Tq;
  // the first partials are loaded before the exact pass so their latency overlaps it
  const float m0 = tid < S_all ? m_of(tid) : -INFINITY;
  const float l0 = tid < S_all ? l_of(tid) : 0.0f;
  float mp[NPRE];
  float4 op[NPRE];
#pragma unroll
  for (int k = 0; k < NPRE; ++k) {
    const int s = part + PARTS * k;
    mp[k] = s < S_all ? m_of(s) : -INFINITY;
    op[k] = s < S_all ? o_of(s, c4) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  // exact rows attended here: their own partial (me, le, oe) joins the coded ones
  float me = -INFINITY, le = 0.0f;
  float4 oe = make_float4(0.f, 0.f, 0.f, 0.f);
  if (a.ex.n > 0) exact_partial<DT, D>(a.ex, b, hq, t, bh, sl, red, me, le, oe, c4, part);
  float m = m0;
  for (int s = tid + kMergeThreads; s < S_all; s += kMergeThreads) m = fmaxf(m, m_of(s));
  const float M = block_reduce_256(m, true, red);
  float l = m0 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m0 - M) * l0;
  for (int s = tid + kMergeThreads; s < S_all; s += kMergeThreads) {
    const float ms = m_of(s);
    if (ms != -INFINITY) l += __builtin_amdgcn_exp2f(ms - M) * l_of(s);
  }
  const float Lc = block_reduce_256(l, false, red);
  const float Mx = fmaxf(M, me);
  const float wc = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M - Mx);
  const float we = me == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(me - Mx);
  const float L = wc * Lc + we * le;
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int k = 0; k < NPRE; ++k) {
    const float w = mp[k] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mp[k] - M);
    o.x = __builtin_fmaf(w, op[k].x, o.x);
    o.y = __builtin_fmaf(w, op[k].y, o.y);
    o.z = __builtin_fmaf(w, op[k].z, o.z);
    o.w = __builtin_fmaf(w, op[k].w, o.w);
  }
#pragma unroll 4
  for (int s = part + PARTS * NPRE; s < S_all; s += PARTS) {
    const float ms = m_of(s);
    const float w = ms == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ms - M);
    const float4 v = o_of(s, c4);
    o.x = __builtin_fmaf(w, v.x, o.x);
    o.y = __builtin_fmaf(w, v.y, o.y);
    o.z = __builtin_fmaf(w, v.z, o.z);
    o.w = __builtin_fmaf(w, v.w, o.w);
  }
  o.x = __builtin_fmaf(we, oe.x, wc * o.x);
  o.y = __builtin_fmaf(we, oe.y, wc * o.y);
  o.z = __builtin_fmaf(we, oe.z, wc * o.z);
  o.w = __builtin_fmaf(we, oe.w, wc * o.w);
  part_o[part][c4] = o;
  __syncthreads();
  if (tid < D) {
    const int c = tid;
    float O = 0.0f;
#pragma unroll
    for (int k = 0; k < PARTS; ++k) {
      const float4 v = part_o[k][c >> 2];
      O += (c & 3) == 0 ? v.x : (c & 3) == 1 ? v.y : (c & 3) == 2 ? v.z : v.w;
    }
    store_from_f32<DT>(a.out, ((static_cast<int64_t>(b) * a.Tq + t) * a.Hq + hq) * D + c, O / L);
  }
  if (tid == 0 && a.row_ml != nullptr) {
    a.row_ml[(static_cast<int64_t>(bh) * R + r) * 2] = Mx;
    a.row_ml[(static_cast<int64_t>(bh) * R + r) * 2 + 1] = L;
  }
}

// The merge of a step whose rows have at most NS (<= 32) partials and no exact rows left to attend:
// one wavefront per query row (four rows a workgroup, rows in the order of merge_rows_kernel's
// grid), lane s holding partial s's (m, l) and lane l channels 2 l, 2 l + 1 of every partial's o.
// Every load goes out at once; the row's maximum and sum are wavefront reductions, the weights
// reach every lane by readlane; no LDS and no barrier.  Same partial order and formulas as
// merge_rows_kernel (exact-row partials first).
template <int R, int DT, int NS>
__global__ __launch_bounds__(256) void merge_rows_wave_kernel(MergeArgs a, int n_rows) {
  constexpr int D = 128;
  const int row = static_cast<int>(blockIdx.x) * 4 + static_cast<int>(threadIdx.x >> 6);
  if (row >= n_rows) return;
  const int lane = threadIdx.x & 63;
  const int bh = row / a.R_real, r = row % a.R_real;
  const int S_all = a.S_ex + a.S;
  auto o_ptr = [&](int s) -> const float* {
    return s < a.S_ex ? a.ex_o + ((static_cast<int64_t>(bh) * a.S_ex + s) * R + r) * D
                      : a.ws_o + ((static_cast<int64_t>(bh) * a.S + (s - a.S_ex)) * R + r) * D;
  };
  float ms = -INFINITY, ls = 0.0f;
  if (lane < S_all) {
    ms = lane < a.S_ex ? a.ex_m[(static_cast<int64_t>(bh) * a.S_ex + lane) * R + r]
                       : a.ws_m[(static_cast<int64_t>(bh) * a.S + (lane - a.S_ex)) * R + r];
    ls = lane < a.S_ex ? a.ex_l[(static_cast<int64_t>(bh) * a.S_ex + lane) * R + r]
                       : a.ws_l[(static_cast<int64_t>(bh) * a.S + (lane - a.S_ex)) * R + r];
  }
  float2 ov[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) ov[s] = reinterpret_cast<const float2*>(o_ptr(s < S_all ? s : S_all - 1))[lane];
  const float M = wave_max(ms);
  const float w = ms == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ms - M);
  const float L = wave_sum(w * ls);
  float ox = 0.0f, oy = 0.0f;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const float ws = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), s));   // 0 past S_all
    ox = __builtin_fmaf(ws, ov[s].x, ox);
    oy = __builtin_fmaf(ws, ov[s].y, oy);
  }
  const int b = bh / a.Hkv, h = bh % a.Hkv;
  const int hq = h * a.rep + r / a.Tq, t = r % a.Tq;
  const int64_t o0 = ((static_cast<int64_t>(b) * a.Tq + t) * a.Hq + hq) * D + 2 * lane;
  store_from_f32<DT>(a.out, o0, ox / L);
  store_from_f32<DT>(a.out, o0 + 1, oy / L);
  if (lane == 0 && a.row_ml != nullptr) {
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

// ---- dispatch classes of a one-round launch -------------------------------------------------
// A launch whose blocks are exactly one round with `resident` blocks per CU (one wavefront of each
// per SIMD) fills every CU in `resident` passes over the CUs, and each SIMD's arbiter issues for
// its oldest ready wavefront first: blocks of the first pass progress fastest, those of the last
// slowest, and with equal splits the last class streams alone at the end with too few loads in
// flight.  Such a plan maps blocks class-major (every (b, h) has n_split / classes splits in each
// class) and sizes each split by its class's weight, the rate the classes progress at when they
// share a CU, so the classes finish close together.  Which tokens each wavefront handles is fixed
// by the plan: results stay deterministic.
constexpr int kCUsPerXcd = 32;
// classes of a plan (0: plain mapping, equal splits): blocks go round robin over the 8 XCDs by
// linear id, BH / 8 (b, h) per XCD, each with n_split splits
inline int split_classes(int64_t BH, int64_t n_split, int resident) {
  return (resident == 3 && BH % 8 == 0 && n_split % 3 == 0 && (BH / 8) * (n_split / 3) == kCUsPerXcd) ? 3 : 0;
}
// (b, h) and split of block `id`: XCD-aware (every split of one (b, h) on one XCD, its query rows
// and metadata read through one L2), class-major within the XCD when the plan has classes
__device__ __forceinline__ void class_block_of(int id, int n_split, int classes, int* bh, int* sidx) {
  const int k = id / 8;
  if (classes > 0) {
    const int q = n_split / classes;
    const int cls = k / kCUsPerXcd, slot = k % kCUsPerXcd;
    *bh = id % 8 + 8 * (slot / q);
    *sidx = cls * q + slot % q;
  } else {
    *bh = id % 8 + 8 * (k / n_split);
    *sidx = k % n_split;
  }
}
// sum of the weights of splits [0, s) of a (b, h): w0 / w1 / w2 per class, 1 each without classes
__device__ __forceinline__ int64_t class_weight_before(int s, int n_split, int classes, int w0, int w1, int w2) {
  if (classes <= 0) return s;
  const int q = n_split / classes;
  const int c = s / q;
  const int w[3] = {w0, w1, w2};
  int64_t acc = 0;
  for (int k = 0; k < c && k < 3; ++k) acc += static_cast<int64_t>(q) * w[k];
  // s == n_split (the total) ends on a class boundary: no partial class to add
  return c < 3 ? acc + static_cast<int64_t>(s % q) * w[c] : acc;
}

inline int pow2_rows(int64_t r) {
  int R = 1;
  while (R < r) R <<= 1;
  return R;
}

// launch merge_rows_kernel for a runtime row count R (power of two <= 8) and output dtype
inline int launch_merge_rows(const MergeArgs& a, int R, int BH, int out_dtype, hipStream_t s) {
  const int S_all = a.S_ex + a.S;
  if (a.ex.n == 0 && S_all >= 1 && S_all <= 32) {                // one wavefront per row
    const int n_rows = BH * a.R_real;
    const dim3 wgrid(static_cast<unsigned>((n_rows + 3) / 4));
#define KVQ_MW_N(R_, DT_, N_) hipLaunchKernelGGL((merge_rows_wave_kernel<R_, DT_, N_>), wgrid, dim3(256), 0, s, a, n_rows)
#define KVQ_MW_L(R_, DT_)                                      \
  do {                                                         \
    if (S_all <= 8) KVQ_MW_N(R_, DT_, 8);                      \
    else if (S_all <= 16) KVQ_MW_N(R_, DT_, 16);               \
    else KVQ_MW_N(R_, DT_, 32);                                \
  } while (0)
#define KVQ_MW_R(DT_)                              \
  switch (R) {                                     \
    case 1: KVQ_MW_L(1, DT_); break;               \
    case 2: KVQ_MW_L(2, DT_); break;               \
    case 4: KVQ_MW_L(4, DT_); break;               \
    default: KVQ_MW_L(8, DT_); break;              \
  }
    switch (out_dtype) {
      case KVQ_F32: KVQ_MW_R(KVQ_F32) break;
      case KVQ_F16: KVQ_MW_R(KVQ_F16) break;
      default: KVQ_MW_R(KVQ_BF16) break;
    }
#undef KVQ_MW_R
#undef KVQ_MW_L
#undef KVQ_MW_N
    KVQ_LAUNCH_CHECK("merge_rows");
    return KVQ_OK;
  }
  const dim3 grid(static_cast<unsigned>(BH) * a.R_real);
  constexpr int kParts128 = kMergeThreads / 32;    // partial slices of the D = 128 merge
  const int per = (a.S_ex + a.S + kParts128 - 1) / kParts128;
#define KVQ_MERGE_N(R_, DT_, N_) hipLaunchKernelGGL((merge_rows_kernel<R_, DT_, 128, N_>), grid, dim3(kMergeThreads), 0, s, a)
#define KVQ_MERGE_L(R_, DT_)                                   \
  do {                                                         \
    if (per <= 1) KVQ_MERGE_N(R_, DT_, 1);                     \
    else if (per <= 4) KVQ_MERGE_N(R_, DT_, 4);                \
    else KVQ_MERGE_N(R_, DT_, 16);                             \
  } while (0)
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
#undef KVQ_MERGE_N
  KVQ_LAUNCH_CHECK("merge_rows");
  return KVQ_OK;
}

}  // namespace
}  // namespace kvq
