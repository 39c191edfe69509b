// SnapKV scores on the device (gfx950): the eviction scores of STRATA_KV.py:932-954 (snapkv_scores).
//
// What it computes, per (b, KV head h): the last `w` context queries of each of the rep query heads
// of h (rows r = (head, i), position H - w + i) attend causally to the keys [0, H) (fp32 softmax of
// scaling * q.k); the probabilities of the keys j < H - w are averaged over the rep * w rows
// (mean over the window queries, then over the heads of the group), pooled along j by
// avg_pool1d(kernel, padding kernel / 2, zeros counted), and the w window columns get the global
// maximum + 1.  Output (B, Hkv, H) float32.  Means over rows and pooling along keys are linear along
// different axes, so they are taken in the order that needs one column sum per key.
//
// Passes (one stream, no host synchronisation):
//   1. snap_stats: per (bh, row group, key split) the logits of the group's rows against the split's
//      keys on the matrix cores (v_mfma_f32_16x16x32_{bf16,f16}; fp32 inputs as fp16 hi + lo parts,
//      three products), each lane keeping an online (max, sum) of its rows in base 2; partials out.
//   2. snap_rows: each row's (max, 1 / sum) from the partials.
//   3. snap_cols: per (bh, row group, 256-key chunk) the logits again, probabilities normalised by the
//      row statistics and summed over the group's rows on the way out of the accumulators.
//   4. snap_pool: sum of the row groups' column sums / (rep * w), the pooling window through LDS,
//      and a maximum per block.
//   5. snap_window: the global maximum + 1 into the w window columns.
// Matrix-core mapping (mfma_common.hpp): A = 16 keys x 32 channels (lane l: key l%16, channels
// 8(l/16)..+7 of the k-step), B = 32 channels x 16 query rows, D lane l register i = logit of key
// 4(l/16) + i for row l%16.
#include <algorithm>

#include "common.hpp"
#include "mfma_common.hpp"
#include "row_tiles.hpp"

namespace kvq {
namespace {

constexpr int kSnapThreads = 256;
constexpr int kSnapWaves = 4;
constexpr int kSnapChunk = 256;       // keys of a column-sum workgroup (16 tiles)
constexpr int kSnapPool = 1024;       // keys of a pooling workgroup
constexpr int kSnapMaxPad = 32;       // largest pooling half-width
constexpr float kSnapLog2e = 1.4426950408889634f;

template <int DT>
struct SnapTraits {
  static constexpr int NH = TileOps<DT>::NH;                // operand parts (fp32: fp16 hi, lo)
  static constexpr int NBW = DT == KVQ_F32 ? 2 : 4;         // row blocks of 16 per wavefront
  static constexpr int RG = 16 * NBW * kSnapWaves;          // rows per workgroup
  static constexpr int ESZ = TileOps<DT>::ESZ;
};

struct SnapParams {
  const void* q;
  int64_t q_sb, q_sh, q_st;             // window query rows: (b, head, i) at b*q_sb + head*q_sh + i*q_st
  const void* k;
  int64_t k_sb, k_sh, k_st;             // keys: (b, h, j) at b*k_sb + h*k_sh + j*k_st
  int Hkv, rep, w, H, rows, n_rg, n_split, split_keys, n_chunk, n_pool, kernel;
  float qscale;                         // scaling * log2(e)
  float inv_count;                      // 1 / (rep * w)
  float* part_m;                        // (BH, n_split, rows)
  float* part_l;
  float* row_m;                         // (BH, rows)
  float* row_il;                        // (BH, rows): 1 / row sum
  float* colsum;                        // (BH, n_rg, H - w)
  float* blockmax;                      // (BH, n_pool)
  float* out;                           // (BH, H)
  // fp32 rows: the powers of two of the query rows and the keys (rows_scale_kernel, row_tiles.hpp)
  const float* xs;
};

// the power of two of fp32 view i (0: query rows, 1: keys); 16-bit rows are exact operands: 1
template <int DT>
__device__ __forceinline__ float snap_xs(const SnapParams& p, int i) {
  if constexpr (DT == KVQ_F32) return p.xs[i];
  else return 1.0f;
}

// query operands of this wavefront's row blocks and the position of each lane's row (-1: no row)
template <int DT>
__device__ __forceinline__ void load_queries(const SnapParams& p, int b, int h, int rg, int wave, int g, int n,
                                             u32x4 (&qop)[SnapTraits<DT>::NBW][4][SnapTraits<DT>::NH],
                                             int (&rowpos)[SnapTraits<DT>::NBW], int (&row)[SnapTraits<DT>::NBW]) {
  using T = SnapTraits<DT>;
#pragma unroll
  for (int bw = 0; bw < T::NBW; ++bw) {
    const int r = rg * T::RG + (wave * T::NBW + bw) * 16 + n;
    row[bw] = r;
    if (r < p.rows) {
      const int hq = h * p.rep + r / p.w, i = r % p.w;
      const int64_t base = static_cast<int64_t>(b) * p.q_sb + static_cast<int64_t>(hq) * p.q_sh +
                           static_cast<int64_t>(i) * p.q_st;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) load_op<DT>(p.q, base + 32 * ks + 8 * g, qop[bw][ks], snap_xs<DT>(p, 0));
      rowpos[bw] = p.H - p.w + i;
    } else {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int hh = 0; hh < T::NH; ++hh) qop[bw][ks][hh] = u32x4{0u, 0u, 0u, 0u};
      rowpos[bw] = -1;
    }
  }
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t key_rsrc(const SnapParams& p, int b, int h, int esz) {
  const char* base = static_cast<const char*>(p.k) +
                     (static_cast<int64_t>(b) * p.k_sb + static_cast<int64_t>(h) * p.k_sh) * esz;
  return make_rsrc(base, static_cast<uint32_t>((static_cast<int64_t>(p.H - 1) * p.k_st + 128) * esz));
}

// the A/B operand registers of key kj (channels 32 ks + 8 g .. + 7 of each k-step); keys past the
// resource's range read as zeros
template <int DT>
__device__ __forceinline__ void load_keys(const __amdgpu_buffer_rsrc_t& rk, const SnapParams& p, int kj, int g,
                                          u32x4 (&kop)[4][SnapTraits<DT>::NH]) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    load_op_buf<DT>(rk, static_cast<int>((static_cast<int64_t>(kj) * p.k_st + 32 * ks + 8 * g) * SnapTraits<DT>::ESZ),
                    kop[ks], snap_xs<DT>(p, 1));
}

template <int DT>
__global__ __launch_bounds__(kSnapThreads) void snap_stats(SnapParams p) {
  using T = SnapTraits<DT>;
  const int wave = threadIdx.x / 64, l = threadIdx.x % 64, g = l >> 4, n = l & 15;
  int id = blockIdx.x;
  const int s = id % p.n_split;
  id /= p.n_split;
  const int rg = id % p.n_rg, bh = id / p.n_rg;
  const int b = bh / p.Hkv, h = bh % p.Hkv;
  u32x4 qop[T::NBW][4][T::NH];
  int rowpos[T::NBW], row[T::NBW];
  load_queries<DT>(p, b, h, rg, wave, g, n, qop, rowpos, row);
  float m[T::NBW], ls[T::NBW];
#pragma unroll
  for (int bw = 0; bw < T::NBW; ++bw) {
    m[bw] = -INFINITY;
    ls[bw] = 0.0f;
  }
  const __amdgpu_buffer_rsrc_t rk = key_rsrc(p, b, h, T::ESZ);
  const int k0 = s * p.split_keys, k1 = min(k0 + p.split_keys, p.H);
  const float qsc = p.qscale / (snap_xs<DT>(p, 0) * snap_xs<DT>(p, 1));   // logit scale of the scaled rows
  auto stat_tile = [&](int t0, const u32x4 (&kop)[4][T::NH]) {
#pragma unroll
    for (int bw = 0; bw < T::NBW; ++bw) {
      const f32x4 acc = tile_dots<DT, SnapTraits<DT>::NH, SnapTraits<DT>::NH>(kop, qop[bw]);
      float sv[4];
      float mt = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = t0 + 4 * g + i;
        sv[i] = (j < k1 && j <= rowpos[bw]) ? acc[i] * qsc : -INFINITY;
        mt = fmaxf(mt, sv[i]);
      }
      if (mt > m[bw]) {
        ls[bw] *= __builtin_amdgcn_exp2f(m[bw] - mt);
        m[bw] = mt;
      }
      if (m[bw] != -INFINITY) {
#pragma unroll
        for (int i = 0; i < 4; ++i) ls[bw] += __builtin_amdgcn_exp2f(sv[i] - m[bw]);
      }
    }
  };
  // two key tiles in registers used in turn: the next tile's loads are issued before the current
  // one is computed (tiles past the split are loaded -- keys past H read as zeros -- never used)
  if (k0 < k1) {
    u32x4 ka[4][T::NH], kb[4][T::NH];
    load_keys<DT>(rk, p, k0 + n, g, ka);
    for (int t0 = k0;; t0 += 32) {
      load_keys<DT>(rk, p, t0 + 16 + n, g, kb);
      stat_tile(t0, ka);
      if (t0 + 16 >= k1) break;
      load_keys<DT>(rk, p, t0 + 32 + n, g, ka);
      stat_tile(t0 + 16, kb);
      if (t0 + 32 >= k1) break;
    }
  }
  // the four lanes of a row (xor 16, xor 32) hold disjoint keys of it
#pragma unroll
  for (int bw = 0; bw < T::NBW; ++bw) {
    const float M = xmax32(xmax16(m[bw]));
    const float part = (M == -INFINITY || m[bw] == -INFINITY) ? 0.0f : ls[bw] * __builtin_amdgcn_exp2f(m[bw] - M);
    const float L = xsum32(xsum16(part));
    if (g == 0 && row[bw] < p.rows) {
      const int64_t o = (static_cast<int64_t>(bh) * p.n_split + s) * p.rows + row[bw];
      p.part_m[o] = M;
      p.part_l[o] = L;
    }
  }
}

__global__ __launch_bounds__(kSnapThreads) void snap_rows(SnapParams p, int64_t n_rows_all) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kSnapThreads + threadIdx.x;
  if (t >= n_rows_all) return;
  const int64_t bh = t / p.rows, r = t % p.rows;
  float M = -INFINITY;
  for (int s = 0; s < p.n_split; ++s) M = fmaxf(M, p.part_m[(bh * p.n_split + s) * p.rows + r]);
  float L = 0.0f;
  for (int s = 0; s < p.n_split; ++s) {
    const float ms = p.part_m[(bh * p.n_split + s) * p.rows + r];
    if (ms != -INFINITY) L += p.part_l[(bh * p.n_split + s) * p.rows + r] * __builtin_amdgcn_exp2f(ms - M);
  }
  p.row_m[t] = M;
  p.row_il[t] = 1.0f / L;                 // key 0 is visible to every row: L >= 1
}

template <int DT>
__global__ __launch_bounds__(kSnapThreads) void snap_cols(SnapParams p) {
  using T = SnapTraits<DT>;
  __shared__ float cols[kSnapWaves][kSnapChunk];
  const int wave = threadIdx.x / 64, l = threadIdx.x % 64, g = l >> 4, n = l & 15;
  int id = blockIdx.x;
  const int c = id % p.n_chunk;
  id /= p.n_chunk;
  const int rg = id % p.n_rg, bh = id / p.n_rg;
  const int b = bh / p.Hkv, h = bh % p.Hkv;
  u32x4 qop[T::NBW][4][T::NH];
  int rowpos[T::NBW], row[T::NBW];
  load_queries<DT>(p, b, h, rg, wave, g, n, qop, rowpos, row);
  // operand roles swapped against snap_stats (A = query rows, B = keys): D lane (g, n) register i
  // is the logit of row 16 (wave NBW + bw) + 4 g + i against key t0 + n, so a column sum over the
  // wavefront's rows is a register sum and two cross-lane steps per tile.  Row statistics per
  // register: the rows of lane group g.
  float rm[T::NBW][4], ril[T::NBW][4];
#pragma unroll
  for (int bw = 0; bw < T::NBW; ++bw) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rg * T::RG + (wave * T::NBW + bw) * 16 + 4 * g + i;
      const bool ok = r < p.rows;
      rm[bw][i] = ok ? p.row_m[static_cast<int64_t>(bh) * p.rows + r] : 0.0f;
      ril[bw][i] = ok ? p.row_il[static_cast<int64_t>(bh) * p.rows + r] : 0.0f;
    }
  }
  const __amdgpu_buffer_rsrc_t rk = key_rsrc(p, b, h, T::ESZ);
  const int nc = p.H - p.w;                 // scored keys: every window row sees all of them
  const int c0 = c * kSnapChunk;
  const float qsc = p.qscale / (snap_xs<DT>(p, 0) * snap_xs<DT>(p, 1));   // logit scale of the scaled rows
  auto col_tile = [&](int tt, const u32x4 (&kop)[4][T::NH]) {
    const int t0 = c0 + 16 * tt;
    float colv = 0.0f;
    if (t0 < nc) {
#pragma unroll
      for (int bw = 0; bw < T::NBW; ++bw) {
        const f32x4 acc = tile_dots<DT, SnapTraits<DT>::NH, SnapTraits<DT>::NH>(qop[bw], kop);
#pragma unroll
        for (int i = 0; i < 4; ++i) colv += __builtin_amdgcn_exp2f(acc[i] * qsc - rm[bw][i]) * ril[bw][i];
      }
    }
    // the four lane groups hold disjoint rows of key t0 + n
    colv = xsum32(xsum16(colv));
    if (g == 0) cols[wave][16 * tt + n] = colv;
  };
  // two key tiles in registers used in turn, the next one's loads issued first
  {
    u32x4 ka[4][T::NH], kb[4][T::NH];
    load_keys<DT>(rk, p, c0 + n, g, ka);
    for (int tt = 0; tt < kSnapChunk / 16; tt += 2) {
      load_keys<DT>(rk, p, c0 + 16 * (tt + 1) + n, g, kb);
      col_tile(tt, ka);
      if (tt + 2 < kSnapChunk / 16) load_keys<DT>(rk, p, c0 + 16 * (tt + 2) + n, g, ka);
      col_tile(tt + 1, kb);
    }
  }
  __syncthreads();
  const int j = c0 + threadIdx.x;
  if (j < nc) {
    const float v = (cols[0][threadIdx.x] + cols[1][threadIdx.x]) + (cols[2][threadIdx.x] + cols[3][threadIdx.x]);
    p.colsum[(static_cast<int64_t>(bh) * p.n_rg + rg) * nc + j] = v;
  }
}

__global__ __launch_bounds__(kSnapThreads) void snap_pool(SnapParams p) {
  __shared__ float sc[kSnapPool + 2 * kSnapMaxPad];
  __shared__ float red[kSnapWaves];
  const int bh = blockIdx.x / p.n_pool, pc = blockIdx.x % p.n_pool;
  const int nc = p.H - p.w;
  const int pad = p.kernel / 2;
  const int j0 = pc * kSnapPool;
  const float* cs = p.colsum + static_cast<int64_t>(bh) * p.n_rg * nc;
  // mean probability of keys j0 - pad .. j0 + kSnapPool + pad (zero outside [0, nc))
  for (int t = threadIdx.x; t < kSnapPool + 2 * pad; t += kSnapThreads) {
    const int j = j0 - pad + t;
    float v = 0.0f;
    if (j >= 0 && j < nc) {
      for (int r = 0; r < p.n_rg; ++r) v += cs[static_cast<int64_t>(r) * nc + j];
      v *= p.inv_count;
    }
    sc[t] = v;
  }
  __syncthreads();
  const float inv_k = 1.0f / static_cast<float>(p.kernel);
  float mx = -INFINITY;
  for (int t = threadIdx.x; t < kSnapPool; t += kSnapThreads) {
    const int j = j0 + t;
    if (j < nc) {
      float v = 0.0f;
      for (int e = 0; e < p.kernel; ++e) v += sc[t + e];
      v *= inv_k;
      p.out[static_cast<int64_t>(bh) * p.H + j] = v;
      mx = fmaxf(mx, v);
    }
  }
  mx = wave_max(mx);
  if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = mx;
  __syncthreads();
  if (threadIdx.x == 0)
    p.blockmax[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__global__ __launch_bounds__(kSnapThreads) void snap_window(SnapParams p, int n_blocks) {
  __shared__ float red[kSnapWaves];
  float mx = -INFINITY;
  for (int t = threadIdx.x; t < n_blocks; t += kSnapThreads) mx = fmaxf(mx, p.blockmax[t]);
  mx = wave_max(mx);
  if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = mx;
  __syncthreads();
  const float top = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])) + 1.0f;
  for (int t = threadIdx.x; t < p.w; t += kSnapThreads)
    p.out[static_cast<int64_t>(blockIdx.x) * p.H + (p.H - p.w) + t] = top;
}

struct SnapPlan {
  int n_rg, n_split, split_keys, n_chunk, n_pool;
};

SnapPlan snap_plan(int64_t BH, int64_t rows, int64_t w, int64_t H, int dtype) {
  SnapPlan sp{};
  const int64_t RG = dtype == KVQ_F32 ? SnapTraits<KVQ_F32>::RG : SnapTraits<KVQ_BF16>::RG;
  sp.n_rg = static_cast<int>((rows + RG - 1) / RG);
  // about 1024 workgroups of key splits, whole 16-key tiles
  const int64_t want = std::max<int64_t>(1, (1024 + BH * sp.n_rg - 1) / (BH * sp.n_rg));
  const int64_t tiles = (H + 15) / 16;
  const int64_t ns = std::min<int64_t>(want, tiles);
  sp.split_keys = static_cast<int>(((tiles + ns - 1) / ns) * 16);
  sp.n_split = static_cast<int>((H + sp.split_keys - 1) / sp.split_keys);
  sp.n_chunk = static_cast<int>((H - w + kSnapChunk - 1) / kSnapChunk);
  sp.n_pool = static_cast<int>((H - w + kSnapPool - 1) / kSnapPool);
  return sp;
}

int64_t snap_ws(int64_t BH, int64_t rows, int64_t w, int64_t H, const SnapPlan& sp, int dtype) {
  return 2 * BH * sp.n_split * rows + 2 * BH * rows + BH * sp.n_rg * (H - w) + BH * sp.n_pool +
         (dtype == KVQ_F32 ? kAmaxFloats : 0);
}

}  // namespace
}  // namespace kvq

using namespace kvq;

extern "C" int64_t kvq_snapkv_scores_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t window, int64_t H,
                                               int dtype) {
  if (B <= 0 || Hkv <= 0 || Hq % Hkv != 0 || window <= 0 || H <= window || !valid_dtype(dtype)) return -1;
  const int64_t rows = (Hq / Hkv) * window;
  const SnapPlan sp = snap_plan(B * Hkv, rows, window, H, dtype);
  return snap_ws(B * Hkv, rows, window, H, sp, dtype);
}

extern "C" int kvq_snapkv_scores(const void* q, int dtype, int64_t q_sb, int64_t q_sh, int64_t q_st, const void* k,
                                 int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t B, int64_t Hq, int64_t Hkv,
                                 int64_t d, int64_t window, int64_t H, float scaling, int kernel, float* out,
                                 float* workspace, int64_t workspace_floats, void* stream) {
  KVQ_REQUIRE(valid_dtype(dtype), "kvq_snapkv_scores: bad dtype");
  KVQ_REQUIRE(d == 128, "kvq_snapkv_scores: head_dim must be 128");
  KVQ_REQUIRE(B > 0 && Hkv > 0 && Hq % Hkv == 0 && B * Hkv < 65536, "kvq_snapkv_scores: bad head counts");
  KVQ_REQUIRE(window > 0 && H > window && H < (1LL << 28), "kvq_snapkv_scores: need 0 < window < H");
  KVQ_REQUIRE(kernel >= 1 && kernel % 2 == 1 && kernel / 2 <= kSnapMaxPad,
              "kvq_snapkv_scores: pooling kernel must be odd and at most %d", 2 * kSnapMaxPad + 1);
  KVQ_REQUIRE(q && k && out && workspace, "kvq_snapkv_scores: null pointer");
  const int esz = dtype == KVQ_F32 ? 4 : 2;
  KVQ_REQUIRE((q_sb * esz) % 16 == 0 && (q_sh * esz) % 16 == 0 && (q_st * esz) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(q) % 16 == 0,
              "kvq_snapkv_scores: query rows must be 16-byte aligned");
  KVQ_REQUIRE((k_sb * esz) % 16 == 0 && (k_sh * esz) % 16 == 0 && (k_st * esz) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(k) % 16 == 0 && k_st >= 128,
              "kvq_snapkv_scores: key rows must be 16-byte aligned and not overlap");
  // byte offsets of the last tile's keys (up to H + 15 rows) stay below 2^31
  KVQ_REQUIRE((H + 16) * k_st * esz < (1LL << 31), "kvq_snapkv_scores: one head's keys must span < 2 GiB");
  const int64_t BH = B * Hkv, rows = (Hq / Hkv) * window;
  const SnapPlan sp = snap_plan(BH, rows, window, H, dtype);
  const int64_t need = snap_ws(BH, rows, window, H, sp, dtype);
  KVQ_REQUIRE(workspace_floats >= need, "kvq_snapkv_scores: workspace too small (%lld < %lld floats)",
              (long long)workspace_floats, (long long)need);
  SnapParams p{};
  p.q = q; p.q_sb = q_sb; p.q_sh = q_sh; p.q_st = q_st;
  p.k = k; p.k_sb = k_sb; p.k_sh = k_sh; p.k_st = k_st;
  p.Hkv = static_cast<int>(Hkv); p.rep = static_cast<int>(Hq / Hkv); p.w = static_cast<int>(window);
  p.H = static_cast<int>(H); p.rows = static_cast<int>(rows);
  p.n_rg = sp.n_rg; p.n_split = sp.n_split; p.split_keys = sp.split_keys; p.n_chunk = sp.n_chunk;
  p.n_pool = sp.n_pool; p.kernel = kernel;
  p.qscale = scaling * kSnapLog2e;
  p.inv_count = 1.0f / static_cast<float>(rows);
  float* ws = workspace;
  p.part_m = ws; ws += BH * sp.n_split * rows;
  p.part_l = ws; ws += BH * sp.n_split * rows;
  p.row_m = ws; ws += BH * rows;
  p.row_il = ws; ws += BH * rows;
  p.colsum = ws; ws += BH * sp.n_rg * (H - window);
  p.blockmax = ws; ws += BH * sp.n_pool;
  p.out = out;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 blk(kSnapThreads);
  if (dtype == KVQ_F32) {
    // the powers of two that bring the window's query rows and the keys into the fp16 parts' range
    p.xs = ws + kAmaxViews * kAmaxBlocks;
    const RowView views[2] = {
        RowView{static_cast<const float*>(q), static_cast<int>(B), static_cast<int>(Hq), static_cast<int>(window),
                q_sb, q_sh, q_st},
        RowView{static_cast<const float*>(k), static_cast<int>(B), static_cast<int>(Hkv), static_cast<int>(H), k_sb,
                k_sh, k_st}};
    launch_rows_scales(views, 2, ws, const_cast<float*>(p.xs), s);
    KVQ_LAUNCH_CHECK("kvq_snapkv_scores(fp32 scales)");
  }
  KVQ_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((snap_stats<DT_>), dim3(BH * sp.n_rg * sp.n_split), blk, 0, s, p));
  KVQ_LAUNCH_CHECK("kvq_snapkv_scores(stats)");
  hipLaunchKernelGGL(snap_rows, dim3((BH * rows + kSnapThreads - 1) / kSnapThreads), blk, 0, s, p, BH * rows);
  KVQ_LAUNCH_CHECK("kvq_snapkv_scores(rows)");
  KVQ_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((snap_cols<DT_>), dim3(BH * sp.n_rg * sp.n_chunk), blk, 0, s, p));
  KVQ_LAUNCH_CHECK("kvq_snapkv_scores(cols)");
  hipLaunchKernelGGL(snap_pool, dim3(BH * sp.n_pool), blk, 0, s, p);
  KVQ_LAUNCH_CHECK("kvq_snapkv_scores(pool)");
  hipLaunchKernelGGL(snap_window, dim3(BH), blk, 0, s, p, static_cast<int>(BH * sp.n_pool));
  KVQ_LAUNCH_CHECK("kvq_snapkv_scores(window)");
  return KVQ_OK;
}
