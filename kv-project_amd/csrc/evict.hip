// Eviction: top-k retention of accumulated scores, and the gather + dequantise of the retained
// rows that the retained-set decode reads.
//
// Top-k (SnapKV-style retention, STRATA_KV.py:975 topk, 1022-1023 position order): one block of
// 1024 threads per (b, h) row of scores.  A radix select over order-preserving uint32 keys of the
// fp32 scores (8 bits per pass, LDS histograms) finds the k-th largest key T and how many keys
// equal to T are kept; the retained positions are then written in increasing order.  Among keys
// equal to T the lowest positions are kept (torch.topk leaves that order unspecified).  Rows of up
// to 65536 scores take topk_retain_rows_kernel (row in registers, a 12-bit float-bucket first
// pass, scan-ordered output); longer rows take topk_retain_kernel.
#include "common.hpp"
#include "mfma_common.hpp"

namespace kvq {
namespace {

constexpr int kTopkThreads = 1024;

__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Exclusive prefix sum of v over the block (1024 threads); *total receives the sum.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* wave_sums, uint32_t* total) {
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) wave_sums[wave] = x;
  __syncthreads();
  if (wave == 0) {
    uint32_t w = lane < kTopkThreads / 64 ? wave_sums[lane] : 0u;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const uint32_t y = __shfl_up(w, o, 64);
      if (lane >= o) w += y;
    }
    if (lane < kTopkThreads / 64) wave_sums[16 + lane] = w;       // inclusive wave prefix
  }
  __syncthreads();
  const uint32_t before = (wave > 0 ? wave_sums[16 + wave - 1] : 0u) + x - v;
  *total = wave_sums[16 + kTopkThreads / 64 - 1];
  __syncthreads();                                                 // wave_sums reusable after return
  return before;
}

__global__ __launch_bounds__(kTopkThreads) void topk_retain_kernel(const float* __restrict__ scores,
                                                                   int64_t n, int64_t scores_bh, int64_t k,
                                                                   int32_t* __restrict__ idx, int64_t idx_bh) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t wave_sums[32];
  __shared__ uint32_t sh_prefix, sh_krem;
  const int tid = threadIdx.x;
  const float* s = scores + static_cast<int64_t>(blockIdx.x) * scores_bh;
  int32_t* out = idx + static_cast<int64_t>(blockIdx.x) * idx_bh;
  uint32_t prefix = 0, mask = 0, krem = static_cast<uint32_t>(k);
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
    for (int64_t i = tid; i < n; i += kTopkThreads) {
      const uint32_t u = order_key(s[i]);
      if ((u & mask) == prefix) atomicAdd(&hist[(u >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid == 0) {
      uint32_t acc = 0;
      for (int b = 255; b >= 0; --b) {
        if (acc + hist[b] >= krem) {
          sh_prefix = prefix | (static_cast<uint32_t>(b) << shift);
          sh_krem = krem - acc;
          break;
        }
        acc += hist[b];
      }
    }
    __syncthreads();
    prefix = sh_prefix;
    krem = sh_krem;
    mask |= 0xFFu << shift;
  }
  // prefix = key of the k-th largest score; krem = how many keys equal to it are retained
  const int64_t per = (n + kTopkThreads - 1) / kTopkThreads;
  const int64_t lo = min<int64_t>(n, tid * per), hi = min<int64_t>(n, lo + per);
  uint32_t c_gt = 0, c_eq = 0;
  for (int64_t i = lo; i < hi; ++i) {
    const uint32_t u = order_key(s[i]);
    c_gt += u > prefix;
    c_eq += u == prefix;
  }
  uint32_t total;
  const uint32_t eq_before = block_exclusive_scan(c_eq, wave_sums, &total);
  const uint32_t take_eq = eq_before >= krem ? 0u : min(c_eq, krem - eq_before);
  uint32_t off = block_exclusive_scan(c_gt + take_eq, wave_sums, &total);
  uint32_t taken = 0;
  for (int64_t i = lo; i < hi; ++i) {
    const uint32_t u = order_key(s[i]);
    const bool eq = u == prefix;
    if (u > prefix || (eq && taken < take_eq)) out[off++] = static_cast<int32_t>(i);
    taken += eq;
  }
}

// Rows of at most kTopkSlots * 1024 scores (topk_retain_rows_kernel): thread t holds elements
// 64 t .. 64 t + 63, read once with 16-byte loads and kept in registers as order keys.
//   * The keys are taken relative to the row's smallest key (v = key - min; the order is kept) and
//     the first pass bins the top 12 of the bits the row's key range spans: one 4096-bin LDS
//     histogram of v >> s1 with s1 = max(0, bits(max - min) - 12).  The bins cover the scores
//     the row actually holds, so a row whose scores share their sign and most of their exponent
//     (softmax probabilities do) still spreads over the bins instead of colliding in a few hot
//     ones; a suffix scan over the bins (one block scan) finds the bin of the k-th largest key.
//   * The remaining s1 bits by 8-bit passes (the last one narrower) over the keys still matching
//     the prefix (per-wavefront 256-bin histograms).
//   * Output in position order: per-thread bit masks of the kept slots; one block scan of the
//     tie counts (ties beyond the kept ones dropped, lowest positions first) and one of the kept
//     counts gives every thread its output offset.
constexpr int kTopkSlots = 64;
constexpr int kTopkBins1 = 4096;

__global__ __launch_bounds__(kTopkThreads) void topk_retain_rows_kernel(const float* __restrict__ scores,
                                                                        int n, int64_t scores_bh, int k,
                                                                        int32_t* __restrict__ idx, int64_t idx_bh) {
  constexpr int NW = kTopkThreads / 64;
  __shared__ uint32_t hist1[kTopkBins1];
  __shared__ uint32_t hist[NW][256];
  __shared__ uint32_t wave_sums[32];
  __shared__ uint32_t sh_prefix, sh_krem;
  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const float* s = scores + static_cast<int64_t>(blockIdx.x) * scores_bh;
  int32_t* out = idx + static_cast<int64_t>(blockIdx.x) * idx_bh;
  const int base = tid * kTopkSlots;
  const int nv = min(max(n - base, 0), kTopkSlots);            // slots of this thread that exist
  // buffer loads past n read zero; every load in flight together
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(s, static_cast<uint32_t>(n) * 4u);
  uint32_t u[kTopkSlots];
#pragma unroll
  for (int j = 0; j < kTopkSlots / 4; ++j) {
    const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rs, base * 4 + 16 * j, 0, 0);
    u[4 * j] = w[0];
    u[4 * j + 1] = w[1];
    u[4 * j + 2] = w[2];
    u[4 * j + 3] = w[3];
  }
  // a 16-byte load that straddles n may be range-checked as a whole: the thread holding the
  // row's ragged last chunk (n % 4 != 0) reloads that chunk with 4-byte loads
  if ((n & 3) != 0 && base <= n - 1 && n - 1 < base + kTopkSlots) {
    const int jb = (n - 1 - base) >> 2;
#pragma unroll
    for (int j = 0; j < kTopkSlots / 4; ++j) {
      if (j == jb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) u[4 * j + i] = __builtin_amdgcn_raw_buffer_load_b32(rs, (base + 4 * j + i) * 4, 0, 0);
      }
    }
  }
  uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
#pragma unroll
  for (int e = 0; e < kTopkSlots; ++e) {
    u[e] = order_key(__uint_as_float(u[e]));
    if (e < nv) {
      kmin = min(kmin, u[e]);
      kmax = max(kmax, u[e]);
    }
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    kmin = min(kmin, static_cast<uint32_t>(__shfl_xor(static_cast<int>(kmin), o, 64)));
    kmax = max(kmax, static_cast<uint32_t>(__shfl_xor(static_cast<int>(kmax), o, 64)));
  }
  if (lane == 0) {
    wave_sums[wave] = kmin;
    wave_sums[16 + wave] = kmax;
  }
  for (int bn = tid; bn < kTopkBins1; bn += kTopkThreads) hist1[bn] = 0u;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    kmin = min(kmin, wave_sums[w]);
    kmax = max(kmax, wave_sums[16 + w]);
  }
  // every valid key lies in [kmin, kmax] (kmin <= kmax: a row holds at least one score)
  const int span = 32 - __builtin_clz(kmax - kmin | 1u);           // bits of max - min (>= 1)
  const int s1 = max(0, span - 12);
#pragma unroll
  for (int e = 0; e < kTopkSlots; ++e) {
    u[e] -= kmin;                                                  // wraps for e >= nv: never read
    if (e < nv) atomicAdd(&hist1[u[e] >> s1], 1u);
  }
  __syncthreads();
  // thread t owns bins 4095 - 4t - i (i = 0..3, descending); keys in higher bins come first
  uint32_t c4[4], tot = 0u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    c4[i] = hist1[kTopkBins1 - 1 - 4 * tid - i];
    tot += c4[i];
  }
  uint32_t total;
  uint32_t run = block_exclusive_scan(tot, wave_sums, &total);
  const uint32_t kk = static_cast<uint32_t>(k);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (c4[i] > 0u && run < kk && run + c4[i] >= kk) {
      sh_prefix = static_cast<uint32_t>(kTopkBins1 - 1 - 4 * tid - i) << s1;
      sh_krem = kk - run;
    }
    run += c4[i];
  }
  __syncthreads();
  uint32_t prefix = sh_prefix, krem = sh_krem;
  uint32_t mask = 0xFFFFFFFFu << s1;
  int top = s1 - 1;
  while (top >= 0) {
    const int width = min(8, top + 1);
    const int shift = top - width + 1;
    const uint32_t dmask = (1u << width) - 1u;
    for (int bn = lane; bn < 256; bn += 64) hist[wave][bn] = 0u;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < kTopkSlots; ++e) {
      if (e < nv && (u[e] & mask) == prefix) atomicAdd(&hist[wave][(u[e] >> shift) & dmask], 1u);
    }
    __syncthreads();
    // thread t < 256 holds bin 255 - t: its total and the inclusive sum over the bins above it
    uint32_t bt = 0u;
    if (tid < 256) {
      for (int w = 0; w < NW; ++w) bt += hist[w][255 - tid];
    }
    uint32_t x = bt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (tid < 256 && lane == 63) wave_sums[wave] = x;
    __syncthreads();
    if (tid < 256) {
      uint32_t before = 0u;
      for (int w = 0; w < wave; ++w) before += wave_sums[w];
      const uint32_t incl = before + x, excl = incl - bt;
      if (bt > 0u && excl < krem && incl >= krem) {
        sh_prefix = prefix | (static_cast<uint32_t>(255 - tid) << shift);
        sh_krem = krem - excl;
      }
    }
    __syncthreads();
    prefix = sh_prefix;
    krem = sh_krem;
    mask |= dmask << shift;
    top = shift - 1;
  }
  // prefix = key of the k-th largest score (relative to kmin); krem = how many keys equal to it
  // are kept (those at the lowest positions)
  uint64_t gt = 0, eq = 0;
#pragma unroll
  for (int e = 0; e < kTopkSlots; ++e) {
    gt |= static_cast<uint64_t>(e < nv && u[e] > prefix) << e;
    eq |= static_cast<uint64_t>(e < nv && u[e] == prefix) << e;
  }
  uint32_t total_eq;
  const uint32_t eq_before = block_exclusive_scan(static_cast<uint32_t>(__builtin_popcountll(eq)), wave_sums, &total_eq);
  uint64_t sel = gt;
  if (total_eq == krem) {
    sel |= eq;
  } else {
    uint32_t r = eq_before;
    for (uint64_t m = eq; m != 0 && r < krem; m &= m - 1, ++r) sel |= m & (~m + 1);
  }
  uint32_t off = block_exclusive_scan(static_cast<uint32_t>(__builtin_popcountll(sel)), wave_sums, &total);
  for (uint64_t m = sel; m != 0; m &= m - 1) out[off++] = base + __builtin_ctzll(m);
}

// ---- Top-k over several workgroups per row (a caller's workspace) ----
// A row is cut into slices of kTsSlice scores, one 256-thread workgroup each (thread t: slots
// 16 t .. 16 t + 15 of its slice), and five launches replace the one-workgroup kernel:
//   0. slice minimum and maximum of the order keys; the row's histogram, summary and candidate
//      count cleared;
//   1. a 4096-bin histogram of the top 12 bits of (key - row minimum) over the row's key span (so
//      the bins follow the row's own range), per slice in LDS, added into the row's histogram and
//      its 64-bin summary (64 bins a summary bin);
//   2. every slice finds the bin b of the k-th largest key through the summary (two 64-entry
//      scans), counts its keys in higher bins and appends its keys of bin b (key, position) to the
//      row's candidate list;
//   3. one workgroup per row: radix select (8 bits a pass) of the k-th largest key T among the
//      candidates, then, when only some keys equal to T are kept, the position P of the last one
//      kept (lowest positions first); per-slice kept counts, their exclusive scan = output offsets;
//   4. every slice writes the positions of its keys > T, or == T at positions <= P, in order.
// The candidates' order in the list follows the atomic, but nothing computed from it does.
constexpr int kTsThreads = 256;
constexpr int kTsSlots = 16;
constexpr int kTsSlice = kTsThreads * kTsSlots;        // 4096 scores per workgroup
constexpr int kTsMaxSlices = 4096;                     // rows of up to 2^24 scores
constexpr int kTsBins = 4096;
constexpr int kTsSup = 64;                             // summary bins (bin >> 6)

// per-row workspace (32-bit words): slice min / max [2S]; from 2S rounded up to 4: histogram
// [4096]; summary [64]; 8 row parameters; kept-above counts [S]; output offsets [S]; candidate
// keys (relative to the row minimum) [n]; candidate positions [n]
struct TsLayout {
  int64_t hist, sup, par, selgt, off, ckey, cpos, row;
  __host__ __device__ TsLayout(int S, int64_t n) {
    hist = (2 * static_cast<int64_t>(S) + 3) / 4 * 4;
    sup = hist + kTsBins;
    par = sup + kTsSup;
    selgt = par + 8;
    off = selgt + S;
    ckey = off + S;
    cpos = ckey + n;
    row = (cpos + n + 63) / 64 * 64;
  }
};
enum TsPar { kParCount = 0, kParKmin = 1, kParShift = 2, kParT = 3, kParPos = 4, kParBin = 5, kParAbove = 6 };

// the thread's 16 order keys of slice p; returns how many of them exist
__device__ __forceinline__ int ts_load(const float* __restrict__ row, int64_t n, int p, uint32_t (&u)[kTsSlots]) {
  const int64_t s0 = static_cast<int64_t>(p) * kTsSlice;
  const int len = static_cast<int>(min<int64_t>(n - s0, kTsSlice));
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(row + s0, static_cast<uint32_t>(len) * 4u);
  const int base = threadIdx.x * kTsSlots;
#pragma unroll
  for (int j = 0; j < kTsSlots / 4; ++j) {
    const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rs, base * 4 + 16 * j, 0, 0);
    u[4 * j] = w[0];
    u[4 * j + 1] = w[1];
    u[4 * j + 2] = w[2];
    u[4 * j + 3] = w[3];
  }
  // a 16-byte load straddling the slice's end may be range-checked as a whole: reload it by words
  if ((len & 3) != 0 && base <= len - 1 && len - 1 < base + kTsSlots) {
    const int jb = (len - 1 - base) >> 2;
#pragma unroll
    for (int j = 0; j < kTsSlots / 4; ++j) {
      if (j == jb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) u[4 * j + i] = __builtin_amdgcn_raw_buffer_load_b32(rs, (base + 4 * j + i) * 4, 0, 0);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < kTsSlots; ++e) u[e] = order_key(__uint_as_float(u[e]));
  return min(max(len - base, 0), kTsSlots);
}

// exclusive prefix sum over a 256-thread block; *total = the block's sum
__device__ __forceinline__ uint32_t ts_scan(uint32_t v, uint32_t* ws4, uint32_t* total) {
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) ws4[wave] = x;
  __syncthreads();
  uint32_t before = 0u;
  for (int w = 0; w < wave; ++w) before += ws4[w];
  *total = ws4[0] + ws4[1] + ws4[2] + ws4[3];
  __syncthreads();                                                 // ws4 reusable after return
  return before + x - v;
}

__global__ __launch_bounds__(kTsThreads) void topk_s_minmax(const float* __restrict__ scores, int64_t n,
                                                            int64_t scores_bh, uint32_t* __restrict__ ws,
                                                            int S) {
  __shared__ uint32_t red[8];
  const int p = blockIdx.x, tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const TsLayout L(S, n);
  uint32_t* w = ws + static_cast<int64_t>(blockIdx.y) * L.row;
  uint32_t u[kTsSlots];
  const int nv = ts_load(scores + static_cast<int64_t>(blockIdx.y) * scores_bh, n, p, u);
  uint32_t mn = 0xFFFFFFFFu, mx = 0u;
#pragma unroll
  for (int e = 0; e < kTsSlots; ++e) {
    if (e < nv) {
      mn = min(mn, u[e]);
      mx = max(mx, u[e]);
    }
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    mn = min(mn, static_cast<uint32_t>(__shfl_xor(static_cast<int>(mn), o, 64)));
    mx = max(mx, static_cast<uint32_t>(__shfl_xor(static_cast<int>(mx), o, 64)));
  }
  if (lane == 0) {
    red[wave] = mn;
    red[4 + wave] = mx;
  }
  __syncthreads();
  if (tid == 0) {
    w[2 * p] = min(min(red[0], red[1]), min(red[2], red[3]));
    w[2 * p + 1] = max(max(red[4], red[5]), max(red[6], red[7]));
  }
  // histogram and summary cleared by the row's slices together; the candidate count by slice 0
  for (int b = kTsThreads * p + tid; b < kTsBins + kTsSup; b += kTsThreads * S) w[L.hist + b] = 0u;
  if (p == 0 && tid == 0) w[L.par + kParCount] = 0u;
}

__global__ __launch_bounds__(kTsThreads) void topk_s_hist(const float* __restrict__ scores, int64_t n,
                                                          int64_t scores_bh, uint32_t* __restrict__ ws, int S) {
  __shared__ uint32_t h[kTsBins];
  __shared__ uint32_t red[8];
  const int p = blockIdx.x, tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const TsLayout L(S, n);
  uint32_t* w = ws + static_cast<int64_t>(blockIdx.y) * L.row;
  uint32_t u[kTsSlots];
  const int nv = ts_load(scores + static_cast<int64_t>(blockIdx.y) * scores_bh, n, p, u);
  for (int b = tid; b < kTsBins; b += kTsThreads) h[b] = 0u;
  uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
  for (int q = tid; q < S; q += kTsThreads) {
    kmin = min(kmin, w[2 * q]);
    kmax = max(kmax, w[2 * q + 1]);
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    kmin = min(kmin, static_cast<uint32_t>(__shfl_xor(static_cast<int>(kmin), o, 64)));
    kmax = max(kmax, static_cast<uint32_t>(__shfl_xor(static_cast<int>(kmax), o, 64)));
  }
  if (lane == 0) {
    red[wave] = kmin;
    red[4 + wave] = kmax;
  }
  __syncthreads();
  kmin = min(min(red[0], red[1]), min(red[2], red[3]));
  kmax = max(max(red[4], red[5]), max(red[6], red[7]));
  const int span = 32 - __builtin_clz((kmax - kmin) | 1u);         // bits of max - min (>= 1)
  const int s1 = max(0, span - 12);
  if (p == 0 && tid == 0) {
    w[L.par + kParKmin] = kmin;
    w[L.par + kParShift] = static_cast<uint32_t>(s1);
  }
#pragma unroll
  for (int e = 0; e < kTsSlots; ++e) {
    if (e < nv) atomicAdd(&h[(u[e] - kmin) >> s1], 1u);
  }
  __syncthreads();
  for (int b = tid; b < kTsBins; b += kTsThreads) {
    const uint32_t c = h[b];
    if (c != 0u) atomicAdd(&w[L.hist + b], c);
  }
  // summary bin t = bins 64 t .. 64 t + 63, summed by thread t < 64 (reads rotated by t: no two
  // lanes of a read on one LDS bank)
  if (tid < kTsSup) {
    uint32_t t = 0u;
    for (int i = 0; i < 64; ++i) t += h[64 * tid + ((i + tid) & 63)];
    if (t != 0u) atomicAdd(&w[L.sup + tid], t);
  }
}

// within wave 0: lane l holds count c of entry (63 - l) (largest first); the entry where the
// running count from the top reaches k, and the count above it
__device__ __forceinline__ void ts_find64(uint32_t c, uint32_t k0, uint32_t* sh_idx, uint32_t* sh_above) {
  const int lane = threadIdx.x % 64;
  uint32_t x = c;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  const uint32_t excl = x - c;
  if (c > 0u && excl < k0 && x >= k0) {
    *sh_idx = static_cast<uint32_t>(63 - lane);
    *sh_above = excl;
  }
}

__global__ __launch_bounds__(kTsThreads) void topk_s_cand(const float* __restrict__ scores, int64_t n,
                                                          int64_t scores_bh, int64_t k, uint32_t* __restrict__ ws,
                                                          int S) {
  __shared__ uint32_t ws4[4];
  __shared__ uint32_t sh_sup, sh_sabove, sh_bin, sh_above, sh_base;
  const int p = blockIdx.x, tid = threadIdx.x;
  const TsLayout L(S, n);
  uint32_t* w = ws + static_cast<int64_t>(blockIdx.y) * L.row;
  uint32_t u[kTsSlots];
  const int nv = ts_load(scores + static_cast<int64_t>(blockIdx.y) * scores_bh, n, p, u);
  const uint32_t kk = static_cast<uint32_t>(k);
  const uint32_t kmin = w[L.par + kParKmin];
  const int s1 = static_cast<int>(w[L.par + kParShift]);
  if (tid < 64) ts_find64(w[L.sup + 63 - tid], kk, &sh_sup, &sh_sabove);
  __syncthreads();
  if (tid < 64) {
    const uint32_t sb = sh_sup, above = sh_sabove;
    ts_find64(w[L.hist + 64 * sb + 63 - tid], kk - above, &sh_bin, &sh_above);
  }
  __syncthreads();
  const uint32_t bstar = 64u * sh_sup + sh_bin;
  if (p == 0 && tid == 0) {
    w[L.par + kParBin] = bstar;
    w[L.par + kParAbove] = sh_sabove + sh_above;
  }
  uint32_t ngt = 0u, ncand = 0u;
#pragma unroll
  for (int e = 0; e < kTsSlots; ++e) {
    if (e < nv) {
      const uint32_t bin = (u[e] - kmin) >> s1;
      ngt += bin > bstar ? 1u : 0u;
      ncand += bin == bstar ? 1u : 0u;
    }
  }
  uint32_t gt_total, c_total;
  (void)ts_scan(ngt, ws4, &gt_total);
  uint32_t at = ts_scan(ncand, ws4, &c_total);
  if (tid == 0) {
    w[L.selgt + p] = gt_total;
    sh_base = c_total > 0u ? atomicAdd(&w[L.par + kParCount], c_total) : 0u;
  }
  __syncthreads();
  if (ncand > 0u) {
    at += sh_base;
    const uint32_t pos0 = static_cast<uint32_t>(p) * kTsSlice + tid * kTsSlots;
#pragma unroll
    for (int e = 0; e < kTsSlots; ++e) {
      if (e < nv && ((u[e] - kmin) >> s1) == bstar) {
        w[L.ckey + at] = u[e] - kmin;
        w[L.cpos + at] = pos0 + e;
        ++at;
      }
    }
  }
}

// the digit (bits [shift, shift + width)) of the rank-th entry among the candidates that match
// (key & mask) == prefix (largest first when desc), by one LDS histogram pass; rank is 1-based and
// is replaced by the rank within that digit's bin, *cnt by the bin's count
template <bool ByPos>
__device__ __forceinline__ uint32_t ts_digit(const uint32_t* __restrict__ ck, const uint32_t* __restrict__ cp,
                                             uint32_t ncand, uint32_t keyT, uint32_t mask, uint32_t prefix, int shift,
                                             int width, uint32_t* h, uint32_t* ws4, uint32_t* sh, uint32_t& rank,
                                             uint32_t* cnt) {
  const int tid = threadIdx.x;
  const uint32_t dmask = (1u << width) - 1u;
  h[tid] = 0u;
  __syncthreads();
  for (uint32_t i = tid; i < ncand; i += kTsThreads) {
    const uint32_t key = ck[i];
    const uint32_t v = ByPos ? cp[i] : key;
    if ((!ByPos || key == keyT) && (v & mask) == prefix) atomicAdd(&h[(v >> shift) & dmask], 1u);
  }
  __syncthreads();
  // keys: thread t holds digit 255 - t (largest first); positions: digit t (smallest first)
  const uint32_t dig = ByPos ? static_cast<uint32_t>(tid) : static_cast<uint32_t>(255 - tid);
  const uint32_t bt = dig <= dmask ? h[dig] : 0u;
  uint32_t total;
  const uint32_t excl = ts_scan(bt, ws4, &total);
  if (bt > 0u && excl < rank && excl + bt >= rank) {
    sh[0] = dig;
    sh[1] = rank - excl;
    sh[2] = bt;
  }
  __syncthreads();
  rank = sh[1];
  *cnt = sh[2];
  const uint32_t d = sh[0];
  __syncthreads();
  return d;
}

__global__ __launch_bounds__(kTsThreads) void topk_s_resolve(int64_t n, int64_t k, uint32_t* __restrict__ ws, int S) {
  __shared__ uint32_t h[256];
  __shared__ uint32_t cntS[kTsMaxSlices];
  __shared__ uint32_t ws4[4];
  __shared__ uint32_t sh[3];
  const int tid = threadIdx.x;
  const TsLayout L(S, n);
  uint32_t* w = ws + static_cast<int64_t>(blockIdx.x) * L.row;
  const uint32_t* ck = w + L.ckey;
  const uint32_t* cp = w + L.cpos;
  const uint32_t ncand = w[L.par + kParCount];
  const int s1 = static_cast<int>(w[L.par + kParShift]);
  uint32_t rank = static_cast<uint32_t>(k) - w[L.par + kParAbove];   // 1 .. ncand
  // the k-th largest key: its top bits are the bin's; the low s1 bits by 8-bit passes
  uint32_t prefix = w[L.par + kParBin] << s1, mask = 0xFFFFFFFFu << s1, neq = ncand;
  for (int top = s1 - 1; top >= 0;) {
    const int width = min(8, top + 1), shift = top - width + 1;
    const uint32_t d = ts_digit<false>(ck, cp, ncand, 0u, mask, prefix, shift, width, h, ws4, sh, rank, &neq);
    prefix |= d << shift;
    mask |= ((1u << width) - 1u) << shift;
    top = shift - 1;
  }
  const uint32_t T = prefix;                                 // relative key of the k-th largest
  // rank = how many keys equal to T are kept, neq = how many there are: the lowest positions
  uint32_t pT = 0x7FFFFFFFu;
  if (rank < neq) {
    uint32_t pprefix = 0u, pmask = 0u, dummy;
    for (int top = 23; top >= 0;) {                          // positions < 2^24
      const int width = min(8, top + 1), shift = top - width + 1;
      const uint32_t d = ts_digit<true>(ck, cp, ncand, T, pmask, pprefix, shift, width, h, ws4, sh, rank, &dummy);
      pprefix |= d << shift;
      pmask |= ((1u << width) - 1u) << shift;
      top = shift - 1;
    }
    pT = pprefix;
  }
  // kept candidates per slice, plus each slice's keys above the bin: exclusive scan = offsets
  for (int q = tid; q < S; q += kTsThreads) cntS[q] = w[L.selgt + q];
  __syncthreads();
  for (uint32_t i = tid; i < ncand; i += kTsThreads) {
    const uint32_t key = ck[i], pos = cp[i];
    if (key > T || (key == T && pos <= pT)) atomicAdd(&cntS[pos / kTsSlice], 1u);
  }
  __syncthreads();
  const int per = (S + kTsThreads - 1) / kTsThreads, q0 = tid * per;
  uint32_t tot = 0u;
  for (int q = q0; q < min(S, q0 + per); ++q) tot += cntS[q];
  uint32_t total;
  uint32_t run = ts_scan(tot, ws4, &total);
  for (int q = q0; q < min(S, q0 + per); ++q) {
    w[L.off + q] = run;
    run += cntS[q];
  }
  if (tid == 0) {
    w[L.par + kParT] = T;
    w[L.par + kParPos] = pT;
  }
}

__global__ __launch_bounds__(kTsThreads) void topk_s_write(const float* __restrict__ scores, int64_t n,
                                                           int64_t scores_bh, const uint32_t* __restrict__ ws, int S,
                                                           int64_t k, int32_t* __restrict__ idx, int64_t idx_bh) {
  __shared__ uint32_t ws4[4];
  const int p = blockIdx.x, tid = threadIdx.x;
  const TsLayout L(S, n);
  const uint32_t* w = ws + static_cast<int64_t>(blockIdx.y) * L.row;
  uint32_t u[kTsSlots];
  const int nv = ts_load(scores + static_cast<int64_t>(blockIdx.y) * scores_bh, n, p, u);
  const uint32_t kmin = w[L.par + kParKmin], T = w[L.par + kParT], pT = w[L.par + kParPos];
  const uint32_t pos0 = static_cast<uint32_t>(p) * kTsSlice + tid * kTsSlots;
  uint32_t sel = 0u;
#pragma unroll
  for (int e = 0; e < kTsSlots; ++e) {
    const uint32_t r = u[e] - kmin;
    if (e < nv && (r > T || (r == T && pos0 + e <= pT))) sel |= 1u << e;
  }
  uint32_t total;
  uint32_t at = w[L.off + p] + ts_scan(static_cast<uint32_t>(__builtin_popcount(sel)), ws4, &total);
  int32_t* out = idx + static_cast<int64_t>(blockIdx.y) * idx_bh;
  // exactly k positions are kept; the bound only keeps the writes inside the row should that fail
  for (uint32_t m = sel; m != 0u && at < static_cast<uint32_t>(k); m &= m - 1u)
    out[at++] = static_cast<int32_t>(pos0 + __builtin_ctz(m));
}

// nibble (bit offset / 4) of the value-tile word that holds token slot j
__device__ __constant__ int kNibbleOfSlotG[8] = {0, 4, 1, 5, 2, 6, 3, 7};

// Dequantised key and value rows of the retained positions: thread (row i, 8-channel slice sl) of
// (b, h) reads position t = idx[i] from the packed cache -- the 4 key-code bytes of its channels
// (pack_codes rows), their key scale and zero (16-byte loads from group t / group_k), the value
// codes of its channels from the 32-token tile (one word per channel) and the token's (scale, lo)
// pair of its channel group -- and writes code * scale + lo (fp32 multiply then add, as
// kivi_quant's xhat, STRATA_KV.py:855) rounded to the output type, 8 channels per store.  An index
// outside [0, n_valid) writes NaN rows.  16 rows per 256-thread block, every load of a thread
// issued together after its index.
constexpr int kGatherRows = 16;

template <int DT>
__device__ __forceinline__ void store8(void* base, int64_t i, const float (&x)[8]) {
  if constexpr (DT == KVQ_F32) {
    float4* p = reinterpret_cast<float4*>(static_cast<float*>(base) + i);
    p[0] = make_float4(x[0], x[1], x[2], x[3]);
    p[1] = make_float4(x[4], x[5], x[6], x[7]);
  } else {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t lo = DT == KVQ_F16 ? f32_to_f16(x[2 * k]) : f32_to_bf16(x[2 * k]);
      const uint32_t hi = DT == KVQ_F16 ? f32_to_f16(x[2 * k + 1]) : f32_to_bf16(x[2 * k + 1]);
      w[k] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(base) + i) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

template <int DT>
__global__ __launch_bounds__(256) void gather_dequant_kernel(
    const uint8_t* __restrict__ kc, const uint16_t* __restrict__ k_lo, const uint16_t* __restrict__ k_sc,
    const uint8_t* __restrict__ vc, const uint16_t* __restrict__ vmeta, int64_t cap_t, int64_t n_valid,
    int group_k, int group_v, const int32_t* __restrict__ idx, int64_t count, int64_t idx_bh,
    void* __restrict__ k_out, void* __restrict__ v_out, int64_t out_bh, int64_t total) {
  constexpr int d = 128;
  const int64_t flat = static_cast<int64_t>(blockIdx.x) * kGatherRows + threadIdx.x / 16;
  if (flat >= total) return;
  const int sl = threadIdx.x % 16;                   // channels 8 sl .. 8 sl + 7
  const int64_t bh = flat / count, i = flat % count;
  const int64_t t = idx[bh * idx_bh + i];
  const int64_t o = bh * out_bh + i * d + 8 * sl;
  float kx[8], vx[8];
  if (t < 0 || t >= n_valid) {
#pragma unroll
    for (int k = 0; k < 8; ++k) kx[k] = vx[k] = __int_as_float(0x7fc00000);
  } else {
    // keys: byte 4 sl + b holds channels 8 sl + 2b (high nibble) and 8 sl + 2b + 1 (low nibble)
    const uint32_t kw = *reinterpret_cast<const uint32_t*>(kc + (bh * cap_t + t) * (d / 2) + 4 * sl);
    const int64_t km = (bh * (cap_t / group_k) + t / group_k) * d + 8 * sl;
    const uint4 sc4 = *reinterpret_cast<const uint4*>(k_sc + km);
    const uint4 lo4 = *reinterpret_cast<const uint4*>(k_lo + km);
    // values: channel c's word of the tile holds its 8 token slots of lane group g
    const int64_t chunk = t / 32;
    const int u = static_cast<int>(t % 32);
    const int g = (u % 16) / 4, j = 4 * (u / 16) + (u % 4);
    const int blk = sl / 2;                          // 16-channel block of the tile
    const uint32_t* tile = reinterpret_cast<const uint32_t*>(vc + bh * cap_t * (d / 2) + chunk * 16 * d) +
                           (blk / 4) * 256 + (16 * g + 8 * (sl % 2)) * 4 + (blk % 4);
    uint32_t vw[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) vw[e] = tile[4 * e];
    const int ngv = d / group_v;
    const uint32_t vm = *reinterpret_cast<const uint32_t*>(
        vmeta + ((bh * (cap_t / 32) + chunk) * ngv + (8 * sl) / group_v) * 64 + (8 * g + j) * 2);
    const uint32_t scw[4] = {sc4.x, sc4.y, sc4.z, sc4.w}, low[4] = {lo4.x, lo4.y, lo4.z, lo4.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t byte = (kw >> (8 * (k / 2))) & 0xffu;
      const int kcode = (k & 1) ? static_cast<int>(byte & 15u) : static_cast<int>(byte >> 4);
      const float sc = f16_to_f32(static_cast<uint16_t>(scw[k / 2] >> (16 * (k & 1))));
      const float lo = f16_to_f32(static_cast<uint16_t>(low[k / 2] >> (16 * (k & 1))));
      kx[k] = __fadd_rn(__fmul_rn(static_cast<float>(kcode), sc), lo);
    }
    const float sv = f16_to_f32(static_cast<uint16_t>(vm & 0xffffu));
    const float lv = f16_to_f32(static_cast<uint16_t>(vm >> 16));
    const int shift = 4 * kNibbleOfSlotG[j];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int vcode = static_cast<int>((vw[e] >> shift) & 15u);
      vx[e] = __fadd_rn(__fmul_rn(static_cast<float>(vcode), sv), lv);
    }
  }
  store8<DT>(k_out, o, kx);
  store8<DT>(v_out, o, vx);
}

}  // namespace
}  // namespace kvq

using namespace kvq;

extern "C" int kvq_kivi_gather_dequant(const uint8_t* kc, const uint16_t* k_lo, const uint16_t* k_sc,
                                       const uint8_t* vc, const uint16_t* vmeta, int64_t cap_t, int64_t n_valid,
                                       int group_k, int group_v, int64_t BH, int64_t d, const int32_t* idx,
                                       int64_t count, int64_t idx_bh, void* k_out, void* v_out, int out_dtype,
                                       int64_t out_bh, void* stream) {
  KVQ_REQUIRE(valid_dtype(out_dtype), "kvq_kivi_gather_dequant: bad dtype");
  KVQ_REQUIRE(d == 128, "kvq_kivi_gather_dequant: head_dim must be 128");
  KVQ_REQUIRE(group_k > 0 && group_k % 32 == 0 && cap_t % group_k == 0 && cap_t % 32 == 0,
              "kvq_kivi_gather_dequant: bad group_k / capacity");
  KVQ_REQUIRE(group_v == 32 || group_v == 64 || group_v == 128, "kvq_kivi_gather_dequant: group_v in {32,64,128}");
  KVQ_REQUIRE(0 <= n_valid && n_valid <= cap_t, "kvq_kivi_gather_dequant: bad n_valid");
  KVQ_REQUIRE(BH >= 0 && count >= 0 && idx_bh >= count && out_bh >= count * d, "kvq_kivi_gather_dequant: bad sizes");
  const int64_t total = BH * count;
  if (total == 0) return KVQ_OK;
  KVQ_REQUIRE(kc && k_lo && k_sc && vc && vmeta && idx && k_out && v_out, "kvq_kivi_gather_dequant: null pointer");
  KVQ_REQUIRE(out_bh % 8 == 0, "kvq_kivi_gather_dequant: out_bh must be a multiple of 8 (16-byte row slices)");
  KVQ_REQUIRE(reinterpret_cast<uintptr_t>(k_out) % 16 == 0 && reinterpret_cast<uintptr_t>(v_out) % 16 == 0 &&
              reinterpret_cast<uintptr_t>(k_sc) % 16 == 0 && reinterpret_cast<uintptr_t>(k_lo) % 16 == 0,
              "kvq_kivi_gather_dequant: outputs and key metadata must be 16-byte aligned");
  const int64_t blocks = (total + kGatherRows - 1) / kGatherRows;
  KVQ_REQUIRE(blocks < (1LL << 31), "kvq_kivi_gather_dequant: too many rows");
  hipStream_t s = static_cast<hipStream_t>(stream);
  KVQ_DISPATCH_DTYPE(out_dtype, hipLaunchKernelGGL((gather_dequant_kernel<DT_>), dim3(static_cast<unsigned>(blocks)),
                                                  dim3(256), 0, s, kc, k_lo, k_sc, vc, vmeta, cap_t, n_valid,
                                                  group_k, group_v, idx, count, idx_bh,
                                                  k_out, v_out, out_bh, total));
  KVQ_LAUNCH_CHECK("kvq_kivi_gather_dequant");
  return KVQ_OK;
}

extern "C" int64_t kvq_topk_retain_workspace(int64_t BH, int64_t n) {
  if (BH <= 0 || BH > 65535 || n <= kTsSlice || n > static_cast<int64_t>(kTsSlice) * kTsMaxSlices) return 0;
  const int S = static_cast<int>((n + kTsSlice - 1) / kTsSlice);
  return BH * TsLayout(S, n).row;
}

extern "C" int kvq_topk_retain_ws(const float* scores, int64_t BH, int64_t n, int64_t scores_bh, int64_t k,
                                  int32_t* idx, int64_t idx_bh, uint32_t* workspace, int64_t workspace_words,
                                  void* stream) {
  const int64_t need = kvq_topk_retain_workspace(BH, n);
  if (need == 0) return kvq_topk_retain(scores, BH, n, scores_bh, k, idx, idx_bh, stream);
  KVQ_REQUIRE(k >= 0 && k <= n, "kvq_topk_retain_ws: need 0 <= k <= n");
  KVQ_REQUIRE(scores_bh >= n && idx_bh >= k, "kvq_topk_retain_ws: row strides smaller than the rows");
  if (k == 0) return KVQ_OK;
  KVQ_REQUIRE(scores && idx, "kvq_topk_retain_ws: null pointer");
  KVQ_REQUIRE(workspace && workspace_words >= need, "kvq_topk_retain_ws: workspace smaller than kvq_topk_retain_workspace");
  KVQ_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255) == 0, "kvq_topk_retain_ws: workspace not 256-byte aligned");
  const int S = static_cast<int>((n + kTsSlice - 1) / kTsSlice);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 sg(static_cast<unsigned>(S), static_cast<unsigned>(BH)), blk(kTsThreads);
  hipLaunchKernelGGL(topk_s_minmax, sg, blk, 0, st, scores, n, scores_bh, workspace, S);
  hipLaunchKernelGGL(topk_s_hist, sg, blk, 0, st, scores, n, scores_bh, workspace, S);
  hipLaunchKernelGGL(topk_s_cand, sg, blk, 0, st, scores, n, scores_bh, k, workspace, S);
  hipLaunchKernelGGL(topk_s_resolve, dim3(static_cast<unsigned>(BH)), blk, 0, st, n, k, workspace, S);
  hipLaunchKernelGGL(topk_s_write, sg, blk, 0, st, scores, n, scores_bh, workspace, S, k, idx, idx_bh);
  KVQ_LAUNCH_CHECK("kvq_topk_retain_ws");
  return KVQ_OK;
}

extern "C" int kvq_topk_retain(const float* scores, int64_t BH, int64_t n, int64_t scores_bh, int64_t k,
                               int32_t* idx, int64_t idx_bh, void* stream) {
  KVQ_REQUIRE(BH >= 0 && BH < (1LL << 31), "kvq_topk_retain: bad BH");
  KVQ_REQUIRE(n >= 0 && n < (1LL << 31) && k >= 0 && k <= n, "kvq_topk_retain: need 0 <= k <= n < 2^31");
  KVQ_REQUIRE(scores_bh >= n && idx_bh >= k, "kvq_topk_retain: row strides smaller than the rows");
  if (BH == 0 || k == 0) return KVQ_OK;
  KVQ_REQUIRE(scores && idx, "kvq_topk_retain: null pointer");
  if (n <= static_cast<int64_t>(kTopkSlots) * kTopkThreads)
    hipLaunchKernelGGL(topk_retain_rows_kernel, dim3(static_cast<unsigned>(BH)), dim3(kTopkThreads), 0,
                       static_cast<hipStream_t>(stream), scores, static_cast<int>(n), scores_bh, static_cast<int>(k),
                       idx, idx_bh);
  else
    hipLaunchKernelGGL(topk_retain_kernel, dim3(static_cast<unsigned>(BH)), dim3(kTopkThreads), 0,
                       static_cast<hipStream_t>(stream), scores, n, scores_bh, k, idx, idx_bh);
  KVQ_LAUNCH_CHECK("kvq_topk_retain");
  return KVQ_OK;
}
