// STRATA rate allocation on the device (the compression side's allocation of one layer).
//
// Reference: StrataMethod.compress_layer (STRATA_KV.py:1528-1581) and head_sync_allocate
// (STRATA_KV.py:1307-1351).  Input: the distortion table D (Hkv, n, nlev) float32, columns
// [drop | level 1 .. level L | exact] (nlev = L + 2), the per-option cost (summed over heads), the
// fixed bits per cap and the bit budget.  Output:
//   order  (Hkv, n) int32   per head, tokens by D[..., 0] + D[..., 1] descending (ties by index)
//   dsort  (n, nlev) fp32   the table gathered by that order and summed over heads (head order)
//   choice (n,) int32       the Lagrangian allocation per rank position
//   lev    (n,) int32       choice sorted descending (the monotone allocation the code stores)
//   counts (nlev,) int32    its histogram
//   summary [bits, cap, distortion] float64 (distortion = sum dsort[j, lev_j] / sum dsort[j, 0],
//           each clamped to 1e29)
// The per-head order comes from one stable radix sort of (head, importance) keys with the token
// index as value.  The search evaluates a
// grid of kAGrid multipliers per round in float64, every position a thread, and sums per block
// and then across blocks in fixed trees (interleaved wavefront shuffles); the bracket update runs
// in one workgroup.  Products are rounded before sums (no contraction), so the same
// arithmetic restated on the host gives the same allocation.
#include <algorithm>
#include <cfloat>

#include <hipcub/hipcub.hpp>

#include "common.hpp"

#pragma clang fp contract(off)

namespace kvq {
namespace {

constexpr int kAMaxLev = 16;              // options per position (drop, up to 14 levels, exact)
constexpr int kAGrid = 32;                // multipliers per round (the reference's grid)
constexpr int kAThreads = 256;
constexpr double kALo = -80.0, kAHi = 25.0;

struct AllocConst {
  double cost[kAMaxLev];                  // bits of option l summed over heads
  double fixed[kAMaxLev];                 // fixed bits when the deepest level is c (c = 0 .. L)
  double budget;
  int64_t n;
  int nlev;
  int nblk;                               // blocks of the evaluation passes (64 positions each)
  int nblk_lev;                           // blocks of the lev pass (kAThreads positions each)
};

struct AllocState {
  double g[kAGrid];                       // log multipliers of the current pass
  double lo, hi;
  int cap[kAGrid];
  int M;                                  // multipliers in the current pass
};

__device__ __forceinline__ float sanitize(float x) {   // torch.nan_to_num(x, posinf=1e30)
  if (x != x) return 0.0f;
  if (x == INFINITY) return 1e30f;
  if (x == -INFINITY) return -FLT_MAX;
  return x;
}

// the multipliers lo + (hi - lo) * (k / (grid - 1)), the last one lo + (hi - lo) * 1
__device__ __forceinline__ void write_grid(AllocState* st, double lo, double hi) {
  const double step = 1.0 / (kAGrid - 1);
  for (int k = 0; k < kAGrid - 1; ++k) st->g[k] = lo + (hi - lo) * (static_cast<double>(k) * step);
  st->g[kAGrid - 1] = lo + (hi - lo) * 1.0;
  st->lo = lo;
  st->hi = hi;
  st->M = kAGrid;
}

// sort keys ascending in (head, importance descending): head in bits 32.., the complement of the
// order-preserving bits of the float32 importance below; values = token index (the sort is
// stable, so tied keys keep ascending index)
__global__ __launch_bounds__(kAThreads) void alloc_keys_kernel(const float* __restrict__ D, int64_t n, int nlev,
                                                               int Hkv, uint64_t* __restrict__ keys,
                                                               int32_t* __restrict__ vals, AllocState* st,
                                                               int32_t* __restrict__ counts) {
  const int64_t total = static_cast<int64_t>(Hkv) * n;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kAThreads + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kAThreads) {
    const float* row = D + i * nlev;
    const float k = (sanitize(row[0]) + sanitize(row[1])) + 0.0f;   // -0 -> +0
    uint32_t b = __float_as_uint(k);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);               // ascending in k
    keys[i] = (static_cast<uint64_t>(i / n) << 32) | static_cast<uint64_t>(~b);
    vals[i] = static_cast<int32_t>(i % n);
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) write_grid(st, kALo, kAHi);
  if (blockIdx.x == 0 && threadIdx.x < static_cast<unsigned>(nlev)) counts[threadIdx.x] = 0;   // histogram target
}

// order from the sorted values; Dsort rows (heads summed in float32, head order)
__global__ __launch_bounds__(kAThreads) void alloc_dsort_kernel(const float* __restrict__ D,
                                                                const int32_t* __restrict__ sorted, int Hkv,
                                                                int64_t n, int nlev, int32_t* __restrict__ order,
                                                                float* __restrict__ dsort) {
  for (int64_t j = static_cast<int64_t>(blockIdx.x) * kAThreads + threadIdx.x; j < n;
       j += static_cast<int64_t>(gridDim.x) * kAThreads) {
    float acc[kAMaxLev];
    for (int h0 = 0; h0 < Hkv; h0 += 8) {                         // eight heads' rows in flight
      int32_t tok[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) tok[u] = h0 + u < Hkv ? sorted[static_cast<int64_t>(h0 + u) * n + j] : 0;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int h = h0 + u;
        if (h >= Hkv) break;
        order[static_cast<int64_t>(h) * n + j] = tok[u];
        const float* row = D + (static_cast<int64_t>(h) * n + tok[u]) * nlev;
#pragma unroll
        for (int l = 0; l < kAMaxLev; ++l)
          if (l < nlev) acc[l] = h == 0 ? sanitize(row[l]) : acc[l] + sanitize(row[l]);
      }
    }
#pragma unroll
    for (int l = 0; l < kAMaxLev; ++l)
      if (l < nlev) dsort[j * nlev + l] = acc[l];
  }
}

__device__ __forceinline__ double wave_sum_f64(double x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

// N independent wave sums, interleaved (their shuffle latencies overlap)
template <int N>
__device__ __forceinline__ void wave_sum_arr(double (&v)[N]) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1)
#pragma unroll
    for (int c = 0; c < N; ++c) v[c] += __shfl_xor(v[c], o, 64);
}

// One evaluation pass over every position for the state's multipliers: a block holds 64
// positions (lane = position) and each wavefront kAGrid / 4 of the multipliers.
//   TOT:  part[g][blk][c] = sum over the block's positions of min(base, best level <= c)
//         (c = 0: base), the totals the cap is chosen from
//   else: part[g][blk] (compact) = sum of cost[choice] under the chosen cap; choice written if asked
template <bool TOT, int MAXC>
__global__ __launch_bounds__(kAThreads) void alloc_eval_kernel(const float* __restrict__ dsort, AllocConst k,
                                                               const AllocState* __restrict__ st,
                                                               double* __restrict__ part,
                                                               int32_t* __restrict__ choice_out) {
  constexpr int GC = kAGrid / (kAThreads / 64);                   // multipliers per wavefront
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int M = st->M;
  const int g0 = wave * GC;
  if (g0 >= M) return;                                            // wave-uniform; no barrier below
  const int64_t j = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  const bool valid = j < k.n;
  const int nlev = k.nlev, L = nlev - 2;
  double D[kAMaxLev];
#pragma unroll
  for (int l = 0; l < kAMaxLev; ++l) D[l] = valid && l < nlev ? static_cast<double>(dsort[j * nlev + l]) : 0.0;
  double v[GC * (TOT ? MAXC : 1)];
#pragma unroll
  for (int u = 0; u < GC; ++u) {
    const int g = g0 + u;
    const double mu = exp(st->g[g < M ? g : 0]);
    double Q[kAMaxLev];                                           // columns past nlev: cost 0, unused
#pragma unroll
    for (int l = 0; l < kAMaxLev; ++l) Q[l] = D[l] + mu * k.cost[l];
    double qx = Q[0];
#pragma unroll
    for (int l = 1; l < kAMaxLev; ++l)
      if (l == nlev - 1) qx = Q[l];
    const double q0 = Q[0];
    const double base = fmin(q0, qx);
    const int bidx = q0 <= qx ? 0 : nlev - 1;
    if (TOT) {                                                    // v[c]: min(base, best level <= c)
      v[u * MAXC] = valid ? base : 0.0;
      double cm = 0.0;
#pragma unroll
      for (int c = 1; c < MAXC; ++c) {
        cm = c == 1 ? Q[c] : (Q[c] <= cm ? Q[c] : cm);            // running minimum over levels <= c
        v[u * MAXC + c] = valid && c <= L ? fmin(base, cm) : 0.0;
      }
    } else {
      const int cap = g < M ? st->cap[g] : 0;
      double cm = 0.0;
      int ci = 0;
#pragma unroll
      for (int c = 1; c < kAMaxLev - 1; ++c) {                    // the best level <= cap, later on ties
        if (c > cap) break;
        if (c == 1 || Q[c] <= cm) {
          cm = Q[c];
          ci = c;
        }
      }
      const int ch = cap > 0 && cm < base ? ci : bidx;
      if (choice_out != nullptr && valid && g < M) choice_out[j] = ch;
      double cch = 0.0;                                           // k.cost[ch] without a dynamic index
#pragma unroll
      for (int o = 0; o < kAMaxLev; ++o) cch = ch == o ? k.cost[o] : cch;
      v[u] = valid ? cch : 0.0;
    }
  }
  wave_sum_arr(v);
  if (lane == 0)
#pragma unroll
    for (int u = 0; u < GC; ++u) {
      const int g = g0 + u;
      if (g >= M) break;
      if (TOT) {
        double* pp = part + (static_cast<int64_t>(g) * k.nblk + blockIdx.x) * kAMaxLev;
#pragma unroll
        for (int c = 0; c < MAXC; ++c)
          if (c <= L) pp[c] = v[u * MAXC + c];
      } else {
        part[static_cast<int64_t>(g) * k.nblk + blockIdx.x] = v[u];   // compact [g][blk]
      }
    }
}

// per multiplier (one block each): the cap with the first minimal total
__global__ __launch_bounds__(kAThreads) void alloc_pick_kernel(AllocConst k, AllocState* st,
                                                               const double* __restrict__ part) {
  __shared__ double red[kAThreads / 64][kAMaxLev];
  const int g = blockIdx.x;
  if (g >= st->M) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nv = k.nlev - 1;                                      // caps 0 .. L
  double v[kAMaxLev - 1];
#pragma unroll
  for (int c = 0; c < kAMaxLev - 1; ++c) v[c] = 0.0;
  for (int b = tid; b < k.nblk; b += kAThreads) {
    const double* pp = part + (static_cast<int64_t>(g) * k.nblk + b) * kAMaxLev;
#pragma unroll
    for (int c = 0; c < kAMaxLev - 1; ++c)
      if (c < nv) v[c] += pp[c];
  }
  wave_sum_arr(v);
  if (lane == 0)
#pragma unroll
    for (int c = 0; c < kAMaxLev - 1; ++c) red[wave][c] = v[c];
  __syncthreads();
  if (tid != 0) return;
  const double mu = exp(st->g[g]);
  double best = 0.0;
  int bc = 0;
  for (int c = 0; c < nv; ++c) {
    const double tot = (((red[0][c] + red[1][c]) + red[2][c]) + red[3][c]) + mu * k.fixed[c];
    if (c == 0 || tot < best) {
      best = tot;
      bc = c;
    }
  }
  st->cap[g] = bc;
}

// sum over the blocks' partials at the given stride (one wavefront, fixed order)
__device__ __forceinline__ double wave_sum_blocks(const double* p, int nblk, int stride, int lane) {
  double s = 0.0;
  for (int b = lane; b < nblk; b += 64) s += p[static_cast<int64_t>(b) * stride];
  return wave_sum_f64(s);
}

// bits per multiplier, the first feasible one brackets the next round's grid (or, with last,
// the final pass's single multiplier hi)
constexpr int kARoundThreads = 1024;

__global__ __launch_bounds__(kARoundThreads) void alloc_round_kernel(AllocConst k, AllocState* st,
                                                                     const double* __restrict__ part, int last) {
  __shared__ int ok[kAGrid];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int M = st->M;
  constexpr int GW = kAGrid / (kARoundThreads / 64);              // multipliers per wavefront
  double v[GW];
#pragma unroll
  for (int u = 0; u < GW; ++u) {
    const int g = wave * GW + u;
    v[u] = 0.0;
    if (g < M) {
      const double* pg = part + static_cast<int64_t>(g) * k.nblk;  // compact bits partials
#pragma unroll 8
      for (int b = lane; b < k.nblk; b += 64) v[u] += pg[b];
    }
  }
  wave_sum_arr(v);
  if (lane == 0)
#pragma unroll
    for (int u = 0; u < GW; ++u) {
      const int g = wave * GW + u;
      if (g < M) ok[g] = v[u] + k.fixed[st->cap[g]] <= k.budget;
    }
  __syncthreads();
  if (tid != 0) return;
  int i = M - 1;
  for (int t = 0; t < M; ++t)
    if (ok[t]) {
      i = t;
      break;
    }
  const double lo = st->g[i > 0 ? i - 1 : 0], hi = st->g[i];
  if (last) {
    st->g[0] = hi;
    st->lo = lo;
    st->hi = hi;
    st->M = 1;
  } else {
    write_grid(st, lo, hi);
  }
}

// the final pass's single multiplier = the bracket's upper end (also for zero rounds)
__global__ void alloc_final_kernel(AllocState* st) {
  st->g[0] = st->hi;
  st->M = 1;
}

// histogram of the choice (per-block counts added to the zeroed histogram: integer, so exact in
// any order); block 0 also writes bits and cap of the final pass (or of the all-drop allocation)
__global__ __launch_bounds__(kAThreads) void alloc_count_kernel(AllocConst k, const AllocState* __restrict__ st,
                                                                const double* __restrict__ partb,
                                                                const int32_t* __restrict__ choice, int search,
                                                                int32_t* __restrict__ counts,
                                                                double* __restrict__ summary) {
  __shared__ int hist[kAMaxLev];
  if (threadIdx.x < kAMaxLev) hist[threadIdx.x] = 0;
  __syncthreads();
  const int64_t j = static_cast<int64_t>(blockIdx.x) * kAThreads + threadIdx.x;
  const int ch = j < k.n ? choice[j] : -1;
  int cnt[kAMaxLev];
#pragma unroll
  for (int o = 0; o < kAMaxLev; ++o) cnt[o] = ch == o;
#pragma unroll
  for (int sh = 32; sh > 0; sh >>= 1)
#pragma unroll
    for (int o = 0; o < kAMaxLev; ++o) cnt[o] += __shfl_xor(cnt[o], sh, 64);
  if ((threadIdx.x & 63) == 0)
#pragma unroll
    for (int o = 0; o < kAMaxLev; ++o)
      if (o < k.nlev && cnt[o]) atomicAdd(&hist[o], cnt[o]);
  __syncthreads();
  if (static_cast<int>(threadIdx.x) < k.nlev && hist[threadIdx.x]) atomicAdd(&counts[threadIdx.x], hist[threadIdx.x]);
  if (blockIdx.x != 0) return;
  const double sb = threadIdx.x < 64 ? wave_sum_blocks(partb, k.nblk, 1, threadIdx.x) : 0.0;
  if (threadIdx.x == 0) {
    if (search) {
      summary[0] = sb + k.fixed[st->cap[0]];
      summary[1] = st->cap[0];
    } else {
      summary[0] = k.fixed[0];
      summary[1] = 0;
    }
  }
}

__global__ __launch_bounds__(kAThreads) void alloc_zero_kernel(int32_t* __restrict__ choice, int64_t n) {
  for (int64_t j = static_cast<int64_t>(blockIdx.x) * kAThreads + threadIdx.x; j < n;
       j += static_cast<int64_t>(gridDim.x) * kAThreads)
    choice[j] = 0;
}

// lev = choice sorted descending (from the histogram); per-block sums of the clamped distortions
__global__ __launch_bounds__(kAThreads) void alloc_lev_kernel(AllocConst k, const int32_t* __restrict__ counts,
                                                              const float* __restrict__ dsort,
                                                              int32_t* __restrict__ lev, double* __restrict__ part) {
  __shared__ double red[kAThreads / 64][2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t j = static_cast<int64_t>(blockIdx.x) * kAThreads + tid;
  double fin = 0.0, ref = 0.0;
  if (j < k.n) {
    int o = k.nlev - 1;
    int64_t end = counts[o];
    while (j >= end && o > 0) end += counts[--o];
    lev[j] = o;
    fin = fmin(static_cast<double>(dsort[j * k.nlev + o]), 1e29);
    ref = fmin(static_cast<double>(dsort[j * k.nlev]), 1e29);
  }
  fin = wave_sum_f64(fin);
  ref = wave_sum_f64(ref);
  if (lane == 0) {
    red[wave][0] = fin;
    red[wave][1] = ref;
  }
  __syncthreads();
  if (tid < 2) part[static_cast<int64_t>(blockIdx.x) * kAMaxLev + tid] =
      ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
}

__global__ __launch_bounds__(64) void alloc_ratio_kernel(AllocConst k, const double* __restrict__ part,
                                                         double* __restrict__ summary) {
  const double fin = wave_sum_blocks(part, k.nblk_lev, kAMaxLev, threadIdx.x);
  const double ref = wave_sum_blocks(part + 1, k.nblk_lev, kAMaxLev, threadIdx.x);
  if (threadIdx.x == 0) summary[2] = fin / fmax(ref, 1e-30);
}

struct AllocLayout {
  size_t keys_in, keys_out, vals_in, vals_out, state, part, partb, temp, temp_bytes, total;
};

int sort_end_bit(int64_t Hkv) {                  // key bits that can differ: 32 + the head's
  int hb = 0;
  while ((1LL << hb) < Hkv) ++hb;
  return 32 + hb;
}

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

int alloc_layout(int64_t Hkv, int64_t n, AllocLayout& a) {
  const int64_t total = Hkv * n;
  const int64_t nblk = (n + 63) / 64;                   // evaluation blocks (the lev pass needs fewer)
  size_t temp = 0;
  const hipError_t e = hipcub::DeviceRadixSort::SortPairs(
      nullptr, temp, static_cast<const uint64_t*>(nullptr), static_cast<uint64_t*>(nullptr),
      static_cast<const int32_t*>(nullptr), static_cast<int32_t*>(nullptr), static_cast<int>(total), 0,
      sort_end_bit(Hkv), static_cast<hipStream_t>(nullptr));
  if (e != hipSuccess) return KVQ_EINVAL;
  size_t off = 0;
  a.keys_in = off;
  off += align256(total * sizeof(uint64_t));
  a.keys_out = off;
  off += align256(total * sizeof(uint64_t));
  a.vals_in = off;
  off += align256(total * sizeof(int32_t));
  a.vals_out = off;
  off += align256(total * sizeof(int32_t));
  a.state = off;
  off += align256(sizeof(AllocState));
  a.part = off;
  off += align256(static_cast<size_t>(kAGrid) * nblk * kAMaxLev * sizeof(double));
  a.partb = off;
  off += align256(static_cast<size_t>(kAGrid) * nblk * sizeof(double));
  a.temp = off;
  a.temp_bytes = temp;
  off += align256(temp);
  a.total = off;
  return KVQ_OK;
}

}  // namespace
}  // namespace kvq

using namespace kvq;

extern "C" int64_t kvq_strata_allocate_workspace(int64_t Hkv, int64_t n, int nlev) {
  if (Hkv <= 0 || Hkv >= kAThreads || n <= 0 || Hkv * n >= (1LL << 31) || nlev < 2 || nlev > kAMaxLev) return -1;
  AllocLayout a;
  if (alloc_layout(Hkv, n, a) != KVQ_OK) return -1;
  return static_cast<int64_t>(a.total);
}

extern "C" int kvq_strata_allocate(const float* D, int64_t Hkv, int64_t n, int nlev, const double* cost,
                                   const double* fixed, double budget, int rounds, int32_t* order, float* dsort,
                                   int32_t* choice, int32_t* lev, int32_t* counts, double* summary, void* workspace,
                                   int64_t workspace_bytes, void* stream) {
  KVQ_REQUIRE(Hkv > 0 && Hkv < kAThreads && n > 0 && Hkv * n < (1LL << 31),
              "kvq_strata_allocate: need 0 < Hkv < %d, n > 0 and Hkv n < 2^31", kAThreads);
  KVQ_REQUIRE(nlev >= 2 && nlev <= kAMaxLev, "kvq_strata_allocate: nlev must be in [2, %d]", kAMaxLev);
  KVQ_REQUIRE(D && cost && fixed && order && dsort && choice && lev && counts && summary && workspace,
              "kvq_strata_allocate: null pointer");
  KVQ_REQUIRE(rounds <= 64, "kvq_strata_allocate: at most 64 rounds");
  KVQ_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "kvq_strata_allocate: workspace must be 256-byte aligned");
  AllocLayout lay;
  KVQ_REQUIRE(alloc_layout(Hkv, n, lay) == KVQ_OK, "kvq_strata_allocate: sort workspace query failed");
  KVQ_REQUIRE(workspace_bytes >= static_cast<int64_t>(lay.total),
              "kvq_strata_allocate: workspace of %lld bytes, need %lld", static_cast<long long>(workspace_bytes),
              static_cast<long long>(lay.total));
  AllocConst k{};
  for (int l = 0; l < nlev; ++l) k.cost[l] = cost[l];
  for (int c = 0; c < nlev - 1; ++c) k.fixed[c] = fixed[c];
  k.budget = budget;
  k.n = n;
  k.nlev = nlev;
  k.nblk = static_cast<int>((n + 63) / 64);
  k.nblk_lev = static_cast<int>((n + kAThreads - 1) / kAThreads);
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint64_t* keys_in = reinterpret_cast<uint64_t*>(ws + lay.keys_in);
  uint64_t* keys_out = reinterpret_cast<uint64_t*>(ws + lay.keys_out);
  int32_t* vals_in = reinterpret_cast<int32_t*>(ws + lay.vals_in);
  int32_t* vals_out = reinterpret_cast<int32_t*>(ws + lay.vals_out);
  AllocState* state = reinterpret_cast<AllocState*>(ws + lay.state);
  double* part = reinterpret_cast<double*>(ws + lay.part);
  double* partb = reinterpret_cast<double*>(ws + lay.partb);
  const int64_t total = Hkv * n;
  const unsigned kb = static_cast<unsigned>(std::min<int64_t>((total + kAThreads - 1) / kAThreads, 4096));
  hipLaunchKernelGGL(alloc_keys_kernel, dim3(kb), dim3(kAThreads), 0, st, D, n, nlev, static_cast<int>(Hkv), keys_in,
                     vals_in, state, counts);
  KVQ_LAUNCH_CHECK("kvq_strata_allocate(keys)");
  size_t temp_bytes = lay.temp_bytes;
  const hipError_t se = hipcub::DeviceRadixSort::SortPairs(ws + lay.temp, temp_bytes, keys_in, keys_out, vals_in,
                                                           vals_out, static_cast<int>(total), 0, sort_end_bit(Hkv), st);
  KVQ_REQUIRE(se == hipSuccess, "kvq_strata_allocate: radix sort failed: %s", hipGetErrorString(se));
  const unsigned nb = static_cast<unsigned>(k.nblk_lev), ne = static_cast<unsigned>(k.nblk);
  hipLaunchKernelGGL(alloc_dsort_kernel, dim3(nb), dim3(kAThreads), 0, st, D, vals_out, static_cast<int>(Hkv), n, nlev,
                     order, dsort);
  KVQ_LAUNCH_CHECK("kvq_strata_allocate(dsort)");
  const int search = rounds >= 0;
  if (search) {
    const int L1 = nlev - 1;                                      // caps 0 .. L
#define KVQ_AEVAL(TOT_, P_, CH_)                                                                                      \
  do {                                                                                                            \
    if (L1 <= 4) hipLaunchKernelGGL((alloc_eval_kernel<TOT_, 4>), dim3(ne), dim3(kAThreads), 0, st, dsort, k, state, P_, CH_); \
    else if (L1 <= 8) hipLaunchKernelGGL((alloc_eval_kernel<TOT_, 8>), dim3(ne), dim3(kAThreads), 0, st, dsort, k, state, P_, CH_); \
    else hipLaunchKernelGGL((alloc_eval_kernel<TOT_, 15>), dim3(ne), dim3(kAThreads), 0, st, dsort, k, state, P_, CH_); \
  } while (0)
    for (int r = 0; r < rounds; ++r) {
      KVQ_AEVAL(true, part, nullptr);
      hipLaunchKernelGGL(alloc_pick_kernel, dim3(kAGrid), dim3(kAThreads), 0, st, k, state, part);
      KVQ_AEVAL(false, partb, nullptr);
      hipLaunchKernelGGL(alloc_round_kernel, dim3(1), dim3(kARoundThreads), 0, st, k, state, partb,
                         r == rounds - 1 ? 1 : 0);
    }
    if (rounds == 0) hipLaunchKernelGGL(alloc_final_kernel, dim3(1), dim3(1), 0, st, state);
    KVQ_AEVAL(true, part, nullptr);
    hipLaunchKernelGGL(alloc_pick_kernel, dim3(kAGrid), dim3(kAThreads), 0, st, k, state, part);
    KVQ_AEVAL(false, partb, choice);
#undef KVQ_AEVAL
  } else {
    hipLaunchKernelGGL(alloc_zero_kernel, dim3(nb), dim3(kAThreads), 0, st, choice, n);
  }
  KVQ_LAUNCH_CHECK("kvq_strata_allocate(search)");
  hipLaunchKernelGGL(alloc_count_kernel, dim3(nb), dim3(kAThreads), 0, st, k, state, partb, choice, search, counts,
                     summary);
  hipLaunchKernelGGL(alloc_lev_kernel, dim3(nb), dim3(kAThreads), 0, st, k, counts, dsort, lev, part);
  hipLaunchKernelGGL(alloc_ratio_kernel, dim3(1), dim3(64), 0, st, k, part, summary);
  KVQ_LAUNCH_CHECK("kvq_strata_allocate(finish)");
  return KVQ_OK;
}
