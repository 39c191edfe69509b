// STRATA coverage statistics on the device (gfx950): coverage_stats, STRATA_KV.py:1225-1298.
//
// For every coverage group g (host-drawn query positions, coverage_groups 1206-1222) and KV head h,
// the rows r = (query head of h, query) attend causally to the keys [0, max position]; their
// probabilities p and outputs o give, for the coded tokens j in [rs, min(re, max position + 1)) read
// at distance >= local: pR = p_j, u = ||v_j - o||^2_M (M the query head's output metric), the drop
// term (pR / max(1 - pR, 1e-6))^2 u, the key term a = pR^2 u and the read mass pR^2, averaged over
// the group's queries and normalised by the group's drop total N (over every head and token); then
// averaged over the live groups, S = sum of alpha q q^T (alpha = a row's key-term mass) normalised
// by sum_j A_j, Mbar = read-weighted mean metric, and every output + floor x its mean.
//
// Rows are laid out per KV head as [group][query head r][query, padded to 16] (row_base of a group in
// the group table); padded rows have position -1 and contribute nothing.  Launches (one stream, no
// host synchronisation, no atomics: every sum has a fixed order):
//   cov_rowstats  per (group, 64-row block, h): logits of 16-key tiles on the matrix cores
//                 (row_tiles.hpp), online max / sum per row -> row max (base 2) and 1 / sum; every
//                 key tile feeds all the block's rows a wavefront holds, the wavefronts split the keys.
//   cov_output    per (group, 64-row block, h, key split): the logits again, p = 2^(s - max) / sum in
//                 registers as the A operand of the PV product (hi + lo parts; the two 16-key tiles
//                 of a 32-key step give every lane 8 keys of its row, in an order the B operand
//                 follows), B = values of the step from an LDS tile; the split's part of o, fp32.
//   cov_metric    x M and x M x for 32 vectors per workgroup with the query head's metric staged in
//                 LDS: the row outputs (the key splits' parts summed in order; o M) and the coded
//                 values (v M v).
//   cov_terms<A>  per (h, 256-token chunk, group split): for every group of the split reaching the
//                 chunk, logits and v.(oM) of 16-token tiles on the matrix cores (rows as the A side:
//                 a lane holds four rows of one token), then the per-(row, token) terms: the group's
//                 drop total and every row's key-term mass, as partials per chunk.
//   cov_groups    N per group -> weight 1 / N (0 if N = 0), live flag.
//   cov_roww      per row: its group's weight x its key-term mass.
//   cov_terms<B>  the same tiles with the weights: A, DD and the read mass per query head, one partial
//                 per group split; cov_split_sums adds the splits in order.
//   cov_smat      S = sum over rows of weight * alpha * (scaling q)(scaling q)^T.
//   cov_final     live average, S / sum_j A_j, Mbar, floors (one workgroup for the sums, then all).
#include <algorithm>

#include "common.hpp"
#include "mfma_common.hpp"
#include "row_tiles.hpp"

namespace kvq {
namespace {

constexpr int kCD = 128;
constexpr int kCThreads = 256;
constexpr int kCWaves = 4;
constexpr int kChunkTok = 256;          // tokens of a cov_terms workgroup
constexpr int kGT = 8;                  // ints per group-table entry
constexpr int kMetricRows = 32;         // vectors of a cov_metric workgroup
constexpr int kOSplit = 4;              // key splits of cov_output (workgroups per 64-row item)
constexpr int kTSplit = 4;              // group splits of cov_terms (workgroups per token chunk)
constexpr int kTermsLdsRep = 8;         // most query heads per KV head of cov_terms' LDS form
constexpr int kSSplit = 16;             // row splits of cov_smat (workgroups per 16 rows of S)
constexpr float kCLog2e = 1.4426950408889634f;

// group table entry (kGT ints): row_base, nq, nq_pad, mmax, te, local, 0, 0
struct CovParams {
  const void* qr;                        // (Hkv, NR, d) group query rows (unscaled), DT
  const int32_t* rowpos;                 // (NR): position of each row (-1: padding)
  const int32_t* gtab;                   // (G, kGT)
  const int32_t* items;                  // (n_items, 2): (group, 64-row block)
  const void* k;
  const void* v;
  int64_t k_sh, k_st, v_sh, v_st;        // element strides of the (head, token) axes
  const float* M;                        // (Hq, d, d)
  int Hkv, rep, NR, G, n_items, rs, re, n, n_chunks, T;
  float qscale;                          // scaling * log2(e)
  float scaling, eta;
  float* row_m;                          // (Hkv, NR) row max (base 2)
  float* row_il;                         // (Hkv, NR) 1 / row sum
  float* o;                              // (Hkv, NR, d) o M (cov_metric over the summed outputs)
  float* o_part;                         // (kOSplit, Hkv, NR, d) fp32 outputs of each key split
  float* oMo;                            // (Hkv, NR)
  uint32_t* mop;                         // (Hkv, NR, 4 ks, 4 g, 2 parts) u32x4: o M operand parts
  float* rowf;                           // (Hkv, NR) float4: row max, 1 / sum, o M o, o M scale
  float* vmv;                            // (Hkv, rep, n)
  float* ddpart;                         // (G, Hkv, n_chunks, 4): drop totals per wavefront
  float* alpha_part;                     // (Hkv, n_chunks, NR)
  float* gw;                             // (2 G + 1): 1 / N or 0 per group; [G + 1 + group]: 1 if live
  float* roww;                           // (Hkv, NR): weight * alpha
  float* red;                            // finalisation sums
  float* sums;                           // (Hkv, 2 + rep): per-head sums of A, DD, read masses
  float* A;                              // (Hkv, n)
  float* W;                              // (Hkv, n)
  float* DD;                             // (Hkv, n)
  float* WVa;                            // (Hkv, rep, n)
  float* A_part;                         // (kTSplit, Hkv, n) weighted pass: each group split's sums
  float* DD_part;                        // (kTSplit, Hkv, n)
  float* WVa_part;                       // (kTSplit, Hkv, rep, n)
  float* S;                              // (Hkv, d, d)
  float* S_part;                         // (kSSplit, Hkv, d, d): each row split's sum
  float* Mbar;                           // (Hkv, d, d)
  // fp32 rows: the powers of two of qr, k and v (rows_scale_kernel, row_tiles.hpp); null otherwise
  const float* xs;
};

// the power of two of fp32 view i (0: qr, 1: k, 2: v); 16-bit rows are exact operands: 1
template <int DT>
__device__ __forceinline__ float cov_xs(const CovParams& p, int i) {
  if constexpr (DT == KVQ_F32) return p.xs[i];
  else return 1.0f;
}

// the rows of head h as a buffer resource covering T token rows (reads past it return zero)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t head_rsrc(const void* base, int64_t sh, int64_t st, int h, int T,
                                                           int esz) {
  const char* b = static_cast<const char*>(base) + static_cast<int64_t>(h) * sh * esz;
  return make_rsrc(b, static_cast<uint32_t>((static_cast<int64_t>(T - 1) * st + kCD) * esz));
}

// Work unit of this block when each XCD (blocks b % 8, dispatched round-robin) takes a contiguous
// range of the units, so neighbouring units, which read overlapping keys and values, share one L2;
// -1 past the last unit (grids are rounded up to a multiple of 8)
__device__ __forceinline__ int xcd_unit(int n_units) {
  const int per = (n_units + 7) / 8;
  const int u = static_cast<int>(blockIdx.x % 8) * per + static_cast<int>(blockIdx.x / 8);
  return u < n_units ? u : -1;
}
inline unsigned xcd_grid(int64_t n_units) { return static_cast<unsigned>(8 * ((n_units + 7) / 8)); }

template <int DT>
__device__ __forceinline__ void zero_ops(u32x4 (&op)[4][TileOps<DT>::NH]) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int hh = 0; hh < TileOps<DT>::NH; ++hh) op[ks][hh] = u32x4{0u, 0u, 0u, 0u};
}

// query operands (B) of the 16 rows starting at row0 of head h; returns this lane's row position
template <int DT>
__device__ __forceinline__ int load_rows(const CovParams& p, int h, int row0, int g, int n,
                                         u32x4 (&qop)[4][TileOps<DT>::NH]) {
  const int row = row0 + n;
  const int pos = row < p.NR ? p.rowpos[row] : -1;
  if (pos >= 0) {
    const int64_t base = (static_cast<int64_t>(h) * p.NR + row) * kCD;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) load_op<DT>(p.qr, base + 32 * ks + 8 * g, qop[ks], cov_xs<DT>(p, 0));
  } else {
    zero_ops<DT>(qop);
  }
  return pos;
}

// A operand (tokens) of the 16-token tile at t0: this lane's token t0 + n
template <int DT>
__device__ __forceinline__ void load_tile(__amdgpu_buffer_rsrc_t rs, int64_t st, int t0, int g, int n,
                                          u32x4 (&op)[4][TileOps<DT>::NH], float sc) {
  const int64_t tok = t0 + n;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    load_op_buf<DT>(rs, static_cast<int>((tok * st + 32 * ks + 8 * g) * TileOps<DT>::ESZ), op[ks], sc);
}

// Every key tile a wavefront loads feeds several of the item's 16-row blocks (16-bit data: all four,
// eight wavefronts (two per SIMD) splitting the keys in eighths; fp32 operands take twice the
// registers: two blocks, four wavefronts in halves), so the workgroup reads its keys once instead of
// once per row block.  The wavefronts' states of a row meet in LDS, split by split in a fixed order.
// The items go in reverse plan order: the groups at the end of the context, whose keys reach
// furthest, start first.
template <int DT>
__global__ __launch_bounds__(DT == KVQ_F32 ? kCThreads : 2 * kCThreads) void cov_rowstats(CovParams p) {
  constexpr int NH = TileOps<DT>::NH;
  constexpr int NW = DT == KVQ_F32 ? kCWaves : 2 * kCWaves;  // wavefronts (16-bit: two per SIMD)
  constexpr int NRB = DT == KVQ_F32 ? 2 : 4;                 // row blocks per wavefront
  constexpr int KS = NW * NRB / 4;                           // key splits (wavefronts sharing blocks)
  __shared__ float st[NW][NRB][16][2];
  const int wave = threadIdx.x / 64, l = threadIdx.x % 64, g = l >> 4, n = l & 15;
  const int unit = xcd_unit(p.Hkv * p.n_items);                // (h, item), h outermost
  if (unit < 0) return;
  const int item = p.n_items - 1 - unit % p.n_items, h = unit / p.n_items;
  const int grp = p.items[2 * item], rb = p.items[2 * item + 1];
  const int32_t* gt = p.gtab + kGT * grp;
  const int rows_g = p.rep * gt[2];
  const int mmax = gt[3];
  const int ks = wave % KS, rgrp = wave / KS;
  u32x4 qop[NRB][4][NH];
  int pos[NRB];
#pragma unroll
  for (int b = 0; b < NRB; ++b) {
    const int rl = 64 * rb + 16 * (rgrp * NRB + b);           // first row of the block in the group
    if (rl < rows_g) {
      pos[b] = load_rows<DT>(p, h, gt[0] + rl, g, n, qop[b]);
    } else {
      pos[b] = -1;
      zero_ops<DT>(qop[b]);
    }
  }
  // this split's keys: whole 16-key tiles
  const int ntile = (mmax + 15) / 16;
  const int k0 = 16 * (ntile * ks / KS), k1 = min(mmax, 16 * (ntile * (ks + 1) / KS));
  const __amdgpu_buffer_rsrc_t rk = head_rsrc(p.k, p.k_sh, p.k_st, h, p.T, TileOps<DT>::ESZ);
  const float qsc = p.qscale / (cov_xs<DT>(p, 0) * cov_xs<DT>(p, 1));   // logit scale of the scaled rows
  float m[NRB], ls[NRB];
#pragma unroll
  for (int b = 0; b < NRB; ++b) {
    m[b] = -INFINITY;
    ls[b] = 0.0f;
  }
  // three key tiles in rotation: two in flight behind the one computed (a tile past the split reads
  // zeros through the buffer resource or in-range keys, masked or never computed)
  u32x4 kt[3][4][NH];
  load_tile<DT>(rk, p.k_st, k0, g, n, kt[0], cov_xs<DT>(p, 1));
  load_tile<DT>(rk, p.k_st, k0 + 16, g, n, kt[1], cov_xs<DT>(p, 1));
  auto tile = [&](int t0, const u32x4 (&kop)[4][NH]) {
#pragma unroll
    for (int b = 0; b < NRB; ++b) {
      const f32x4 d = tile_dots<DT, NH, NH>(kop, qop[b]);
      float sv[4], mt = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = t0 + 4 * g + i;
        sv[i] = (j <= pos[b] && j < mmax) ? d[i] * qsc : -INFINITY;
        mt = fmaxf(mt, sv[i]);
      }
      if (mt > m[b]) {
        ls[b] *= __builtin_amdgcn_exp2f(m[b] - mt);
        m[b] = mt;
      }
      if (m[b] != -INFINITY) {
#pragma unroll
        for (int i = 0; i < 4; ++i) ls[b] += __builtin_amdgcn_exp2f(sv[i] - m[b]);
      }
    }
  };
  for (int t0 = k0; t0 < k1; t0 += 48) {
    load_tile<DT>(rk, p.k_st, t0 + 32, g, n, kt[2], cov_xs<DT>(p, 1));
    tile(t0, kt[0]);
    if (t0 + 16 >= k1) break;
    load_tile<DT>(rk, p.k_st, t0 + 48, g, n, kt[0], cov_xs<DT>(p, 1));
    tile(t0 + 16, kt[1]);
    if (t0 + 32 >= k1) break;
    load_tile<DT>(rk, p.k_st, t0 + 64, g, n, kt[1], cov_xs<DT>(p, 1));
    tile(t0 + 32, kt[2]);
  }
  // lanes (0..3, n) hold disjoint keys of row n: this split's state of the row
#pragma unroll
  for (int b = 0; b < NRB; ++b) {
    const float M = xmax32(xmax16(m[b]));
    const float part = (M == -INFINITY || m[b] == -INFINITY) ? 0.0f : ls[b] * __builtin_amdgcn_exp2f(m[b] - M);
    const float L = xsum32(xsum16(part));
    if (g == 0) {
      st[wave][b][n][0] = M;
      st[wave][b][n][1] = L;
    }
  }
  __syncthreads();
  // thread t < 64: row t % 16 of the item's block t / 16, its splits combined in order
  if (threadIdx.x < 64) {
    const int rbi = threadIdx.x / 16, row = threadIdx.x % 16;
    const int rg = rbi / NRB, b = rbi % NRB;
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < KS; ++s) M = fmaxf(M, st[rg * KS + s][b][row][0]);
    float L = 0.0f;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const float ms = st[rg * KS + s][b][row][0];
      if (ms != -INFINITY) L += st[rg * KS + s][b][row][1] * __builtin_amdgcn_exp2f(ms - M);
    }
    const int rl = 64 * rb + 16 * rbi;
    const int r_abs = gt[0] + rl + row;
    if (rl < rows_g && r_abs < p.NR) {
      const int64_t o = static_cast<int64_t>(h) * p.NR + r_abs;
      p.row_m[o] = M == -INFINITY ? 0.0f : M;                // padding rows: every p is masked to 0 below
      p.row_il[o] = L > 0.0f ? 1.0f / L : 0.0f;
    }
  }
}

// values of one 32-key step in LDS: [key][channel].  fp32 rows are padded by 8 bytes against bank
// conflicts; 16-bit rows take 288 bytes (72 words), so that the transposed reads of a channel block
// (16 lanes reading 8 bytes each of 4 keys x 4 channel quads) fall on distinct banks
template <int DT>
constexpr int vrow_words() { return DT == KVQ_F32 ? (kCD * 4 + 8) / 4 : 72; }

typedef short tr16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) tr16x4 lds_tr16x4;

template <int DT>
__global__ __launch_bounds__(kCThreads) void cov_output(CovParams p) {
  constexpr int ESZ = TileOps<DT>::ESZ;
  constexpr int VRW = vrow_words<DT>();
  constexpr int U16 = kCD * ESZ / 16;                        // 16-byte units of a value row
  __shared__ __align__(16) uint32_t vt[32 * VRW];
  const int wave = threadIdx.x / 64, l = threadIdx.x % 64, g = l >> 4, n = l & 15;
  // work units (h, item, key split), h outermost; the items in reverse plan order, so the groups at
  // the end of the context, whose keys reach furthest, start first and the short ones fill the tail
  const int unit = xcd_unit(p.Hkv * kOSplit * p.n_items);
  if (unit < 0) return;
  const int h = unit / (p.n_items * kOSplit), w = unit % (p.n_items * kOSplit);
  const int item = p.n_items - 1 - w / kOSplit, sp = w % kOSplit;
  const int grp = p.items[2 * item], rb = p.items[2 * item + 1];
  const int32_t* gt = p.gtab + kGT * grp;
  const int rows_g = p.rep * gt[2];
  const int row0 = gt[0] + 64 * rb + 16 * wave;
  const bool active = 64 * rb + 16 * wave < rows_g;        // inactive wavefronts still join the barriers
  u32x4 qop[4][TileOps<DT>::NH];
  int pos = -1;
  if (active)
    pos = load_rows<DT>(p, h, row0, g, n, qop);
  else
    zero_ops<DT>(qop);
  const float rm = (active && row0 + n < p.NR) ? p.row_m[static_cast<int64_t>(h) * p.NR + row0 + n] : 0.0f;
  const int mmax = gt[3];
  // this workgroup's keys: split sp of the item's 32-key steps (every split writes its partial,
  // zeros when it holds no keys; the probabilities use the row's global maximum and sum, so the
  // partials add up to o)
  const int nstep = (mmax + 31) / 32;
  const int k0 = 32 * (nstep * sp / kOSplit), k1 = min(mmax, 32 * (nstep * (sp + 1) / kOSplit));
  const __amdgpu_buffer_rsrc_t rk = head_rsrc(p.k, p.k_sh, p.k_st, h, p.T, ESZ);
  const __amdgpu_buffer_rsrc_t rv = head_rsrc(p.v, p.v_sh, p.v_st, h, p.T, ESZ);
  const float qsc = p.qscale / (cov_xs<DT>(p, 0) * cov_xs<DT>(p, 1));   // logit scale of the scaled rows
  const float vsc = cov_xs<DT>(p, 2);
  f32x4 acc[8];
#pragma unroll
  for (int cb = 0; cb < 8; ++cb) acc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  // a step's loads: its 32 value rows (this thread's 16-byte units; rows at or past mmax as zeros:
  // p = 0 there must not meet a NaN) and this wavefront's two key tiles.  The next step's loads go
  // out as soon as the current key tiles have entered the logit products.
  constexpr int KU = (32 * U16 + kCThreads - 1) / kCThreads;
  u32x4 vr[KU];
  u32x4 kr[2][4][TileOps<DT>::NH];
  auto load_step = [&](int t0) {
#pragma unroll
    for (int k = 0; k < KU; ++k) {
      const int u = threadIdx.x + kCThreads * k;
      const int key = u / U16, w16 = u % U16;
      vr[k] = u32x4{0u, 0u, 0u, 0u};
      if (u < 32 * U16 && t0 + key < k1)
        vr[k] = __builtin_amdgcn_raw_buffer_load_b128(
            rv, static_cast<int>((static_cast<int64_t>(t0 + key) * p.v_st) * ESZ + 16 * w16), 0, 0);
    }
#pragma unroll
    for (int tau = 0; tau < 2; ++tau) load_tile<DT>(rk, p.k_st, t0 + 16 * tau, g, n, kr[tau], cov_xs<DT>(p, 1));
  };
  if (k0 < k1) load_step(k0);
  for (int t0 = k0; t0 < k1; t0 += 32) {
    // LDS-only barriers: the key tiles of the step stay in flight while its value rows are stored
    block_lds_barrier();                                     // the previous step's value rows are read
#pragma unroll
    for (int k = 0; k < KU; ++k) {
      const int u = threadIdx.x + kCThreads * k;
      if (u < 32 * U16) {
        uint32_t* dst = vt + (u / U16) * VRW + 4 * (u % U16);
        if constexpr (DT == KVQ_F32) {
          dst[0] = vr[k][0];
          dst[1] = vr[k][1];
          dst[2] = vr[k][2];
          dst[3] = vr[k][3];
        } else {
          *reinterpret_cast<u32x4*>(dst) = vr[k];                // 288-byte rows: 16-byte aligned
        }
      }
    }
    block_lds_barrier();
    // probabilities of the two 16-key tiles: lane (g, n) holds keys t0 + 4g + i and t0 + 16 + 4g + i
    // of row n
    f32x4 dd[2];
#pragma unroll
    for (int tau = 0; tau < 2; ++tau) dd[tau] = tile_dots<DT, TileOps<DT>::NH, TileOps<DT>::NH>(kr[tau], qop);
    if (t0 + 32 < k1) load_step(t0 + 32);
    float pr[8];
#pragma unroll
    for (int tau = 0; tau < 2; ++tau) {
      const f32x4 d = dd[tau];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = t0 + 16 * tau + 4 * g + i;
        pr[4 * tau + i] = (j <= pos && j < mmax) ? __builtin_amdgcn_exp2f(d[i] * qsc - rm) : 0.0f;
      }
    }
    // A operand: row n, k-index 8g + kk <-> key kk < 4 ? 4g + kk : 16 + 4g + kk - 4 (hi and lo parts)
    u32x4 ph, pl;
    f32_parts<DT>(pr, ph, pl);
    // B operand per 16-channel block cb: lane (g, n) holds the values of those keys at channel 16cb + n
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) {
      const int c = 16 * cb + n;
      if constexpr (DT == KVQ_F32) {
        float x[8];
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const int key = kk < 4 ? 4 * g + kk : 16 + 4 * g + kk - 4;
          x[kk] = __uint_as_float(vt[key * VRW + c]) * vsc;
        }
        u32x4 vh, vl;
        f32_parts<DT>(x, vh, vl);
        acc[cb] = tile_mfma<DT>(ph, vh, acc[cb]);
        acc[cb] = tile_mfma<DT>(pl, vh, acc[cb]);
        acc[cb] = tile_mfma<DT>(ph, vl, acc[cb]);
      } else {
        // LDS transpose reads (ds_read_b64_tr_b16): within each 16-lane group, lane n receives
        // element n & 3 of the 8-byte loads of lanes (n >> 2) + 4 j, j = 0..3.  Lane (g, q + 4 j)
        // therefore points at key 4g + j (then 16 + 4g + j), channels 16 cb + 4q .. + 3, and lane
        // (g, n) receives keys 4g .. 4g + 3 (16 + 4g ..) of channel 16 cb + n: the B operand
        const int src_key = 4 * g + (n >> 2), src_ch = 16 * cb + 4 * (n & 3);
        const uint32_t* a0 = vt + src_key * VRW + src_ch / 2;
        const tr16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_tr16x4*)(a0));
        const tr16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_tr16x4*)(a0 + 16 * VRW));
        const uint2 lw = __builtin_bit_cast(uint2, lo), hw = __builtin_bit_cast(uint2, hi);
        const u32x4 vb = u32x4{lw.x, lw.y, hw.x, hw.y};
        acc[cb] = tile_mfma<DT>(ph, vb, acc[cb]);
        acc[cb] = tile_mfma<DT>(pl, vb, acc[cb]);
      }
    }
  }
  if (!active) return;
  // D lane (g, n) register i: row 4g + i of the block, channel 16cb + n
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = row0 + 4 * g + i;
    if (row >= p.NR) continue;
    const float il = p.row_il[static_cast<int64_t>(h) * p.NR + row] / vsc;   // exact: vsc a power of two
    float* dst = p.o_part + ((static_cast<int64_t>(sp) * p.Hkv + h) * p.NR + row) * kCD + n;
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) dst[16 * cb] = acc[cb][i] * il;
  }
}

// v M v of the coded values on the matrix cores (the row outputs' o M stays on cov_metric): per
// (query head hr = (h, r), kVmvPer values) a workgroup stages that head's metric M transposed in LDS
// as fp16 hi + lo parts of M x 2^(8 - em) (its largest entry brought to [128, 256)); each wavefront
// then takes tiles of 16 values, every value row x scaled by its own power of two the same way and
// split into parts, y = x M by the products hi*hi + hi*lo + lo*hi (fp32 accumulation, about 2^-22
// relative), and x . y by a row sum with x exchanged through the wavefront's LDS into the layout
// of the products' output.
constexpr int kVmvPer = 512;             // values of a cov_vmv workgroup
constexpr int kMtStride = kCD + 8;       // halves per LDS row of M^T (16-byte aligned rows)

template <int DT>
__global__ __launch_bounds__(kCThreads) void cov_vmv(CovParams p) {
  __shared__ __align__(16) uint16_t mt[2][kCD * kMtStride];   // [part][col][k]
  __shared__ __align__(16) float xs[kCWaves][16][kCD + 4];
  __shared__ float red[kCWaves];
  __shared__ int xex[kCWaves][16];
  const int tiles = (p.n + kVmvPer - 1) / kVmvPer;
  const int hr = blockIdx.x / tiles, tile = blockIdx.x % tiles;
  const int h = hr / p.rep;
  const int wave = threadIdx.x / 64, l = threadIdx.x % 64, g = l >> 4, n = l & 15;
  // the metric's largest entry over the workgroup, then its transposed parts
  const float* Mg = p.M + static_cast<int64_t>(hr) * kCD * kCD;
  constexpr int kPer = kCD * kCD / kCThreads;
  float mv[kPer];
  float mx = 0.0f;
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    mv[e] = Mg[threadIdx.x + kCThreads * e];
    mx = fmaxf(mx, fabsf(mv[e]));
  }
  mx = wave_max(mx);
  if (l == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int em = 0;
  if (mx > 0.0f) (void)frexpf(mx, &em);
  const float upm = ldexpf(1.0f, 8 - em);
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int idx = threadIdx.x + kCThreads * e, k = idx / kCD, c = idx % kCD;
    const float x = mv[e] * upm;
    const _Float16 hi = static_cast<_Float16>(x);
    const _Float16 lo = static_cast<_Float16>(x - static_cast<float>(hi));
    mt[0][c * kMtStride + k] = __builtin_bit_cast(uint16_t, hi);
    mt[1][c * kMtStride + k] = __builtin_bit_cast(uint16_t, lo);
  }
  __syncthreads();
  for (int t0 = 0; t0 < kVmvPer; t0 += 64) {
    const int j0 = tile * kVmvPer + t0 + 16 * wave;         // this wavefront's 16 values
    const int j = j0 + n;                                   // lane (g, n): value n, channels 32 ks + 8 g ..
    float x[4][8];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (j < p.n) {
        load8<DT>(p.v, static_cast<int64_t>(h) * p.v_sh + static_cast<int64_t>(p.rs + j) * p.v_st + 32 * ks + 8 * g,
                  x[ks]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[ks][e] = 0.0f;
      }
    }
    float mxv = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) mxv = fmaxf(mxv, fabsf(x[ks][e]));
    mxv = xmax32(xmax16(mxv));                               // over the four lanes of value n
    int ex = 0;
    if (mxv > 0.0f) (void)frexpf(mxv, &ex);
    const float upx = ldexpf(1.0f, 8 - ex);
    u32x4 xh[4], xl[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      float xs8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) xs8[e] = x[ks][e] * upx;
      f32_parts<KVQ_F16>(xs8, xh[ks], xl[ks]);
      *reinterpret_cast<float4*>(&xs[wave][n][32 * ks + 8 * g]) = make_float4(xs8[0], xs8[1], xs8[2], xs8[3]);
      *reinterpret_cast<float4*>(&xs[wave][n][32 * ks + 8 * g + 4]) = make_float4(xs8[4], xs8[5], xs8[6], xs8[7]);
    }
    if (g == 0) xex[wave][n] = ex;
    wave_lds_fence();
    float dot[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) {
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int o = (16 * cb + n) * kMtStride + 32 * ks + 8 * g;
        const u32x4 bh = *reinterpret_cast<const u32x4*>(&mt[0][o]);
        const u32x4 bl = *reinterpret_cast<const u32x4*>(&mt[1][o]);
        acc = mfma(as_half8(xh[ks]), as_half8(bh), acc);
        acc = mfma(as_half8(xh[ks]), as_half8(bl), acc);
        acc = mfma(as_half8(xl[ks]), as_half8(bh), acc);
      }
      // D lane (g, n) register i: value 4g + i, column 16 cb + n
#pragma unroll
      for (int i = 0; i < 4; ++i) dot[i] = __builtin_fmaf(acc[i], xs[wave][4 * g + i][16 * cb + n], dot[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float q = row_sum16(dot[i]);                    // over the 16 columns a lane group holds
      const int jj = j0 + 4 * g + i;
      if (n == 0 && jj < p.n) {
        // x M x = q x 2^(2 ex + em - 24): x and M entered as x 2^(8 - ex) and M 2^(8 - em)
        p.vmv[static_cast<int64_t>(hr) * p.n + jj] = ldexpf(q, 2 * xex[wave][4 * g + i] + em - 24);
      }
    }
    wave_lds_fence();                                       // xs, xex of this tile are read
  }
}

// x M and x M x for 32 vectors per workgroup, M = the metric of query head (h, r) staged in LDS in
// two halves of 64 rows.  ROWS: the row outputs of query head r (o M replaces o, o M o out);
// otherwise the coded values (v M v out).  Grid: (h, r, tile of 32 vectors).
template <int DT, bool ROWS>
__global__ __launch_bounds__(kCThreads) void cov_metric(CovParams p, const int32_t* rlist, int n_rlist) {
  constexpr int XS = kCD + 1;                          // odd stride: the rows' reads hit distinct banks
  __shared__ float Ms[64 * kCD];                       // 32 KiB
  __shared__ float xs[kMetricRows * XS];
  __shared__ float red[kMetricRows][8];
  const int count = ROWS ? n_rlist : p.n;
  const int per = (count + kMetricRows - 1) / kMetricRows;
  const int hr = blockIdx.x / per, tile = blockIdx.x % per;
  const int h = hr / p.rep, r = hr % p.rep;
  const float* Mg = p.M + static_cast<int64_t>(h * p.rep + r) * kCD * kCD;
  const int32_t* rl = ROWS ? rlist + static_cast<int64_t>(r) * n_rlist : nullptr;
  for (int u = threadIdx.x; u < kMetricRows * kCD; u += kCThreads) {
    const int k = u / kCD, c = u % kCD;
    const int idx = kMetricRows * tile + k;
    float x = 0.0f;
    if (idx < count) {
      if constexpr (ROWS) {
        if (rl[idx] >= 0) {                            // the key splits' outputs, summed in order
          const int64_t o = (static_cast<int64_t>(h) * p.NR + rl[idx]) * kCD + c;
          const int64_t split = static_cast<int64_t>(p.Hkv) * p.NR * kCD;
#pragma unroll
          for (int sp = 0; sp < kOSplit; ++sp) x += p.o_part[sp * split + o];
        }
      } else {
        x = load_as_f32<DT>(p.v, static_cast<int64_t>(h) * p.v_sh + static_cast<int64_t>(p.rs + idx) * p.v_st + c);
      }
    }
    xs[k * XS + c] = x;
  }
  // thread: vector k = t / 8, output channels 16 (t % 8) .. + 15
  const int k = threadIdx.x / 8, c8 = threadIdx.x % 8;
  float y[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) y[e] = 0.0f;
  for (int hf = 0; hf < 2; ++hf) {
    __syncthreads();
    for (int u = threadIdx.x; u < 64 * kCD / 4; u += kCThreads)
      reinterpret_cast<float4*>(Ms)[u] = reinterpret_cast<const float4*>(Mg + 64 * hf * kCD)[u];
    __syncthreads();
    for (int d = 0; d < 64; ++d) {
      const float xd = xs[k * XS + 64 * hf + d];
      const float4* mr = reinterpret_cast<const float4*>(Ms + d * kCD + 16 * c8);
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const float4 mv = mr[e4];
        y[4 * e4] = __builtin_fmaf(xd, mv.x, y[4 * e4]);
        y[4 * e4 + 1] = __builtin_fmaf(xd, mv.y, y[4 * e4 + 1]);
        y[4 * e4 + 2] = __builtin_fmaf(xd, mv.z, y[4 * e4 + 2]);
        y[4 * e4 + 3] = __builtin_fmaf(xd, mv.w, y[4 * e4 + 3]);
      }
    }
  }
  float dot = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) dot = __builtin_fmaf(y[e], xs[k * XS + 16 * c8 + e], dot);
  red[k][c8] = dot;
  __syncthreads();
  const int idx = kMetricRows * tile + k;
  if (idx >= count) return;
  const float tot = ((red[k][0] + red[k][1]) + (red[k][2] + red[k][3])) +
                    ((red[k][4] + red[k][5]) + (red[k][6] + red[k][7]));
  if constexpr (ROWS) {
    if (rl[idx] < 0) return;
    const int64_t rid = static_cast<int64_t>(h) * p.NR + rl[idx];
    float* dst = p.o + rid * kCD + 16 * c8;             // this workgroup staged its rows before any write
#pragma unroll
    for (int e = 0; e < 16; ++e) dst[e] = y[e];
    if (c8 == 0) p.oMo[rid] = tot;
  } else {
    if (c8 == 0) p.vmv[(static_cast<int64_t>(h) * p.rep + r) * p.n + idx] = tot;
  }
}

__global__ __launch_bounds__(kCThreads) void cov_clear(float* x, int64_t count) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kCThreads + threadIdx.x;
  if (t < count) x[t] = 0.0f;
}

// the weighted pass's group splits summed in split order: A, DD (Hkv, n) and WVa (Hkv, rep, n)
__global__ __launch_bounds__(kCThreads) void cov_split_sums(CovParams p) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kCThreads + threadIdx.x;
  const int64_t nA = static_cast<int64_t>(p.Hkv) * p.n, nW = nA * p.rep;
  if (t < nA) {
    float a = 0.0f, dd = 0.0f;
#pragma unroll
    for (int s = 0; s < kTSplit; ++s) {
      a += p.A_part[s * nA + t];
      dd += p.DD_part[s * nA + t];
    }
    p.A[t] = a;
    p.DD[t] = dd;
  }
  if (t < nW) {
    float w = 0.0f;
#pragma unroll
    for (int s = 0; s < kTSplit; ++s) w += p.WVa_part[s * nW + t];
    p.WVa[t] = w;
  }
}

// Once per row (after cov_metric): o M as the A operand of cov_terms' v.(oM) products -- times a
// power of two that brings its largest entry to [128, 256) (inside the range of fp16 parts), in two
// parts of the operand type -- and the row's values as one float4 (row max, 1 / sum, o M o, the
// power of two back).  Thread (row, ks, g) converts channels 32 ks + 8 g .. + 7; a row's 16 threads
// are one DPP row of a wavefront.
template <int DT>
__global__ __launch_bounds__(kCThreads) void cov_rowprep(CovParams p) {
  const int64_t rid = static_cast<int64_t>(blockIdx.x) * (kCThreads / 16) + threadIdx.x / 16;
  const int sl = threadIdx.x % 16, ks = sl / 4, g = sl % 4;
  if (rid >= static_cast<int64_t>(p.Hkv) * p.NR) return;          // whole rows: 16 lanes alike
  const float4* src = reinterpret_cast<const float4*>(p.o + rid * kCD + 32 * ks + 8 * g);
  const float4 a = src[0], b = src[1];
  float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  float mx = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(x[e]));
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  int ex = 0;
  if (mx > 0.0f) (void)frexpf(mx, &ex);
  const float up = ldexpf(1.0f, 8 - ex);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] *= up;
  u32x4 hi, lo;
  f32_parts<DT>(x, hi, lo);
  u32x4* dst = reinterpret_cast<u32x4*>(p.mop) + rid * 32 + (ks * 4 + g) * 2;
  dst[0] = hi;
  dst[1] = lo;
  if (sl == 0)
    reinterpret_cast<float4*>(p.rowf)[rid] = make_float4(p.row_m[rid], p.row_il[rid], p.oMo[rid], ldexpf(1.0f, ex - 8));
}

// per (h, 256-token chunk, group split): every group reaching the chunk, its rows in 64-row blocks
// (one 16-row block per wavefront, one query head per block since nq_pad is a multiple of 16),
// 16-token tiles.  WEIGHTED = false: drop totals (one partial per wavefront, combined in order by
// cov_groups) and key-term masses; true: the weighted per-token sums.
// LDS (16-bit keys and values, rep <= kTermsLdsRep): the chunk's 256 key and value rows (128 KiB)
// and its v M v of every query head are staged in LDS once, and every group and wavefront reads its
// tiles there (a tile used to come from L2 once per group and wavefront); the weighted pass also
// keeps its read masses there until the end.  Row t of a tensor holds its 16-byte column c at
// c ^ (t & 15), so the 16 tokens of a tile read in one instruction fall on distinct banks.  The workgroup is two quads of wavefronts (two per SIMD, so one's products overlap
// the other's terms): for the drop totals the quads take alternate groups with work; for the weighted
// sums every group, quad q the tokens [c0 + 128 q, c0 + 128 q + 128), a lane's sums over the groups
// kept in registers and added across the lane groups once at the end.  LDS = false: tiles and v M v
// from memory, one tile ahead, one quad, a token's sums over the groups in LDS.
template <int DT, bool WEIGHTED, bool LDS>
__global__ __launch_bounds__(LDS ? 2 * kCThreads : kCThreads) void cov_terms(CovParams p) {
  constexpr int NH = TileOps<DT>::NH;
  static_assert(!LDS || NH == 1, "LDS tiles hold 16-bit rows");
  constexpr int NT = LDS ? 2 * kCThreads : kCThreads;
  __shared__ u32x4 kv_lds[LDS ? 2 * kChunkTok * 16 : 1];         // [K, V][token][16-byte column]
  __shared__ float vmv_lds[LDS ? kTermsLdsRep * kChunkTok : 1];  // [query head][token]
  __shared__ float wva_lds[LDS && WEIGHTED ? kTermsLdsRep * kChunkTok : 1];   // read masses [head][token]
  __shared__ float accA[kCWaves][kChunkTok];
  __shared__ float accD[kCWaves][kChunkTok];
  __shared__ float accW[kCWaves][kChunkTok];             // read mass of the wavefront's current block
  const int wave = threadIdx.x / 64, l = threadIdx.x % 64, g = l >> 4, n = l & 15;
  const int quad = wave / kCWaves, wq = wave % kCWaves;
  // groups ts, ts + kTSplit, ... of (h, chunk): the chunks near the start, which every group reaches,
  // spread over kTSplit workgroups.  Work units u = (h, chunk, ts) in order; block b runs on XCD b % 8
  // (round-robin dispatch), and each XCD takes a contiguous range of units, so the splits of a chunk
  // share one L2 and its key and value tiles stay there.
  const int u = xcd_unit(p.Hkv * p.n_chunks * kTSplit);
  if (u < 0) return;
  const int ts = u % kTSplit;
  const int h = u / kTSplit / p.n_chunks, chunk = u / kTSplit % p.n_chunks;
  const int c0 = p.rs + chunk * kChunkTok;               // first token of the chunk
  const int c1 = min(c0 + kChunkTok, p.re);
  const __amdgpu_buffer_rsrc_t rk = head_rsrc(p.k, p.k_sh, p.k_st, h, p.T, TileOps<DT>::ESZ);
  const __amdgpu_buffer_rsrc_t rv = head_rsrc(p.v, p.v_sh, p.v_st, h, p.T, TileOps<DT>::ESZ);
  const float qsc = p.qscale / (cov_xs<DT>(p, 0) * cov_xs<DT>(p, 1));   // logit scale of the scaled rows
  if constexpr (WEIGHTED) {
    for (int u = threadIdx.x; u < kCWaves * kChunkTok; u += NT) {
      (&accA[0][0])[u] = 0.0f;
      (&accD[0][0])[u] = 0.0f;
    }
    if constexpr (LDS)
      for (int u = threadIdx.x; u < kTermsLdsRep * kChunkTok; u += NT) wva_lds[u] = 0.0f;
  }
  // weighted LDS form: every group with work has 16 padded queries, so a wavefront's 16 rows are one
  // query head and a head's read masses only ever come from one wavefront (no barrier between blocks)
  bool solo = LDS && WEIGHTED;
  // a group has work in this chunk if it reaches it (and, weighted, has a nonzero weight)
  auto has_work = [&](int grp) { return p.gtab[kGT * grp + 4] > c0 && (!WEIGHTED || p.gw[grp] != 0.0f); };
  if constexpr (LDS) {
    bool used = false;                                   // some group of this split reaches the chunk
    for (int grp = ts; grp < p.G; grp += kTSplit) {
      const bool w = has_work(grp);
      used = used || w;
      solo = solo && (!w || p.gtab[kGT * grp + 2] == 16);
    }
    if (used) {
      // 16-byte unit u = (tensor, token, column): all of a thread's loads issued before its stores
      constexpr int kPer = 2 * kChunkTok * 16 / NT;
      u32x4 x[kPer];
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int u = i * NT + static_cast<int>(threadIdx.x);
        const int tok = (u >> 4) & (kChunkTok - 1), col = u & 15;
        const bool key = u < kChunkTok * 16;
        const int64_t off = (static_cast<int64_t>(c0 + tok) * (key ? p.k_st : p.v_st) + 8 * col) * 2;
        x[i] = __builtin_amdgcn_raw_buffer_load_b128(key ? rk : rv, static_cast<int>(off), 0, 0);
      }
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int u = i * NT + static_cast<int>(threadIdx.x);
        const int tok = (u >> 4) & (kChunkTok - 1), col = u & 15;
        kv_lds[((u < kChunkTok * 16 ? 0 : kChunkTok) + tok) * 16 + (col ^ (tok & 15))] = x[i];
      }
      for (int u = threadIdx.x; u < p.rep * kChunkTok; u += NT) {
        const int r = u / kChunkTok, j = c0 + u % kChunkTok;
        vmv_lds[u] = j < c1 ? p.vmv[(static_cast<int64_t>(h) * p.rep + r) * p.n + (j - p.rs)] : 0.0f;
      }
    }
    __syncthreads();
  }
  int n_work = 0;                                        // groups with work so far (drop totals, LDS)
  // weighted LDS form: this lane's token sums over the groups, tile by tile of the quad's half
  float rA[kChunkTok / 32], rD[kChunkTok / 32];
#pragma unroll
  for (int it = 0; it < kChunkTok / 32; ++it) rA[it] = rD[it] = 0.0f;
  for (int grp = ts; grp < p.G; grp += kTSplit) {
    const int32_t* gt = p.gtab + kGT * grp;
    const int row_base = gt[0], nq = gt[1], nq_pad = gt[2], te = gt[4], local = gt[5];
    const int rows_g = p.rep * nq_pad;
    const int64_t dd_at = ((static_cast<int64_t>(grp) * p.Hkv + h) * p.n_chunks + chunk) * kCWaves;
    if (te <= c0) {                                      // the group does not reach this chunk
      if constexpr (!WEIGHTED) {
        if (quad == 0) {
          for (int u = threadIdx.x; u < rows_g; u += kCThreads)
            p.alpha_part[(static_cast<int64_t>(h) * p.n_chunks + chunk) * p.NR + row_base + u] = 0.0f;
          if (threadIdx.x < kCWaves) p.ddpart[dd_at + threadIdx.x] = 0.0f;
        }
      }
      continue;
    }
    if (WEIGHTED && p.gw[grp] == 0.0f) continue;        // N = 0: every term of the group is zero
    if constexpr (LDS && !WEIGHTED) {
      if ((n_work++ & 1) != quad) continue;              // the other quad's group
    }
    const int t_end = min(c1, te);
    // the tiles of this quad: weighted LDS form, its half of the chunk
    const int ta0 = LDS && WEIGHTED ? c0 + (kChunkTok / 2) * quad : c0;
    const int ta1 = LDS && WEIGHTED ? min(t_end, ta0 + kChunkTok / 2) : t_end;
    const float wq_w = (WEIGHTED ? p.gw[grp] : 1.0f) / static_cast<float>(nq);
    float dsum = 0.0f;                                   // drop terms of this wavefront (pass A)
    for (int rb0 = 0; rb0 < rows_g; rb0 += 64) {
      const int rbl = rb0 + 16 * wq;                      // this wavefront's first row in the group
      const bool act = rbl < rows_g;
      const int r = act ? rbl / nq_pad : 0;
      const int row0 = row_base + rbl;
      // operands (lane n: row n of the block, channels 8g + 32 ks ..) as the A side of the products,
      // the token tiles as the B side: the results hold rows 4g + i of token n in lane (g, n), so a
      // token's sums over the rows are three in-lane adds and two cross-group steps, and a row's sums
      // over the tokens stay in the lane until the block's end
      u32x4 qop[4][NH], mop[4][2];
      int pos[4];
      float rm[4], ril[4], omo[4], msc[4];
      if (act) {
        // row n's operands and rows 4g + i's values, prepared once per row by cov_rowprep: one
        // round of independent loads
        (void)load_rows<DT>(p, h, row0, g, n, qop);
        const u32x4* mp = reinterpret_cast<const u32x4*>(p.mop) + (static_cast<int64_t>(h) * p.NR + row0 + n) * 32;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          mop[ks][0] = mp[(ks * 4 + g) * 2];
          mop[ks][1] = mp[(ks * 4 + g) * 2 + 1];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = row0 + 4 * g + i;
          const float4 f = reinterpret_cast<const float4*>(p.rowf)[static_cast<int64_t>(h) * p.NR + row];
          pos[i] = p.rowpos[row];
          rm[i] = f.x;
          ril[i] = f.y;
          omo[i] = f.z;
          msc[i] = f.w / cov_xs<DT>(p, 2);                  // v M o of the scaled values: exact
        }
      } else {
        zero_ops<DT>(qop);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) mop[ks][0] = mop[ks][1] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pos[i] = -1;
          rm[i] = ril[i] = omo[i] = 0.0f;
          msc[i] = 1.0f;
        }
      }
      if constexpr (WEIGHTED && !LDS) {
        for (int u = l; u < kChunkTok; u += 64) accW[wq][u] = 0.0f;
        wave_lds_fence();
      }
      float alpha[4] = {0.0f, 0.0f, 0.0f, 0.0f};          // key-term mass of rows 4g + i (pass A)
      // a tile's operands (key and value tiles, v M v of this lane's token); the next tile's are
      // fetched as soon as the current tiles have entered the matrix products
      const int64_t vmv_base = (static_cast<int64_t>(h) * p.rep + r) * p.n - p.rs;   // + token j
      u32x4 kop[4][NH], vop[4][NH];
      float vmv1;
      auto load_t = [&](int t0) {
        const int j = t0 + n;
        if constexpr (LDS) {
          const int row = t0 - c0 + n;                     // (t0 - c0) % 16 == 0: row & 15 == n
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            kop[ks][0] = kv_lds[row * 16 + ((4 * ks + g) ^ n)];
            vop[ks][0] = kv_lds[(kChunkTok + row) * 16 + ((4 * ks + g) ^ n)];
          }
          vmv1 = (act && j < t_end) ? vmv_lds[r * kChunkTok + row] : 0.0f;
        } else {
          load_tile<DT>(rk, p.k_st, t0, g, n, kop, cov_xs<DT>(p, 1));
          load_tile<DT>(rv, p.v_st, t0, g, n, vop, cov_xs<DT>(p, 2));
          vmv1 = (act && j < t_end) ? p.vmv[vmv_base + j] : 0.0f;
        }
      };
      // the terms of (row 4g + i, token t0 + n) from the tile's products
      auto terms = [&](int t0, const f32x4& s, const f32x4& ov, float vmv, float (&ta)[4], float (&td)[4],
                       float (&tw)[4]) {
        const int j = t0 + n;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool far = act && j < t_end && j <= pos[i] - local;
          const float pr = far ? __builtin_amdgcn_exp2f(s[i] * qsc - rm[i]) * ril[i] : 0.0f;
          const float u2 = far ? fmaxf(vmv - 2.0f * (ov[i] * msc[i]) + omo[i], 0.0f) : 0.0f;
          // pr / b for b = max(1 - pr, 1e-6) in [1e-6, 1]: the reciprocal's quotient and one
          // residual correction (no subnormal, infinite or zero operand can occur)
          const float qb = fmaxf(1.0f - pr, 1e-6f), rb = __builtin_amdgcn_rcpf(qb);
          const float q0 = pr * rb;
          const float qd = __builtin_fmaf(__builtin_fmaf(-qb, q0, pr), rb, q0);
          td[i] = qd * qd * u2;
          ta[i] = pr * pr * u2;
          tw[i] = pr * pr;
        }
      };
      if constexpr (LDS && WEIGHTED) {
        // the quad's eight tiles unrolled: token t0 + n's sums over the groups stay in registers, each
        // lane's four rows apart from the other lane groups' until the workgroup ends (a masked token
        // adds +0)
        float wr[kChunkTok / 32];
        if (ta0 < ta1) load_t(ta0);
#pragma unroll
        for (int it = 0; it < kChunkTok / 32; ++it) {
          const int t0 = ta0 + 16 * it;
          wr[it] = 0.0f;
          if (t0 < ta1) {
            const f32x4 s = tile_dots<DT, NH, NH>(qop, kop);
            const f32x4 ov = tile_dots<DT, 2, NH>(mop, vop);
            const float vmv = vmv1;
            if (t0 + 16 < ta1) load_t(t0 + 16);
            float ta[4], td[4], tw[4];
            terms(t0, s, ov, vmv, ta, td, tw);
            rA[it] += ((ta[0] + ta[1]) + (ta[2] + ta[3])) * wq_w;
            rD[it] += ((td[0] + td[1]) + (td[2] + td[3])) * wq_w;
            wr[it] = ((tw[0] + tw[1]) + (tw[2] + tw[3])) * wq_w;
          }
        }
        // the block's read mass of token t0 + n: the four lane groups' rows added
#pragma unroll
        for (int it = 0; it < kChunkTok / 32; ++it) wr[it] = xsum32(xsum16(wr[it]));
        if (solo) {
          if (g == 0 && act) {
#pragma unroll
            for (int it = 0; it < kChunkTok / 32; ++it) wva_lds[r * kChunkTok + ta0 - c0 + 16 * it + n] += wr[it];
          }
        } else if (g == 0) {
#pragma unroll
          for (int it = 0; it < kChunkTok / 32; ++it) accW[wq][ta0 - c0 + 16 * it + n] = wr[it];
        }
      } else {
        if (ta0 < ta1) load_t(ta0);
        for (int t0 = ta0; t0 < ta1; t0 += 16) {
          const f32x4 s = tile_dots<DT, NH, NH>(qop, kop);
          const f32x4 ov = tile_dots<DT, 2, NH>(mop, vop);
          const float vmv = vmv1;
          if (t0 + 16 < ta1) load_t(t0 + 16);
          const int j = t0 + n;
          float ta[4], td[4], tw[4];
          terms(t0, s, ov, vmv, ta, td, tw);
          if constexpr (!WEIGHTED) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              dsum += td[i];
              alpha[i] += ta[i];
            }
          } else {
            // token t0 + n: its sums over the block's 16 rows (the lane's four, then the lane groups')
            float sa = (ta[0] + ta[1]) + (ta[2] + ta[3]);
            float sd = (td[0] + td[1]) + (td[2] + td[3]);
            float sw = (tw[0] + tw[1]) + (tw[2] + tw[3]);
            sa = xsum32(xsum16(sa));
            sd = xsum32(xsum16(sd));
            sw = xsum32(xsum16(sw));
            if (g == 0 && act && j < t_end) {
              accA[wq][j - c0] += sa * wq_w;
              accD[wq][j - c0] += sd * wq_w;
              accW[wq][j - c0] += sw * wq_w;
            }
          }
        }
      }
      if constexpr (!WEIGHTED) {
        // rows 4g + i: their key-term mass over this chunk (the 16 lanes of group g hold its tokens)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float a_row = row_sum16(alpha[i]);
          if (act && n == 0)
            p.alpha_part[(static_cast<int64_t>(h) * p.n_chunks + chunk) * p.NR + row0 + 4 * g + i] =
                a_row / static_cast<float>(nq);
        }
      } else if (!solo) {
        // the wavefronts' read masses into their query heads' rows of WVa, in wavefront order (LDS:
        // kept in LDS until the workgroup ends, then stored once)
        __syncthreads();
        for (int u = threadIdx.x; u < t_end - c0; u += NT) {
          for (int w = 0; w < kCWaves; ++w) {
            const int rbw = rb0 + 16 * w;
            if (rbw >= rows_g) break;
            if constexpr (LDS)
              wva_lds[(rbw / nq_pad) * kChunkTok + u] += accW[w][u];
            else
              p.WVa_part[((static_cast<int64_t>(ts) * p.Hkv + h) * p.rep + rbw / nq_pad) * p.n + (c0 + u - p.rs)] +=
                  accW[w][u];
          }
        }
        __syncthreads();
      }
    }
    if constexpr (!WEIGHTED) {
      dsum = wave_sum(dsum);                             // cov_groups adds the four in order
      if (l == 0) p.ddpart[dd_at + wq] = dsum;
    }
  }
  if constexpr (WEIGHTED) {
    if constexpr (LDS) {
#pragma unroll
      for (int it = 0; it < kChunkTok / 32; ++it) {
        rA[it] = xsum32(xsum16(rA[it]));
        rD[it] = xsum32(xsum16(rD[it]));
      }
      if (g == 0) {
        const int tb = (kChunkTok / 2) * quad;
#pragma unroll
        for (int it = 0; it < kChunkTok / 32; ++it) {
          accA[wq][tb + 16 * it + n] = rA[it];
          accD[wq][tb + 16 * it + n] = rD[it];
        }
      }
    }
    __syncthreads();
    if constexpr (LDS) {
      // this workgroup is the only writer of its (split, h, heads, chunk) read masses
      for (int u = threadIdx.x; u < p.rep * kChunkTok; u += NT) {
        const int r = u / kChunkTok, t = u % kChunkTok;
        if (c0 + t < c1) p.WVa_part[((static_cast<int64_t>(ts) * p.Hkv + h) * p.rep + r) * p.n + (c0 + t - p.rs)] = wva_lds[u];
      }
    }
    for (int u = threadIdx.x; u < c1 - c0; u += NT) {
      const int64_t o = (static_cast<int64_t>(ts) * p.Hkv + h) * p.n + (c0 + u - p.rs);
      p.A_part[o] = (accA[0][u] + accA[1][u]) + (accA[2][u] + accA[3][u]);
      p.DD_part[o] = (accD[0][u] + accD[1][u]) + (accD[2][u] + accD[3][u]);
    }
  }
}

// N per group (over heads and chunks) -> weight 1 / N (0 if N = 0) in gw[group], and whether the
// group is live (N > 0) in gw[G + 1 + group]; one workgroup per group
__global__ __launch_bounds__(kCThreads) void cov_groups(CovParams p) {
  __shared__ float red[kCWaves];
  const int grp = blockIdx.x;
  const int per = p.Hkv * p.n_chunks;
  // the drop total of (group, h, chunk): cov_terms' four wavefront partials, in order, over nq
  const float nq = static_cast<float>(p.gtab[kGT * grp + 1]);
  float s = 0.0f;
  for (int u = threadIdx.x; u < per; u += kCThreads) {
    const float* d = p.ddpart + (static_cast<int64_t>(grp) * per + u) * kCWaves;
    s += ((d[0] + d[1]) + (d[2] + d[3])) / nq;
  }
  s = wave_sum(s);
  if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float N = (red[0] + red[1]) + (red[2] + red[3]);
    p.gw[grp] = N > 0.0f ? 1.0f / N : 0.0f;
    p.gw[p.G + 1 + grp] = N > 0.0f ? 1.0f : 0.0f;
  }
}

// per row: its group's weight x its key-term mass (summed over the chunks)
__global__ __launch_bounds__(kCThreads) void cov_roww(CovParams p, const int32_t* rowgrp) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kCThreads + threadIdx.x;
  if (t >= static_cast<int64_t>(p.Hkv) * p.NR) return;
  const int h = static_cast<int>(t / p.NR), row = static_cast<int>(t % p.NR);
  const int grp = rowgrp[row];
  if (grp < 0 || p.rowpos[row] < 0) {
    p.roww[t] = 0.0f;
    return;
  }
  float a = 0.0f;
  for (int c = 0; c < p.n_chunks; ++c) a += p.alpha_part[(static_cast<int64_t>(h) * p.n_chunks + c) * p.NR + row];
  p.roww[t] = a * p.gw[grp];
}

// S[h] = sum over rows of roww * (scaling q)(scaling q)^T: per (h, 16 output rows, row split), 64
// rows per stage staged with 16-byte loads; each split writes its partial sum, cov_smat_sum adds the
// splits in order
template <int DT>
__global__ __launch_bounds__(kCThreads) void cov_smat(CovParams p) {
  constexpr int ESZ = TileOps<DT>::ESZ;
  constexpr int U = kCD * ESZ / 16;                     // 16-byte units of a row
  __shared__ float qs[64][kCD + 4];
  __shared__ float ws[64];
  const int sp = blockIdx.x % kSSplit, c1b = blockIdx.x / kSSplit % (kCD / 16);
  const int h = blockIdx.x / kSSplit / (kCD / 16);
  const int c1 = 16 * c1b + threadIdx.x / 16, c2 = 8 * (threadIdx.x % 16);   // 8 output columns per thread
  const int per = (p.NR + 64 * kSSplit - 1) / (64 * kSSplit) * 64;            // rows of a split, whole stages
  const int rb = sp * per, re = min(p.NR, rb + per);
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
  for (int r0 = rb; r0 < re; r0 += 64) {
    __syncthreads();
    for (int u = threadIdx.x; u < 64 * U; u += kCThreads) {
      const int k = u / U, w = u % U;
      const int row = r0 + k;
      float x[16 / ESZ];
      const bool live = row < re && p.rowpos[row] >= 0;
      if constexpr (DT == KVQ_F32) {
        const float4 v = live ? *reinterpret_cast<const float4*>(static_cast<const float*>(p.qr) +
                                                                 (static_cast<int64_t>(h) * p.NR + row) * kCD + 4 * w)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
        x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
      } else {
        if (live) {
          load8<DT>(p.qr, (static_cast<int64_t>(h) * p.NR + row) * kCD + 8 * w, x);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = 0.0f;
        }
      }
#pragma unroll
      for (int e = 0; e < 16 / ESZ; ++e) qs[k][(16 / ESZ) * w + e] = x[e] * p.scaling;
    }
    if (threadIdx.x < 64)
      ws[threadIdx.x] = r0 + static_cast<int>(threadIdx.x) < re ? p.roww[static_cast<int64_t>(h) * p.NR + r0 + threadIdx.x] : 0.0f;
    __syncthreads();
    for (int k = 0; k < 64; ++k) {
      const float a = ws[k] * qs[k][c1];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = __builtin_fmaf(a, qs[k][c2 + e], acc[e]);
    }
  }
  float* dst = p.S_part + ((static_cast<int64_t>(sp) * p.Hkv + h) * kCD + c1) * kCD + c2;
#pragma unroll
  for (int e = 0; e < 8; ++e) dst[e] = acc[e];
}

__global__ __launch_bounds__(kCThreads) void cov_smat_sum(CovParams p) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kCThreads + threadIdx.x;
  const int64_t total = static_cast<int64_t>(p.Hkv) * kCD * kCD;
  if (t >= total) return;
  float a = 0.0f;
#pragma unroll
  for (int sp = 0; sp < kSSplit; ++sp) a += p.S_part[sp * total + t];
  p.S[t] = a;
}

// finalisation sums: red[0..2] the means of the live-averaged A, DD, W; red[3] the live count;
// red[4 + h rep + r] omega (live-averaged read mass per query head); red[4 + Hkv rep + h] sum_j A
// (live-averaged).  First every per-head sum over the n tokens, one workgroup each (sums[h][0] A,
// [1] DD, [2 + r] the read mass of query head r), then one thread combines them in a fixed order.
__global__ __launch_bounds__(1024) void cov_final_sums(CovParams p) {
  __shared__ float part[16];
  const int nk = 2 + p.rep;
  const int h = blockIdx.x / nk, kind = blockIdx.x % nk;
  const float* src = kind == 0 ? p.A + static_cast<int64_t>(h) * p.n
                   : kind == 1 ? p.DD + static_cast<int64_t>(h) * p.n
                               : p.WVa + (static_cast<int64_t>(h) * p.rep + (kind - 2)) * p.n;
  float v = 0.0f;
  for (int j = threadIdx.x; j < p.n; j += 1024) v += src[j];
  v = wave_sum(v);
  if (threadIdx.x % 64 == 0) part[threadIdx.x / 64] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.0f;
    for (int w = 0; w < 16; ++w) t += part[w];
    p.sums[blockIdx.x] = t;
  }
}

__global__ void cov_final_combine(CovParams p) {
  if (threadIdx.x != 0) return;
  float live = 0.0f;                                      // live groups, counted in group order
  for (int g = 0; g < p.G; ++g) live += p.gw[p.G + 1 + g];
  live = fmaxf(live, 1.0f);
  const int nk = 2 + p.rep;
  float gA = 0.0f, gD = 0.0f, gW = 0.0f;
  for (int h = 0; h < p.Hkv; ++h) {
    const float sA = p.sums[h * nk], sD = p.sums[h * nk + 1];
    float sW = 0.0f;
    for (int r = 0; r < p.rep; ++r) {
      const float om = p.sums[h * nk + 2 + r];
      p.red[4 + h * p.rep + r] = om / live;
      sW += om;
    }
    p.red[4 + p.Hkv * p.rep + h] = sA / live;
    gA += sA;
    gD += sD;
    gW += sW;
  }
  const float cnt = static_cast<float>(p.Hkv) * static_cast<float>(p.n);
  p.red[0] = gA / live / cnt;
  p.red[1] = gD / live / cnt;
  p.red[2] = gW / live / cnt;
  p.red[3] = live;
}

__global__ __launch_bounds__(kCThreads) void cov_final(CovParams p) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kCThreads + threadIdx.x;
  const float live = p.red[3];
  const int64_t nA = static_cast<int64_t>(p.Hkv) * p.n;
  const int64_t nS = static_cast<int64_t>(p.Hkv) * kCD * kCD;
  if (t < nA) {
    const int h = static_cast<int>(t / p.n), j = static_cast<int>(t % p.n);
    float w = 0.0f;
    for (int r = 0; r < p.rep; ++r) w += p.WVa[(static_cast<int64_t>(h) * p.rep + r) * p.n + j];
    p.A[t] = p.A[t] / live + p.eta * p.red[0];
    p.DD[t] = p.DD[t] / live + p.eta * p.red[1];
    p.W[t] = w / live + p.eta * p.red[2];
  }
  if (t < nS) {
    const int h = static_cast<int>(t / (kCD * kCD)), e = static_cast<int>(t % (kCD * kCD));
    const float sA = p.red[4 + p.Hkv * p.rep + h];
    p.S[t] = p.S[t] / live / fmaxf(sA, 1e-30f);
    float om = 0.0f, acc = 0.0f, mean = 0.0f;
    for (int r = 0; r < p.rep; ++r) {
      const float o = p.red[4 + h * p.rep + r];
      const float mv = p.M[static_cast<int64_t>(h * p.rep + r) * kCD * kCD + e];
      om += o;
      acc = __builtin_fmaf(o, mv, acc);
      mean += mv;
    }
    p.Mbar[t] = om > 0.0f ? acc / om : mean / static_cast<float>(p.rep);
  }
}

}  // namespace
}  // namespace kvq

using namespace kvq;

// workspace layout (floats): row_m, row_il, oMo, roww (Hkv NR each); o (Hkv NR d); o_part (kOSplit Hkv
// NR d); vmv (Hkv rep n); ddpart (G Hkv n_chunks 4); alpha_part (Hkv n_chunks NR); gw (2 G + 1); red (4 +
// Hkv rep + Hkv); WVa (Hkv rep n); A_part, DD_part (kTSplit Hkv n each); WVa_part (kTSplit Hkv rep n);
// mop (Hkv NR 128), rowf (Hkv NR 4), 16-byte aligned; S_part (kSSplit Hkv d d); sums (Hkv (2 + rep));
// fp32 rows: partial maxima and scales (kAmaxFloats)
extern "C" int64_t kvq_coverage_stats_workspace(int64_t Hkv, int64_t rep, int64_t n, int64_t NR, int64_t G) {
  if (Hkv <= 0 || rep <= 0 || n <= 0 || NR <= 0 || G <= 0) return -1;
  const int64_t nch = (n + kChunkTok - 1) / kChunkTok;
  return 4 * Hkv * NR + (1 + kOSplit) * Hkv * NR * kCD + Hkv * rep * n + G * Hkv * nch * kCWaves + Hkv * nch * NR + (2 * G + 1) +
         (4 + Hkv * rep + Hkv) + Hkv * rep * n + kTSplit * (2 * Hkv * n + Hkv * rep * n) + 132 * Hkv * NR + 4 + kSSplit * Hkv * kCD * kCD + Hkv * (2 + rep) +
         kAmaxFloats;
}

extern "C" int kvq_coverage_stats(const void* qr, int dtype, int64_t NR, const int32_t* rowpos, const int32_t* rowgrp,
                                  const int32_t* rlist, int64_t n_rlist, const int32_t* gtab, int64_t G,
                                  const int32_t* items, int64_t n_items, const void* k, int64_t k_sh, int64_t k_st,
                                  const void* v, int64_t v_sh, int64_t v_st, int64_t T, const float* M, int64_t Hkv,
                                  int64_t rep, int64_t d, int64_t rs, int64_t re, float scaling, float eta, float* A,
                                  float* W, float* DD, float* S, float* Mbar, float* workspace,
                                  int64_t workspace_floats, void* stream) {
  KVQ_REQUIRE(valid_dtype(dtype), "kvq_coverage_stats: bad dtype");
  KVQ_REQUIRE(d == kCD, "kvq_coverage_stats: head_dim must be 128");
  KVQ_REQUIRE(Hkv > 0 && rep > 0 && Hkv * rep <= 1024, "kvq_coverage_stats: bad head counts");
  KVQ_REQUIRE(0 <= rs && rs < re && re <= T && T < (1 << 28), "kvq_coverage_stats: need 0 <= rs < re <= T");
  KVQ_REQUIRE(G > 0 && n_items > 0 && NR > 0 && NR % 16 == 0 && Hkv * NR < (1LL << 31) / kCD && n_rlist > 0 &&
                  n_rlist * rep <= NR,
              "kvq_coverage_stats: bad group plan");
  KVQ_REQUIRE(qr && rowpos && rowgrp && rlist && gtab && items && k && v && M && A && W && DD && S && Mbar && workspace,
              "kvq_coverage_stats: null pointer");
  const int esz = dtype == KVQ_F32 ? 4 : 2;
  KVQ_REQUIRE((k_sh * esz) % 16 == 0 && (k_st * esz) % 16 == 0 && (v_sh * esz) % 16 == 0 && (v_st * esz) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(k) % 16 == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(qr) % 16 == 0 && reinterpret_cast<uintptr_t>(workspace) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(M) % 16 == 0 && k_st >= kCD && v_st >= kCD,
              "kvq_coverage_stats: rows must be 16-byte aligned and not overlap");
  KVQ_REQUIRE((T + 48) * std::max(k_st, v_st) * esz < (1LL << 31), "kvq_coverage_stats: one head's rows must span < 2 GiB");
  const int64_t n = re - rs;
  const int64_t need = kvq_coverage_stats_workspace(Hkv, rep, n, NR, G);
  KVQ_REQUIRE(workspace_floats >= need, "kvq_coverage_stats: workspace too small (%lld < %lld floats)",
              (long long)workspace_floats, (long long)need);
  CovParams p{};
  p.qr = qr; p.rowpos = rowpos; p.gtab = gtab; p.items = items;
  p.k = k; p.v = v; p.k_sh = k_sh; p.k_st = k_st; p.v_sh = v_sh; p.v_st = v_st;
  p.M = M;
  p.Hkv = (int)Hkv; p.rep = (int)rep; p.NR = (int)NR; p.G = (int)G; p.n_items = (int)n_items;
  p.rs = (int)rs; p.re = (int)re; p.n = (int)n; p.n_chunks = (int)((n + kChunkTok - 1) / kChunkTok); p.T = (int)T;
  p.scaling = scaling; p.qscale = scaling * kCLog2e; p.eta = eta;
  float* w = workspace;
  p.row_m = w; w += Hkv * NR;
  p.row_il = w; w += Hkv * NR;
  p.oMo = w; w += Hkv * NR;
  p.roww = w; w += Hkv * NR;
  p.o = w; w += Hkv * NR * kCD;
  p.o_part = w; w += kOSplit * Hkv * NR * kCD;
  p.vmv = w; w += Hkv * rep * n;
  p.ddpart = w; w += G * Hkv * p.n_chunks * kCWaves;
  p.alpha_part = w; w += Hkv * p.n_chunks * NR;
  p.gw = w; w += 2 * G + 1;
  p.red = w; w += 4 + Hkv * rep + Hkv;
  p.WVa = w; w += Hkv * rep * n;
  p.A_part = w; w += kTSplit * Hkv * n;
  p.DD_part = w; w += kTSplit * Hkv * n;
  p.WVa_part = w; w += kTSplit * Hkv * rep * n;
  w += (4 - (reinterpret_cast<uintptr_t>(w) / 4) % 4) % 4;       // 16-byte alignment of the next two
  p.mop = reinterpret_cast<uint32_t*>(w); w += 128 * Hkv * NR;
  p.rowf = w; w += 4 * Hkv * NR;
  p.S_part = w; w += kSSplit * Hkv * kCD * kCD;
  p.sums = w; w += Hkv * (2 + rep);
  float* amax_part = w;                                       // fp32 rows: partial maxima, then scales
  p.xs = dtype == KVQ_F32 ? w + kAmaxViews * kAmaxBlocks : nullptr;
  p.A = A; p.W = W; p.DD = DD; p.S = S; p.Mbar = Mbar;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 blk(kCThreads);
  if (dtype == KVQ_F32) {
    // the powers of two that bring the query rows, keys and values into the fp16 parts' range
    const RowView views[3] = {
        RowView{static_cast<const float*>(qr), static_cast<int>(Hkv), static_cast<int>(NR), 1, NR * kCD, kCD, 0},
        RowView{static_cast<const float*>(k), static_cast<int>(Hkv), static_cast<int>(T), 1, k_sh, k_st, 0},
        RowView{static_cast<const float*>(v), static_cast<int>(Hkv), static_cast<int>(T), 1, v_sh, v_st, 0}};
    launch_rows_scales(views, 3, amax_part, const_cast<float*>(p.xs), s);
    KVQ_LAUNCH_CHECK("kvq_coverage_stats(fp32 scales)");
  }
  KVQ_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((cov_rowstats<DT_>), dim3(xcd_grid(n_items * Hkv)),
                                               dim3(DT_ == KVQ_F32 ? kCThreads : 2 * kCThreads), 0, s, p));
  KVQ_LAUNCH_CHECK("kvq_coverage_stats(rowstats)");
  KVQ_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((cov_output<DT_>), dim3(xcd_grid(n_items * Hkv * kOSplit)), blk, 0, s, p));
  KVQ_LAUNCH_CHECK("kvq_coverage_stats(output)");
  hipLaunchKernelGGL((cov_metric<KVQ_F32, true>), dim3(Hkv * rep * ((n_rlist + kMetricRows - 1) / kMetricRows)), blk,
                     0, s, p, rlist, (int)n_rlist);
  KVQ_LAUNCH_CHECK("kvq_coverage_stats(o M)");
  KVQ_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((cov_vmv<DT_>),
                                               dim3(Hkv * rep * ((n + kVmvPer - 1) / kVmvPer)), blk, 0, s, p));
  KVQ_LAUNCH_CHECK("kvq_coverage_stats(v M v)");
  const unsigned terms_blocks = xcd_grid(Hkv * p.n_chunks * kTSplit);
  KVQ_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((cov_rowprep<DT_>), dim3((Hkv * NR + 15) / 16), blk, 0, s, p));
  KVQ_LAUNCH_CHECK("kvq_coverage_stats(row operands)");
  // 16-bit rows and up to kTermsLdsRep query heads per KV head: the chunk's rows staged in LDS, two
  // quads of wavefronts
  const bool terms_lds = dtype != KVQ_F32 && rep <= kTermsLdsRep;
  const dim3 blk2(2 * kCThreads);
  if (terms_lds) {
    if (dtype == KVQ_BF16) hipLaunchKernelGGL((cov_terms<KVQ_BF16, false, true>), dim3(terms_blocks), blk2, 0, s, p);
    else hipLaunchKernelGGL((cov_terms<KVQ_F16, false, true>), dim3(terms_blocks), blk2, 0, s, p);
  } else {
    KVQ_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((cov_terms<DT_, false, false>), dim3(terms_blocks), blk, 0, s, p));
  }
  KVQ_LAUNCH_CHECK("kvq_coverage_stats(terms)");
  hipLaunchKernelGGL(cov_groups, dim3(static_cast<unsigned>(G)), blk, 0, s, p);
  KVQ_LAUNCH_CHECK("kvq_coverage_stats(groups)");
  hipLaunchKernelGGL(cov_roww, dim3((Hkv * NR + kCThreads - 1) / kCThreads), blk, 0, s, p, rowgrp);
  KVQ_LAUNCH_CHECK("kvq_coverage_stats(row weights)");
  // the read masses are accumulated by the weighted pass: cleared by a fill kernel (graph-capture safe)
  const int64_t nwp = kTSplit * Hkv * rep * n;
  hipLaunchKernelGGL(cov_clear, dim3((nwp + kCThreads - 1) / kCThreads), blk, 0, s, p.WVa_part, nwp);
  KVQ_LAUNCH_CHECK("kvq_coverage_stats(clear)");
  if (terms_lds) {
    if (dtype == KVQ_BF16) hipLaunchKernelGGL((cov_terms<KVQ_BF16, true, true>), dim3(terms_blocks), blk2, 0, s, p);
    else hipLaunchKernelGGL((cov_terms<KVQ_F16, true, true>), dim3(terms_blocks), blk2, 0, s, p);
  } else {
    KVQ_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((cov_terms<DT_, true, false>), dim3(terms_blocks), blk, 0, s, p));
  }
  KVQ_LAUNCH_CHECK("kvq_coverage_stats(weighted terms)");
  hipLaunchKernelGGL(cov_split_sums, dim3((Hkv * rep * n + kCThreads - 1) / kCThreads), blk, 0, s, p);
  KVQ_LAUNCH_CHECK("kvq_coverage_stats(split sums)");
  KVQ_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((cov_smat<DT_>), dim3(Hkv * (kCD / 16) * kSSplit), blk, 0, s, p));
  KVQ_LAUNCH_CHECK("kvq_coverage_stats(S parts)");
  hipLaunchKernelGGL(cov_smat_sum, dim3((Hkv * kCD * kCD + kCThreads - 1) / kCThreads), blk, 0, s, p);
  KVQ_LAUNCH_CHECK("kvq_coverage_stats(S)");
  hipLaunchKernelGGL(cov_final_sums, dim3(static_cast<unsigned>(Hkv * (2 + rep))), dim3(1024), 0, s, p);
  KVQ_LAUNCH_CHECK("kvq_coverage_stats(sums)");
  hipLaunchKernelGGL(cov_final_combine, dim3(1), dim3(64), 0, s, p);
  KVQ_LAUNCH_CHECK("kvq_coverage_stats(combine)");
  const int64_t nmax = std::max<int64_t>(Hkv * n, Hkv * kCD * kCD);
  hipLaunchKernelGGL(cov_final, dim3((nmax + kCThreads - 1) / kCThreads), blk, 0, s, p);
  KVQ_LAUNCH_CHECK("kvq_coverage_stats(final)");
  return KVQ_OK;
}
