// Blockwise token-axis DCT coding of K/V (A9) and the decode over it.
//
// The reference has no DCT; this contract follows the reference's own conventions: per (KV head,
// channel, 64-token block) an orthonormal DCT-II along tokens, coefficients 0..15 kept, each
// (block, channel) quantised with symmetric absmax at 4 bits (absmax_quant, STRATA_KV.py:549-554:
// s = max(fp16(max|X| / 7), 2^-24), codes clamp(round(X / s), -7, 7)), stored offset-binary (+7) as
// TILT_KV.py:2621-2625 does.
//
// Encoder arithmetic order (restated by the CPU oracle, so codes and scales agree bit for bit):
// X_k = sum over n = 0..63 in increasing n of float32(C[k][n] * x_n), no fused multiply-add, C the
// float32 table of the kept rows (passed in); s and codes in float32 with IEEE division.
//
// Stored per (b, h, block):
//   key codes   16 rows (coefficients) x 16 words: word D of row k holds the codes of channels
//               8D .. 8D+7 of coefficient k, channel 8D + e at nibble kNib[e] = {0,4,1,5,2,6,3,7}[e]
//               (the value tiles' nibble order: masking a word in place yields the 8 codes as fp16
//               subnormals in channel order)
//   key scales  128 fp16 (by channel)
//   value codes 1 KiB decode tile: word (gp * 16 + n) * 8 + blk (gp = coefficient half 0/1, n = 0..15,
//               blk = 0..7) holds the codes of coefficients 8gp .. 8gp+7 of channel 16*blk + n, code
//               of coefficient 8gp + e at nibble kNib[e] = {0,4,1,5,2,6,3,7}[e]
//   value scales 128 fp16 ordered [n][blk] (channel 16*blk + n)
//
// Decode (coefficient domain, four matrix-core stages per block and wavefront):
//   u_k   = sum_c q_c s^K_c (code_kc - 7)             (q x key codes, the KIVI key-group machinery)
//   s_n   = sum_k C[k][n] u_k                         (logits of the block's 64 tokens)
//   w_k   = sum_n C[k][n] p_n                         (after the online softmax)
//   out_c += s^V_c (sum_k w_k code_kc - 7 sum_k w_k)  (w transposed through LDS against value codes)
#include "common.hpp"
#include "mfma_common.hpp"
#include "partials.hpp"

namespace kvq {
namespace {

constexpr int kDB = 64;                   // tokens per block
constexpr int kDK = 16;                   // kept coefficients
constexpr int kDD = 128;                  // head_dim
constexpr int kDThreads = 256;
constexpr int kDWaves = 4;

__device__ __forceinline__ float as_stored_h(float x) {
  x = fminf(fmaxf(x, -65504.0f), 65504.0f);
  return f16_to_f32(f32_to_f16(x));
}

__device__ __constant__ int kNibOfElem[8] = {0, 4, 1, 5, 2, 6, 3, 7};

// one thread per (b, h, block, channel)
template <int DT>
__global__ __launch_bounds__(256) void dct_encode_kernel(const void* __restrict__ x, int64_t T, int64_t x_bh,
                                                         const float* __restrict__ ctab, int for_values,
                                                         uint8_t* __restrict__ codes, uint16_t* __restrict__ scales,
                                                         int64_t total) {
  const int64_t id = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (id >= total) return;
  const int c = static_cast<int>(id % kDD);
  const int64_t blk_all = id / kDD;                // (bh, block)
  const int64_t nb = T / kDB;
  const int64_t bh = blk_all / nb, blk = blk_all % nb;
  const int64_t base = bh * x_bh + blk * kDB * kDD + c;
  float X[kDK];
#pragma unroll
  for (int k = 0; k < kDK; ++k) X[k] = 0.0f;
  for (int n = 0; n < kDB; ++n) {
    const float xv = load_as_f32<DT>(x, base + static_cast<int64_t>(n) * kDD);
#pragma unroll
    for (int k = 0; k < kDK; ++k) X[k] = __fadd_rn(X[k], __fmul_rn(ctab[k * kDB + n], xv));
  }
  float amax = 0.0f;
#pragma unroll
  for (int k = 0; k < kDK; ++k) amax = fmaxf(amax, fabsf(X[k]));
  const float s = fmaxf(as_stored_h(__fdiv_rn(amax, 7.0f)), 5.9604644775390625e-08f);
  int q[kDK];
#pragma unroll
  for (int k = 0; k < kDK; ++k) q[k] = static_cast<int>(fminf(fmaxf(rintf(__fdiv_rn(X[k], s)), -7.0f), 7.0f)) + 7;
  uint8_t* out = codes + blk_all * 1024;
  if (!for_values) {
    scales[blk_all * kDD + c] = f32_to_f16(s);
    // the 8 channels of a word are 8 consecutive lanes (total is a multiple of 128, so every
    // wavefront that reaches here is whole): OR their nibbles together across the lanes
    uint32_t* words = reinterpret_cast<uint32_t*>(out);
#pragma unroll
    for (int k = 0; k < kDK; ++k) {
      uint32_t w = static_cast<uint32_t>(q[k]) << (4 * kNibOfElem[c & 7]);
      w |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(w), 1, 64));
      w |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(w), 2, 64));
      w |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(w), 4, 64));
      if ((c & 7) == 0) words[k * 16 + c / 8] = w;
    }
  } else {
    const int n = c % 16, b8 = c / 16;
    scales[blk_all * kDD + n * 8 + b8] = f32_to_f16(s);
    uint32_t* words = reinterpret_cast<uint32_t*>(out);
#pragma unroll
    for (int gp = 0; gp < 2; ++gp) {
      uint32_t w = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) w |= static_cast<uint32_t>(q[8 * gp + e]) << (4 * kNibOfElem[e]);
      words[(gp * 16 + n) * 8 + b8] = w;
    }
  }
}


struct DctParams {
  const void* q;
  int64_t q_sb, q_sh, q_st;
  int Hq, Hkv, Tq, rep, R_real, BH;
  float qscale;
  int64_t nb;                     // blocks per (b, h)
  const uint8_t* kc;              // (BH, nb, 16, 64)
  const uint16_t* ks;             // (BH, nb, 128)
  const uint8_t* vc;              // (BH, nb, 1024)
  const uint16_t* vs;             // (BH, nb, 128) [n][blk]
  const float* ctab;              // (16, 64) float32
  int n_split;
  float* ws_o;
  float* ws_m;
  float* ws_l;
  int S_all;
  const float* ex_o;
  const float* ex_m;
  const float* ex_l;
  int S_ex;
  void* out;
};

__device__ __forceinline__ int64_t dct_q_offset(const DctParams& p, int b, int h, int r) {
  const int hq = h * p.rep + r / p.Tq, t = r % p.Tq;
  return static_cast<int64_t>(b) * p.q_sb + static_cast<int64_t>(hq) * p.q_sh + static_cast<int64_t>(t) * p.q_st;
}

template <int R, int DT>
__device__ void dct_block(const DctParams& p, int bh, int sidx, float* smem) {
  const int b = bh / p.Hkv, h = bh % p.Hkv;
  float (*qs)[kDD] = reinterpret_cast<float (*)[kDD]>(smem);                    // q * qscale
  uint32_t* bq_all = reinterpret_cast<uint32_t*>(smem + R * kDD);               // [wave][2R][64]
  uint32_t* bv_all = bq_all + kDWaves * 2 * R * kBqStride;                            // [wave][R][16]
  float* wsm_all = reinterpret_cast<float*>(bv_all + kDWaves * R * 16);         // [wave][R][17] + [R] + [R]
  u32x4* cst = reinterpret_cast<u32x4*>(wsm_all + kDWaves * R * 19);            // [12][64] lane constants
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const int l = threadIdx.x % 64;
  const int g = l >> 4, n = l & 15;
  const int r_n = n % R;
  const int hl = (n / R) & 1;
  const int ci = (l >> 2) & 3, ck = l & 3;
  const int c0 = 32 * g + 8 * ci + 2 * ck;          // key words unpack in channel order
  const int c1 = c0 + 1;
  const float kinv = (ck & 1) ? 1.0f : 16.0f;
  uint32_t* bq = bq_all + wave * 2 * R * kBqStride;
  uint32_t* bv = bv_all + wave * R * 16;
  float* wsm = wsm_all + wave * R * 19;            // [R][17] w values (stride 17: bank-spread), [R] sum w, [R] alpha

  for (int idx = threadIdx.x; idx < R * kDD; idx += kDThreads) {
    const int r = idx / kDD, c = idx % kDD;
    qs[r][c] = r < p.R_real ? load_as_f32<DT>(p.q, dct_q_offset(p, b, h, r) + c) * p.qscale : 0.0f;
  }
  // the DCT table, staged once: (16, 64) float32 = 256 float4, one per thread
  float* ct = reinterpret_cast<float*>(cst + 12 * 64);
  reinterpret_cast<float4*>(ct)[threadIdx.x] = reinterpret_cast<const float4*>(p.ctab)[threadIdx.x];
  __syncthreads();
  // lane constants (the same for every wavefront; each wavefront builds three of the twelve):
  // C^T tiles of the logit stage, hi / lo, 4 nonzero slots each (waves 0, 1: tiles 2w, 2w+1);
  // C slices of the coefficient stage, hi / lo per k-step (waves 2, 3: k-step w - 2)
  if (wave < 2) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int t = 2 * wave + tt;
      uint32_t hi[2], lo[2];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const float a = ct[(4 * g + 2 * kk) * kDB + 16 * t + n];
        const float bb = ct[(4 * g + 2 * kk + 1) * kDB + 16 * t + n];
        const _Float16 ah = static_cast<_Float16>(a), bh16 = static_cast<_Float16>(bb);
        hi[kk] = pack_h2(ah, bh16);
        lo[kk] = pack_h2(static_cast<_Float16>(a - static_cast<float>(ah)), static_cast<_Float16>(bb - static_cast<float>(bh16)));
      }
      cst[(2 * t) * 64 + l] = u32x4{hi[0], hi[1], 0u, 0u};
      cst[(2 * t + 1) * 64 + l] = u32x4{lo[0], lo[1], 0u, 0u};
    }
  } else {
    const int ks = wave - 2;
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      float v[2];
      _Float16 vh[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int j = 2 * jj + u;
        const int tok = 32 * ks + 16 * (j >> 2) + 4 * g + (j & 3);
        v[u] = ct[n * kDB + tok];                       // row n = coefficient (M index m = n)
        vh[u] = static_cast<_Float16>(v[u]);
      }
      hi[jj] = pack_h2(vh[0], vh[1]);
      lo[jj] = pack_h2(static_cast<_Float16>(v[0] - static_cast<float>(vh[0])),
                       static_cast<_Float16>(v[1] - static_cast<float>(vh[1])));
    }
    cst[(8 + 2 * ks) * 64 + l] = u32x4{hi[0], hi[1], hi[2], hi[3]};
    cst[(8 + 2 * ks + 1) * 64 + l] = u32x4{lo[0], lo[1], lo[2], lo[3]};
  }
  __syncthreads();

  const int NW = p.n_split * kDWaves;
  const int w_all = sidx * kDWaves + wave;
  const int b0 = static_cast<int>(static_cast<int64_t>(w_all) * p.nb / NW);
  const int b1 = static_cast<int>(static_cast<int64_t>(w_all + 1) * p.nb / NW);

  const __amdgpu_buffer_rsrc_t rk = make_rsrc(p.kc + static_cast<int64_t>(bh) * p.nb * 1024,
                                              static_cast<uint32_t>(p.nb * 1024));
  const __amdgpu_buffer_rsrc_t rks = make_rsrc(p.ks + static_cast<int64_t>(bh) * p.nb * kDD,
                                               static_cast<uint32_t>(p.nb * kDD * 2));
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.vc + static_cast<int64_t>(bh) * p.nb * 1024,
                                              static_cast<uint32_t>(p.nb * 1024));
  const __amdgpu_buffer_rsrc_t rvs = make_rsrc(p.vs + static_cast<int64_t>(bh) * p.nb * kDD,
                                               static_cast<uint32_t>(p.nb * kDD * 2));
  // value-code lanes: coefficient half g < 2 reads its 8 words; g >= 2 reads past the range (zero)
  const int vo_v = g < 2 ? (g * 16 + n) * 32 : 0x40000000;

  struct Blk {
    u32x4 kw;
    uint32_t ks0, ks1;
    u32x4 vw[2];
    u32x4 vsw;
  };
  auto load_blk = [&](int bi, Blk& c) {
    bi = min(bi, b1 - 1);
    const int so = __builtin_amdgcn_readfirstlane(bi * 1024);
    c.kw = __builtin_amdgcn_raw_buffer_load_b128(rk, n * 64 + 16 * g, so, 2);
    const int sk = __builtin_amdgcn_readfirstlane(bi * kDD * 2);
    c.ks0 = __builtin_amdgcn_raw_buffer_load_b16(rks, c0 * 2, sk, 0);
    c.ks1 = __builtin_amdgcn_raw_buffer_load_b16(rks, c1 * 2, sk, 0);
    c.vw[0] = __builtin_amdgcn_raw_buffer_load_b128(rv, vo_v, so, 2);
    c.vw[1] = __builtin_amdgcn_raw_buffer_load_b128(rv, vo_v + 16, so, 2);
    c.vsw = __builtin_amdgcn_raw_buffer_load_b128(rvs, n * 16, sk, 2);
  };

  auto unpack = [](uint32_t w) -> half8 {
    const uint32_t w8 = w >> 8;
    return as_half8(u32x4{w & 0x000F000Fu, w & 0x00F000F0u, w8 & 0x000F000Fu, w8 & 0x00F000F0u});
  };
  constexpr float kTwo20 = 1048576.0f;
  constexpr float kTwo24 = 16777216.0f;
  constexpr float kLazy = 4.0f;
  constexpr float kPOff = 6.0f;   // probabilities carry 2^6 so their fp16 parts stay normal; m is stored minus it
  const half8 tiny = as_half8(u32x4{0x00100010u, 0x00100010u, 0x00100010u, 0x00100010u});   // 2^-20
  const half2v hl_neg = hl ? half2v{static_cast<_Float16>(-1.0f), static_cast<_Float16>(-1.0f)}
                           : half2v{static_cast<_Float16>(0.0f), static_cast<_Float16>(0.0f)};
  const u32x4* bq_src = reinterpret_cast<const u32x4*>(bq + (2 * r_n + hl) * kBqStride + g * 16);
  const u32x4* bv_src = reinterpret_cast<const u32x4*>(bv + r_n * 16 + g * 4);

  float acc[8][2];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k][0] = acc[k][1] = 0.0f;
  float m_run = -INFINITY, la = 0.0f;
  // split of an fp32 value into the fp16 hi (variant 0) or lo (variant 1) part this lane feeds
  auto part = [&](float x) -> _Float16 {
    const _Float16 hi16 = static_cast<_Float16>(x);
    return hl ? static_cast<_Float16>(x - static_cast<float>(hi16)) : hi16;
  };

  auto step = [&](const Blk& c) {
    // ---- key group of this block: B operand q * sK (hi / lo), bias -7 q . sK ----
    wave_lds_fence();
    {
      const float sc0 = h2f(c.ks0, 0), sc1 = h2f(c.ks1, 0);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float qa = qs[r][c0], qb = qs[r][c1];
        const float qak = qa * kinv, qbk = qb * kinv;
        const _Float16 h0 = static_cast<_Float16>(qak * sc0);
        const _Float16 h1 = static_cast<_Float16>(qbk * sc1);
        const _Float16 e0 = static_cast<_Float16>(qak * sc0 - static_cast<float>(h0));
        const _Float16 e1 = static_cast<_Float16>(qbk * sc1 - static_cast<float>(h1));
        bq[(2 * r) * kBqStride + l] = pack_h2(h0, h1);
        bq[(2 * r + 1) * kBqStride + l] = pack_h2(e0, e1);
        float P = -7.0f * (qa * sc0 + qb * sc1);
        P += dpp<kQuadSwap1>(P);
        P += dpp<kQuadSwap2>(P);
        if (ck == 0) {
          const _Float16 ph = static_cast<_Float16>(P);
          const _Float16 pl = static_cast<_Float16>(P - static_cast<float>(ph));
          bv[r * 16 + g * 4 + ci] = pack_h2(ph, pl);
        }
      }
    }
    wave_lds_fence();
    half8 bqk[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) bqk[i] = as_half8(bq_src[i]);
    u32x4 bvr = *bv_src;
    if (hl) bvr = u32x4{0u, 0u, 0u, 0u};
    // ---- u_k (coefficient k = 4g + i), log2 units ----
    f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) d = mfma(unpack(c.kw[i]), bqk[i], d);
    d = mfma(tiny, as_half8(bvr), d);
    float u[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) u[i] = (d[i] + dpp<kRowRor + R>(d[i])) * kTwo20;
    // ---- logits of the 64 tokens: s = C^T u (token 16t + 4g + i in register 4t + i) ----
    const half8 b2 = as_half8(u32x4{pack_h2(part(u[0]), part(u[1])), pack_h2(part(u[2]), part(u[3])), 0u, 0u});
    float s[16];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      f32x4 e = mfma(as_half8(cst[(2 * t) * 64 + l]), b2, f32x4{0.f, 0.f, 0.f, 0.f});
      e = mfma(as_half8(cst[(2 * t + 1) * 64 + l]), b2, e);
#pragma unroll
      for (int i = 0; i < 4; ++i) s[4 * t + i] = e[i] + dpp<kRowRor + R>(e[i]);
    }
    // ---- online softmax, lazy maximum ----
    float lm = s[0];
#pragma unroll
    for (int j = 1; j < 16; ++j) lm = fmaxf(lm, s[j]);
    if (__any(lm > m_run + kLazy)) {
      const float m_new = fmaxf(m_run, xmax32(xmax16(lm)));
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      la *= alpha;
      m_run = m_new;
      if (g == 0 && n < R) wsm[R * 18 + n] = alpha;           // alpha of row n for the value lanes
      wave_lds_fence();
#pragma unroll
      for (int jr = 0; jr < 2; ++jr) {
        const int r = 2 * g + jr;
        const float a = r < R ? wsm[R * 18 + r] : 1.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k][jr] *= a;
      }
    }
    float pr[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      pr[j] = __builtin_amdgcn_exp2f(s[j] - m_run + kPOff);
      la += pr[j];
    }
    // ---- w_k = sum_n C[k][n] p_n (coefficient 4g + i) ----
    f32x4 dw = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      uint32_t words[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int j0 = 2 * jj, j1 = 2 * jj + 1;
        const float x0 = pr[4 * (2 * ks + (j0 >> 2)) + (j0 & 3)];
        const float x1 = pr[4 * (2 * ks + (j1 >> 2)) + (j1 & 3)];
        const half2v hi2 = half2v{static_cast<_Float16>(x0), static_cast<_Float16>(x1)};
        const half2v cn = hi2 * hl_neg;
        words[jj] = w2(half2v{static_cast<_Float16>(x0 + static_cast<float>(cn[0])),
                              static_cast<_Float16>(x1 + static_cast<float>(cn[1]))});
      }
      const half8 b4 = as_half8(u32x4{words[0], words[1], words[2], words[3]});
      dw = mfma(as_half8(cst[(8 + 2 * ks) * 64 + l]), b4, dw);
      dw = mfma(as_half8(cst[(8 + 2 * ks + 1) * 64 + l]), b4, dw);
    }
    // ---- w to LDS (rows of the value stage), and sum_k w per row ----
    float wsum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float w = dw[i] + dpp<kRowRor + R>(dw[i]);
      wsum += w;
      if (n < R) wsm[n * 17 + 4 * g + i] = w;
    }
    wsum = xsum32(xsum16(wsum));
    if (g == 0 && n < R) wsm[R * 17 + n] = wsum;
    wave_lds_fence();
    // A operand: row m = 2r + hl5 of w (hi / lo), coefficients 8g .. 8g+7 (g < 2), element e / 16
    // for the high-nibble elements 2, 3, 6, 7
    const int m_r = n >> 1, m_hl = n & 1;
    uint32_t aw[4] = {0u, 0u, 0u, 0u};
    if (g < 2 && m_r < R) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        float x[2];
#pragma unroll
        for (int u2 = 0; u2 < 2; ++u2) {
          const int e = 2 * jj + u2;
          x[u2] = wsm[m_r * 17 + 8 * g + e] * (((e >> 1) & 1) ? 0.0625f : 1.0f);
        }
        _Float16 hh[2];
#pragma unroll
        for (int u2 = 0; u2 < 2; ++u2) {
          const _Float16 hi16 = static_cast<_Float16>(x[u2]);
          hh[u2] = m_hl ? static_cast<_Float16>(x[u2] - static_cast<float>(hi16)) : hi16;
        }
        aw[jj] = pack_h2(hh[0], hh[1]);
      }
    }
    const half8 a5 = as_half8(u32x4{aw[0], aw[1], aw[2], aw[3]});
    const float W0 = 2 * g < R ? wsm[R * 17 + 2 * g] : 0.0f;
    const float W1 = 2 * g + 1 < R ? wsm[R * 17 + 2 * g + 1] : 0.0f;
    // ---- out rows 2g, 2g+1, channel 16*blk + n ----
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
      const f32x4 d5 = mfma(a5, unpack(c.vw[blk >> 2][blk & 3]), f32x4{0.f, 0.f, 0.f, 0.f});
      const float sv = h2f(c.vsw[blk >> 1], blk & 1);
      acc[blk][0] = __builtin_fmaf(sv, __builtin_fmaf(d5[0] + d5[1], kTwo24, -7.0f * W0), acc[blk][0]);
      acc[blk][1] = __builtin_fmaf(sv, __builtin_fmaf(d5[2] + d5[3], kTwo24, -7.0f * W1), acc[blk][1]);
    }
  };

  if (b0 < b1) {
    Blk ca, cb_;
    load_blk(b0, ca);
    for (int bi = b0;; bi += 2) {
      load_blk(bi + 1, cb_);
      step(ca);
      if (bi + 1 >= b1) break;
      load_blk(bi + 2, ca);
      step(cb_);
      if (bi + 2 >= b1) break;
    }
  }

  // ---- epilogue: 4-wave merge of (m, l, o) into this split's partial ----
  const float l_run = xsum32(xsum16(la));
  __syncthreads();
  float* red_o = smem;                            // [wave][R][d]
  float* red_ml = smem + kDWaves * R * kDD;       // [wave][2][R]
#pragma unroll
  for (int blk = 0; blk < 8; ++blk) {
#pragma unroll
    for (int jr = 0; jr < 2; ++jr) {
      const int r = 2 * g + jr;
      if (r < R) red_o[(wave * R + r) * kDD + 16 * blk + n] = acc[blk][jr];
    }
  }
  if (g == 0 && n < R) {
    red_ml[(wave * 2 + 0) * R + n] = m_run - kPOff;
    red_ml[(wave * 2 + 1) * R + n] = l_run;
  }
  __syncthreads();
  const int64_t po = static_cast<int64_t>(bh) * p.S_all + sidx;
  for (int idx = threadIdx.x; idx < p.R_real * kDD; idx += kDThreads) {
    const int r = idx / kDD, c = idx % kDD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDWaves; ++w) M = fmaxf(M, red_ml[(w * 2) * R + r]);
    float O = 0.0f, L = 0.0f;
#pragma unroll
    for (int w = 0; w < kDWaves; ++w) {
      const float mw_ = red_ml[(w * 2) * R + r];
      const float wgt = (mw_ == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw_ - M);
      O += wgt * red_o[(w * R + r) * kDD + c];
      L += wgt * red_ml[(w * 2 + 1) * R + r];
    }
    p.ws_o[(po * R + r) * kDD + c] = O;
    if (c == 0) {
      p.ws_m[po * R + r] = M;
      p.ws_l[po * R + r] = L;
    }
  }
}

template <int R, int DT>
__global__ __launch_bounds__(kDThreads) __attribute__((amdgpu_waves_per_eu(2)))
void dct_split(DctParams p) {
  extern __shared__ float smem[];
  const int k = blockIdx.x / 8;
  const int bh = blockIdx.x % 8 + 8 * (k / p.n_split);
  if (bh < p.BH) dct_block<R, DT>(p, bh, k % p.n_split, smem);
}

// ---------------------------------------------------------------------------------------------
// dct_pair_split<DT>: 16-bit queries and outputs with R = 8 rows (rep * Tq in 5..8; C5's GQA 8).
//
// Each wavefront takes its blocks two at a time (slots A and B).  The 16 columns of every matrix
// product are (slot, row) = (n / 8, n % 8): the logit and coefficient stages, whose constant operand
// (the DCT table) is the same for every block, cover both blocks in one product, and the softmax
// works on 16 useful values per lane.  One fp16 rounding each for q s^K, u, p and w (the bar of
// 16-bit outputs); the -7 offset of the stored codes enters through products with a constant
// operand K7 (-7 2^-24 at low-nibble positions, -112 2^-24 at high-nibble ones).
//
//   key stage    D_c = sum_i K7 x qt_i; D_A = D_c + sum_i codes_A,i x qt_i; D_B likewise.  qt_i is
//                the lane's column's (q x s^K) over channels 32g + 8i + 0..7 with the scales of the
//                column's own block, so D_A is right in slot A's columns and D_B in slot B's:
//                u = n < 8 ? D_A : D_B (coefficient 4g + i), in units of 2^-20
//   logit stage  s = C^T u                       (v_mfma_f32_16x16x16_f16, 4 tiles of 16 tokens)
//   softmax      online, per column, lazy maximum; p carries 2^kPOff
//   coef stage   w' = f C p                      (2 products over 64 tokens; f = 1/16 on the
//                                                 coefficients whose value code is a high nibble)
//   value stage  A = w' block-diagonal (rows of slot A against k < 16, slot B against k >= 16),
//                D_v = A x K7, D_blk = D_v + A x codes_blk; acc += s^V D_blk (units of 2^-24)
//
// Memory: per pair 6 loads of distinct bytes (key words of A and B, 1 KiB each; value words, two
// 1 KiB loads; key and value scales of both blocks, 8 bytes per lane each, handed out through the
// wavefront's LDS).  A step computes two pairs while the next two are in flight (deeper prefetch
// measured slower); every load is unconditional (exact compiler wait counts), and a prefetch past the wavefront's range goes through a resource
// of zero size, which returns zeros without touching memory.  No workgroup barrier before the
// loop: the query operand and the DCT constants load straight into registers.
// dwords per wavefront: scales 2 x 256, w' 2 x 128, zero 4, alpha 16, m 16, pad (two pairs a step)
constexpr int kPWaveLds = 808;

typedef _Float16 half4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma16(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1, f32x4 c) {
  // v_mfma_f32_16x16x16_f16: lane l holds A[l%16][4(l/16) + k], B[4(l/16) + k][l%16], k = 0..3
  const half4v a = __builtin_bit_cast(half4v, (uint64_t)a0 | ((uint64_t)a1 << 32));
  const half4v b = __builtin_bit_cast(half4v, (uint64_t)b0 | ((uint64_t)b1 << 32));
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t pk_mul_h(uint32_t a, uint32_t b) { return w2(h2(a) * h2(b)); }

template <int DT>
__device__ __forceinline__ float half_as_f32(uint32_t w, int hi) {
  const uint32_t hbits = hi ? (w >> 16) : (w & 0xffffu);
  if constexpr (DT == KVQ_BF16) return __uint_as_float(hbits << 16);
  else return f16_to_f32(static_cast<uint16_t>(hbits));
}

template <int DT, int kDepth>
__device__ void dct_pair_block(const DctParams& p, int bh, int sidx, float* smem) {
  constexpr int R = 8;
  const int b = bh / p.Hkv, h = bh % p.Hkv;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const int l = threadIdx.x & 63;
  const int g = l >> 4, n = l & 15;
  const bool colB = n >= 8, rowB = g >= 2;
  // epilogue partials [wave][row][d] + [wave][row][m, l], then the per-wavefront loop buffers
  float* red_o = smem;
  float* red_ml = smem + kDWaves * R * kDD;
  uint32_t* wl = reinterpret_cast<uint32_t*>(red_ml + kDWaves * R * 2) + wave * kPWaveLds;
  // per pair of the step (+256 for the second): [0, 128) key scales of A | B, [128, 256) value scales
  uint32_t* sc_l = wl;
  uint32_t* wt = wl + 512;             // w' [16 columns][8 words] per pair (+128 for the second)
  constexpr int kZero = 256;           // 4 zero words after both w' buffers (offset from wt)
  float* al = reinterpret_cast<float*>(wl + 772);       // 16 alphas
  float* mlw = reinterpret_cast<float*>(wl + 788);      // 16 column maxima (epilogue)

  // ---- this wavefront's pairs ----
  const int64_t np = (p.nb + 1) / 2;
  const int NW = p.n_split * kDWaves;
  const int w_all = sidx * kDWaves + wave;
  const int p0 = static_cast<int>(static_cast<int64_t>(w_all) * np / NW);
  const int p1 = static_cast<int>(static_cast<int64_t>(w_all + 1) * np / NW);
  const int p_last = static_cast<int>(np) - 1;

  const int64_t blk0 = static_cast<int64_t>(bh) * p.nb;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(p.kc + blk0 * 1024, static_cast<uint32_t>(p.nb * 1024));
  const __amdgpu_buffer_rsrc_t rks = make_rsrc(p.ks + blk0 * kDD, static_cast<uint32_t>(p.nb * kDD * 2));
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.vc + blk0 * 1024, static_cast<uint32_t>(p.nb * 1024));
  const __amdgpu_buffer_rsrc_t rvs = make_rsrc(p.vs + blk0 * kDD, static_cast<uint32_t>(p.nb * kDD * 2));
  // zero-size resources: a prefetch past the range reads zeros and no memory
  const __amdgpu_buffer_rsrc_t rk0 = make_rsrc(p.kc, 0), rks0 = make_rsrc(p.ks, 0);
  const __amdgpu_buffer_rsrc_t rv0 = make_rsrc(p.vc, 0), rvs0 = make_rsrc(p.vs, 0);
  const int vk = n * 64 + 16 * g;                  // key words 4g .. 4g+3 of coefficient row n
  const int vv = ((g & 1) * 16 + n) * 32;          // value words ((g & 1) * 16 + n) * 8 + 0..7
  const int vsc = (l & 31) * 8;                    // 8 scale bytes of block A (l < 32) or B

  struct Pair {
    u32x4 ka, kb;          // key words of both blocks
    u32x4 vw[2];           // value words of the row slot's block
    uint2 ks, vs;          // 8 bytes of the key / value scales of A (lanes 0-31) or B (32-63)
  };
  // each pair's loads stay one group in program order (the scheduler may not interleave groups):
  // the hardware counts outstanding loads in issue order, so interleaving would make every wait
  // also wait for later pairs
  auto load_pair = [&](int pi, Pair& c) {
    __builtin_amdgcn_sched_barrier(0);
    const bool live = pi < p1;                     // uniform
    pi = max(0, min(pi, p_last));
    const int bA = 2 * pi;
    const int dB = (bA + 1 < p.nb) ? 1 : 0;        // a final single block stands in for its own slot B
    const int sA = __builtin_amdgcn_readfirstlane(bA * 1024);
    const int sB = __builtin_amdgcn_readfirstlane((bA + dB) * 1024);
    const int sS = __builtin_amdgcn_readfirstlane(bA * kDD * 2);
    const __amdgpu_buffer_rsrc_t k_ = live ? rk : rk0, ks_ = live ? rks : rks0;
    const __amdgpu_buffer_rsrc_t v_ = live ? rv : rv0, vs_ = live ? rvs : rvs0;
    // scales first: the step's first wait (for the LDS hand-off) then leaves the codes in flight
    const int os = vsc + ((l >= 32) ? dB * 256 : 0);
    const auto kk = __builtin_amdgcn_raw_buffer_load_b64(ks_, os, sS, 0);
    const auto vv2 = __builtin_amdgcn_raw_buffer_load_b64(vs_, os, sS, 0);
    c.ka = __builtin_amdgcn_raw_buffer_load_b128(k_, vk, sA, 2);
    c.kb = __builtin_amdgcn_raw_buffer_load_b128(k_, vk, sB, 2);
    const int ov = vv + (rowB ? dB * 1024 : 0);
    c.vw[0] = __builtin_amdgcn_raw_buffer_load_b128(v_, ov, sA, 2);
    c.vw[1] = __builtin_amdgcn_raw_buffer_load_b128(v_, ov + 16, sA, 2);
    c.ks = make_uint2(kk[0], kk[1]);
    c.vs = make_uint2(vv2[0], vv2[1]);
    __builtin_amdgcn_sched_barrier(0);
  };

  // ---- prologue: the first kDepth pairs, then the query operand and the DCT constants, all in flight ----
  // (query and table loads first: the wait for them then leaves the pairs' loads outstanding)
  // query operand of the key stage: row n % 8 (rows past R_real read the last row, then zero),
  // channels 32g + 8i + 2jj, +1; x16 on the low-nibble pairs (jj even)
  const int rq = n & 7;
  const uint4* qrow = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.q) +
                                                     dct_q_offset(p, b, h, min(rq, p.R_real - 1)) + 32 * g);
  uint4 qw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) qw[i] = qrow[i];
  // DCT constants: C (16, 64) then C^T (64, 16) in ctab
  const float4* c4 = reinterpret_cast<const float4*>(p.ctab);
  float4 ctl[4], cwl[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) ctl[t] = c4[256 + ((16 * t + n) * 16 + 4 * g) / 4];             // C^T[16t+n][4g..]
#pragma unroll
  for (int k = 0; k < 4; ++k) cwl[k] = c4[(n * kDB + 32 * (k >> 1) + 16 * (k & 1) + 4 * g) / 4];  // C[n][..]
  __builtin_amdgcn_sched_barrier(0);
  Pair buf[kDepth + 2];
#pragma unroll
  for (int j = 0; j < kDepth; ++j) load_pair(p0 + j, buf[j]);
  if (l < 4) wt[kZero + l] = 0u;

  const float qsc = rq < p.R_real ? p.qscale : 0.0f;
  uint32_t qh[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t wv[4] = {qw[i].x, qw[i].y, qw[i].z, qw[i].w};
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const float f = (jj & 1) ? qsc : 16.0f * qsc;
      qh[i][jj] = pack_h2(static_cast<_Float16>(half_as_f32<DT>(wv[jj], 0) * f),
                          static_cast<_Float16>(half_as_f32<DT>(wv[jj], 1) * f));
    }
  }
  // logit tiles: A[token 16t + n][coefficient 4g + k] = C[4g + k][16t + n]
  uint32_t cl[4][2];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    cl[t][0] = pack_h2(static_cast<_Float16>(ctl[t].x), static_cast<_Float16>(ctl[t].y));
    cl[t][1] = pack_h2(static_cast<_Float16>(ctl[t].z), static_cast<_Float16>(ctl[t].w));
  }
  // coefficient stage: A[coefficient n][8g + j] = f_n C[n][32ks + 16(j >> 2) + 4g + (j & 3)]
  const float fn = ((n >> 1) & 1) ? 0.0625f : 1.0f;
  uint32_t cw[2][4];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int jh = 0; jh < 2; ++jh) {
      const float4 v = cwl[2 * ks + jh];
      cw[ks][2 * jh] = pack_h2(static_cast<_Float16>(fn * v.x), static_cast<_Float16>(fn * v.y));
      cw[ks][2 * jh + 1] = pack_h2(static_cast<_Float16>(fn * v.z), static_cast<_Float16>(fn * v.w));
    }
  const u32x4 k7 = u32x4{0x80078007u, 0x80708070u, 0x80078007u, 0x80708070u};

  auto unpack = [](uint32_t w) -> half8 {
    const uint32_t w8 = w >> 8;
    return as_half8(u32x4{w & 0x000F000Fu, w & 0x00F000F0u, w8 & 0x000F000Fu, w8 & 0x00F000F0u});
  };
  constexpr float kTwo20 = 1048576.0f;
  constexpr float kTwo24 = 16777216.0f;
  constexpr float kLazy = 4.0f;
  constexpr float kPOff = 6.0f;

  float acc[8][4];                                 // rows (slot, row) 4g + i, channel 16 blk + n
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k][0] = acc[k][1] = acc[k][2] = acc[k][3] = 0.0f;
  float m_run = -INFINITY, la = 0.0f;              // column n

  // Two pairs per step: their key, logit, coefficient and value stages are independent chains the
  // scheduler interleaves (one wavefront per SIMD has no other wavefront to hide a chain behind),
  // and one softmax update and one LDS hand-off of each kind serve both.  Pair 1 of a step may be
  // dead (past the wavefront's range): its loads read zeros and its logits are masked.
  auto key_stage = [&](const Pair& c, const u32x4 (&sk)[4], uint32_t& ub0, uint32_t& ub1) {
    u32x4 qt[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) qt[i][jj] = pk_mul_h(qh[i][jj], sk[i][jj]);
    // three independent chains (offset, codes of A, codes of B), joined after the select
    f32x4 dc = f32x4{0.f, 0.f, 0.f, 0.f}, da = dc, db = dc;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dc = mfma(as_half8(k7), as_half8(qt[i]), dc);
      da = mfma(unpack(c.ka[i]), as_half8(qt[i]), da);
      db = mfma(unpack(c.kb[i]), as_half8(qt[i]), db);
    }
    const f32x4 du = (colB ? db : da) + dc;
    ub0 = pack_h2(static_cast<_Float16>(du[0] * kTwo20), static_cast<_Float16>(du[1] * kTwo20));
    ub1 = pack_h2(static_cast<_Float16>(du[2] * kTwo20), static_cast<_Float16>(du[3] * kTwo20));
  };
  // logits: token 16t + 4g + i of column n
  auto logit_stage = [&](uint32_t ub0, uint32_t ub1, bool dead, float (&s)[4][4]) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const f32x4 e = mfma16(cl[t][0], cl[t][1], ub0, ub1, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
      for (int i = 0; i < 4; ++i) s[t][i] = dead ? -INFINITY : e[i];
    }
  };
  // coefficient stage: w'[coefficient 4g + i] of column n
  auto coef_stage = [&](const float (&pr)[4][4]) -> f32x4 {
    f32x4 dw = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const u32x4 pb = u32x4{pack_h2(static_cast<_Float16>(pr[2 * ks][0]), static_cast<_Float16>(pr[2 * ks][1])),
                             pack_h2(static_cast<_Float16>(pr[2 * ks][2]), static_cast<_Float16>(pr[2 * ks][3])),
                             pack_h2(static_cast<_Float16>(pr[2 * ks + 1][0]), static_cast<_Float16>(pr[2 * ks + 1][1])),
                             pack_h2(static_cast<_Float16>(pr[2 * ks + 1][2]), static_cast<_Float16>(pr[2 * ks + 1][3]))};
      dw = mfma(as_half8(u32x4{cw[ks][0], cw[ks][1], cw[ks][2], cw[ks][3]}), as_half8(pb), dw);
    }
    return dw;
  };

  auto step2 = [&](const Pair& c0, const Pair& c1, bool hasB0, bool live1, bool hasB1) {
    // ---- scales of both pairs through the wavefront's LDS ----
    *reinterpret_cast<uint2*>(sc_l + 2 * l) = c0.ks;
    *reinterpret_cast<uint2*>(sc_l + 128 + 2 * l) = c0.vs;
    *reinterpret_cast<uint2*>(sc_l + 256 + 2 * l) = c1.ks;
    *reinterpret_cast<uint2*>(sc_l + 384 + 2 * l) = c1.vs;
    wave_lds_fence();
    u32x4 sk0[4], sk1[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sk0[i] = *reinterpret_cast<const u32x4*>(sc_l + (colB ? 64 : 0) + 16 * g + 4 * i);
      sk1[i] = *reinterpret_cast<const u32x4*>(sc_l + 256 + (colB ? 64 : 0) + 16 * g + 4 * i);
    }
    const u32x4 sv0 = *reinterpret_cast<const u32x4*>(sc_l + 128 + (rowB ? 64 : 0) + 4 * n);
    const u32x4 sv1 = *reinterpret_cast<const u32x4*>(sc_l + 384 + (rowB ? 64 : 0) + 4 * n);
    // ---- key and logit stages ----
    uint32_t u00, u01, u10, u11;
    key_stage(c0, sk0, u00, u01);
    key_stage(c1, sk1, u10, u11);
    float s0[4][4], s1[4][4];
    logit_stage(u00, u01, !hasB0 && colB, s0);
    logit_stage(u10, u11, !live1 || (!hasB1 && colB), s1);
    // ---- online softmax over both pairs, lazy maximum ----
    float lm = s0[0][0];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) lm = fmaxf(lm, fmaxf(s0[t][i], s1[t][i]));
    if (__any(lm > m_run + kLazy)) {
      const float m_new = fmaxf(m_run, xmax32(xmax16(lm)));
      const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      la *= alpha;
      m_run = m_new;
      if (g == 0) al[n] = alpha;                   // alpha of column n for the value-stage rows
      wave_lds_fence();
      const float4 a4 = reinterpret_cast<const float4*>(al)[g];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        acc[k][0] *= a4.x;
        acc[k][1] *= a4.y;
        acc[k][2] *= a4.z;
        acc[k][3] *= a4.w;
      }
    }
    const float mo = (m_run == -INFINITY ? 0.0f : m_run) - kPOff;
    float pr0[4][4], pr1[4][4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pr0[t][i] = __builtin_amdgcn_exp2f(s0[t][i] - mo);
        pr1[t][i] = __builtin_amdgcn_exp2f(s1[t][i] - mo);
      }
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) la += pr0[t][i];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) la += pr1[t][i];
    const f32x4 dw0 = coef_stage(pr0), dw1 = coef_stage(pr1);
    // ---- w' of both pairs transposed through LDS into the block-diagonal A operands ----
    *reinterpret_cast<uint2*>(wt + n * 8 + 2 * g) =
        make_uint2(pack_h2(static_cast<_Float16>(dw0[0]), static_cast<_Float16>(dw0[1])),
                   pack_h2(static_cast<_Float16>(dw0[2]), static_cast<_Float16>(dw0[3])));
    *reinterpret_cast<uint2*>(wt + 128 + n * 8 + 2 * g) =
        make_uint2(pack_h2(static_cast<_Float16>(dw1[0]), static_cast<_Float16>(dw1[1])),
                   pack_h2(static_cast<_Float16>(dw1[2]), static_cast<_Float16>(dw1[3])));
    wave_lds_fence();
    const bool diag = colB == rowB;
    const u32x4 aw0 = *reinterpret_cast<const u32x4*>(wt + (diag ? n * 8 + 4 * (g & 1) : kZero));
    const u32x4 aw1 = *reinterpret_cast<const u32x4*>(wt + (diag ? 128 + n * 8 + 4 * (g & 1) : kZero));
    // ---- value stage ----
    const f32x4 dv0 = mfma(as_half8(aw0), as_half8(k7), f32x4{0.f, 0.f, 0.f, 0.f});
    const f32x4 dv1 = mfma(as_half8(aw1), as_half8(k7), f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
      const f32x4 d0 = mfma(as_half8(aw0), unpack(c0.vw[blk >> 2][blk & 3]), dv0);
      const f32x4 d1 = mfma(as_half8(aw1), unpack(c1.vw[blk >> 2][blk & 3]), dv1);
      const float v0 = h2f(sv0[blk >> 1], blk & 1), v1 = h2f(sv1[blk >> 1], blk & 1);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[blk][i] = __builtin_fmaf(v1, d1[i], __builtin_fmaf(v0, d0[i], acc[blk][i]));
    }
  };

  {
    const int last_full = (p.nb & 1) ? p_last : static_cast<int>(np);   // pairs below it have a block B
    // kDepth pairs in flight behind the two being computed; loads unconditional (a pair past the
    // range reads zeros and no memory), steps guarded
    constexpr int NBUF = kDepth + 2;
    static_assert(kDepth % 2 == 0, "pairs go two a step");
    for (int pi = p0; pi < p1; pi += NBUF) {
#pragma unroll
      for (int j = 0; j < NBUF / 2; ++j) {
        const int q = pi + 2 * j;
        load_pair(q + kDepth, buf[(2 * j + kDepth) % NBUF]);
        load_pair(q + kDepth + 1, buf[(2 * j + kDepth + 1) % NBUF]);
        if (j == 0 || q < p1) step2(buf[2 * j], buf[2 * j + 1], q < last_full, q + 1 < p1, q + 1 < last_full);
      }
    }
  }

  // ---- epilogue ----
  // per column (m, l) to the value-stage layout: lane (g, n) needs columns 4g .. 4g+3
  const float l_col = xsum32(xsum16(la));
  if (g == 0) {
    mlw[n] = m_run;
    reinterpret_cast<float*>(wt)[n] = l_col;        // w' buffer is free now
  }
  wave_lds_fence();
  const float4 m4 = reinterpret_cast<const float4*>(mlw)[g];
  const float4 l4 = reinterpret_cast<const float4*>(wt)[g];
  // slots merged in registers: lanes l and l ^ 32 hold rows 4(g & 1) + i of slots A and B; after a
  // permlane32 swap element 0 is slot A's value and element 1 slot B's in both halves
  const float mi[4] = {m4.x, m4.y, m4.z, m4.w}, li[4] = {l4.x, l4.y, l4.z, l4.w};
  float Mr[4], Lr[4], wA[4], wB[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const auto ms = __builtin_amdgcn_permlane32_swap(__float_as_uint(mi[i]), __float_as_uint(mi[i]), false, false);
    const auto ls = __builtin_amdgcn_permlane32_swap(__float_as_uint(li[i]), __float_as_uint(li[i]), false, false);
    const float ma = __uint_as_float(ms[0]), mb = __uint_as_float(ms[1]);
    const float M = fmaxf(ma, mb);
    wA[i] = ma == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ma - M);
    wB[i] = mb == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mb - M);
    Mr[i] = M;
    Lr[i] = wA[i] * __uint_as_float(ls[0]) + wB[i] * __uint_as_float(ls[1]);
  }
  if (g < 2) {
    if (n == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        red_ml[(wave * R + 4 * g + i) * 2 + 0] = Mr[i];
        red_ml[(wave * R + 4 * g + i) * 2 + 1] = Lr[i];
      }
    }
  }
#pragma unroll
  for (int blk = 0; blk < 8; ++blk)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const auto as = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[blk][i]), __float_as_uint(acc[blk][i]),
                                                       false, false);
      const float o = (wA[i] * __uint_as_float(as[0]) + wB[i] * __uint_as_float(as[1])) * kTwo24;
      if (g < 2) red_o[(wave * R + 4 * g + i) * kDD + 16 * blk + n] = o;
    }
  __syncthreads();
  const int64_t po = static_cast<int64_t>(bh) * p.S_all + sidx;
  for (int idx = threadIdx.x; idx < p.R_real * kDD; idx += kDThreads) {
    const int r = idx / kDD, c = idx % kDD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDWaves; ++w) M = fmaxf(M, red_ml[(w * R + r) * 2]);
    float O = 0.0f, L = 0.0f;
#pragma unroll
    for (int w = 0; w < kDWaves; ++w) {
      const float mw_ = red_ml[(w * R + r) * 2];
      const float wgt = (mw_ == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw_ - M);
      O += wgt * red_o[(w * R + r) * kDD + c];
      L += wgt * red_ml[(w * R + r) * 2 + 1];
    }
    p.ws_o[(po * R + r) * kDD + c] = O;
    if (c == 0) {
      p.ws_m[po * R + r] = M - kPOff;
      p.ws_l[po * R + r] = L;
    }
  }
}

// one workgroup per CU (one wavefront per SIMD) with kPairDepth pairs in flight per wavefront: a
// wavefront's prologue and epilogue are paid over more pairs, and the registers a single
// wavefront may hold carry the prefetch and the two pairs of a step
constexpr int kPairDepth = 2;

template <int DT>
__global__ __launch_bounds__(kDThreads) __attribute__((amdgpu_waves_per_eu(1)))
void dct_pair_split(DctParams p) {
  extern __shared__ float smem[];
  const int k = blockIdx.x / 8;
  const int bh = blockIdx.x % 8 + 8 * (k / p.n_split);
  if (bh < p.BH) dct_pair_block<DT, kPairDepth>(p, bh, k % p.n_split, smem);
}

// LDS of the pair kernel: the epilogue's partials and the wavefronts' loop buffers, disjoint
constexpr size_t kPairSmem = (kDWaves * 8 * kDD + kDWaves * 8 * 2 + kDWaves * kPWaveLds) * 4;

}  // namespace
}  // namespace kvq

using namespace kvq;

extern "C" int kvq_dct_encode(const void* x, int x_dtype, int64_t BH, int64_t T, int64_t d, int64_t x_bh,
                              const float* ctab, int for_values, uint8_t* codes, uint16_t* scales, void* stream) {
  KVQ_REQUIRE(valid_dtype(x_dtype), "kvq_dct_encode: bad dtype");
  KVQ_REQUIRE(d == kDD, "kvq_dct_encode: head_dim must be 128");
  KVQ_REQUIRE(BH >= 0 && T >= 0 && T % kDB == 0 && x_bh >= T * d, "kvq_dct_encode: T must be a multiple of 64");
  const int64_t total = BH * (T / kDB) * kDD;
  if (total == 0) return KVQ_OK;
  KVQ_REQUIRE(x && ctab && codes && scales, "kvq_dct_encode: null pointer");
  KVQ_REQUIRE(total / 256 < (1LL << 31), "kvq_dct_encode: too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  KVQ_DISPATCH_DTYPE(x_dtype, hipLaunchKernelGGL((dct_encode_kernel<DT_>), dim3(static_cast<unsigned>((total + 255) / 256)),
                                                dim3(256), 0, s, x, T, x_bh, ctab, for_values, codes, scales, total));
  KVQ_LAUNCH_CHECK("kvq_dct_encode");
  return KVQ_OK;
}

extern "C" int64_t kvq_kivi_decode_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d, int64_t n_q,
                                             int64_t n_exact, int group_k, int group_v, int64_t split_tokens);
extern "C" int kvq_kivi_decode(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st, int64_t B,
                               int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d, float scaling, const uint8_t* kc,
                               const uint16_t* k_lo, const uint16_t* k_sc, const uint8_t* vc, const uint16_t* vmeta,
                               int64_t cap_t, int64_t n_q, int group_k, int group_v, const void* k_exact,
                               const void* v_exact, int exact_dtype, int64_t cap_e, int64_t n_exact,
                               const int64_t* exact_pos, const int64_t* q_pos, void* out, int out_dtype,
                               float* workspace, int64_t workspace_floats, float* scores, int64_t scores_bh,
                               float score_weight, int64_t split_tokens, int phases, void* stream);

namespace {
// split counts: dct_split runs 3 workgroups per CU (LDS-bound, ~41 KB each at 8 rows) over single
// blocks; dct_pair_split (16-bit, R = 8) 1 per CU over pairs of blocks
int dct_splits_single(int64_t BH, int64_t T) { return T > 0 ? kvq::plan_block_splits(BH, T / 64, 3, 4) : 0; }
int dct_splits_pair(int64_t BH, int64_t T) { return T > 0 ? kvq::plan_block_splits(BH, (T / 64 + 1) / 2, 1, 1) : 0; }
// the pair kernel: 16-bit q with R = 8, query rows 16-byte aligned (it loads them as 16-byte words)
bool dct_uses_pairs(int R, int q_dtype, const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st) {
  return R == 8 && q_dtype != KVQ_F32 && reinterpret_cast<uintptr_t>(q) % 16 == 0 && q_sb % 8 == 0 &&
         q_sh % 8 == 0 && q_st % 8 == 0;
}

// workspace floats; *S receives the split count of the kernel `kind` names (1 pairs, 0 single
// blocks, -1 the larger of the two: a size query that does not know the kernel)
int64_t dct_ws_parts(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t T, int64_t n_exact, int kind,
                     int64_t* ex_floats, int* S) {
  const int R = kvq::pow2_rows((Hq / Hkv) * Tq);
  const int s1 = dct_splits_single(B * Hkv, T);
  const int s2 = R == 8 ? dct_splits_pair(B * Hkv, T) : 0;
  *S = kind < 0 ? std::max(s1, s2) : (kind == 1 ? s2 : s1);
  *ex_floats = (n_exact > 0 && !kvq::exact_in_merge(n_exact))
                   ? kvq_kivi_decode_workspace(B, Hq, Hkv, Tq, 128, 0, n_exact, 32, 32, 0) : 0;
  const int Smax = std::max(s1, s2);
  return *ex_floats + B * Hkv * static_cast<int64_t>(Smax) * R * (128 + 2);
}
}  // namespace

extern "C" int64_t kvq_dct_decode_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d, int64_t T,
                                            int64_t n_exact) {
  if (d != 128 || B <= 0 || Hkv <= 0 || Hq % Hkv != 0 || Tq <= 0 || T < 0 || T % 64 != 0) return -1;
  int64_t ex;
  int S;
  return dct_ws_parts(B, Hq, Hkv, Tq, T, n_exact, -1, &ex, &S);
}

extern "C" int kvq_dct_decode(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st, int64_t B,
                              int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d, float scaling, const float* ctab,
                              int64_t T, const uint8_t* kc, const uint16_t* ks, const uint8_t* vc, const uint16_t* vs,
                              const void* k_exact, const void* v_exact, int64_t cap_e, int64_t n_exact,
                              const int64_t* exact_pos, const int64_t* q_pos, void* out, float* workspace,
                              int64_t workspace_floats, int phases, void* stream) {
  KVQ_REQUIRE(phases >= 1 && phases <= 3, "kvq_dct_decode: phases must be 1, 2 or 3");
  KVQ_REQUIRE(d == kDD, "kvq_dct_decode: head_dim must be 128");
  KVQ_REQUIRE(valid_dtype(q_dtype), "kvq_dct_decode: bad dtype");
  KVQ_REQUIRE(B > 0 && Hkv > 0 && Hq % Hkv == 0 && Tq > 0, "kvq_dct_decode: bad head counts");
  const int64_t R_real = (Hq / Hkv) * Tq;
  KVQ_REQUIRE(R_real <= 8, "kvq_dct_decode: rep*Tq must be <= 8");
  KVQ_REQUIRE(T >= 0 && T % kDB == 0, "kvq_dct_decode: T must be a multiple of 64");
  KVQ_REQUIRE(T / kDB * 1024 < (1LL << 31), "kvq_dct_decode: more than 2^21 blocks per head");
  KVQ_REQUIRE(T == 0 || (ctab && kc && ks && vc && vs), "kvq_dct_decode: null coded cache");
  KVQ_REQUIRE(T == 0 || reinterpret_cast<uintptr_t>(ctab) % 16 == 0, "kvq_dct_decode: ctab must be 16-byte aligned");
  KVQ_REQUIRE(T + n_exact > 0, "kvq_dct_decode: empty cache");
  KVQ_REQUIRE(q && out && workspace, "kvq_dct_decode: null q / out / workspace");
  int64_t ex_floats;
  int S;
  const bool pairs = dct_uses_pairs(pow2_rows(R_real), q_dtype, q, q_sb, q_sh, q_st);
  const int64_t need = dct_ws_parts(B, Hq, Hkv, Tq, T, n_exact, pairs ? 1 : 0, &ex_floats, &S);
  KVQ_REQUIRE(workspace_floats >= need, "kvq_dct_decode: workspace too small (%lld < %lld floats)",
              (long long)workspace_floats, (long long)need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int R = pow2_rows(R_real);
  DctParams p{};
  p.q = q; p.q_sb = q_sb; p.q_sh = q_sh; p.q_st = q_st;
  p.Hq = (int)Hq; p.Hkv = (int)Hkv; p.Tq = (int)Tq; p.rep = (int)(Hq / Hkv); p.R_real = (int)R_real;
  p.BH = (int)(B * Hkv);
  p.qscale = scaling * 1.4426950408889634f;
  p.nb = T / kDB;
  p.kc = kc; p.ks = ks; p.vc = vc; p.vs = vs; p.ctab = ctab;
  p.out = out;
  const bool ex_merge = exact_in_merge(n_exact);
  int ex_rows = 0;
  const int64_t S_ex = (ex_merge || n_exact == 0) ? 0 : plan_exact_blocks(B * Hkv, n_exact, &ex_rows);
  if (n_exact > 0 && !ex_merge) {
    if (phases & 1) {
      const int rc = kvq_kivi_decode(q, q_dtype, q_sb, q_sh, q_st, B, Hq, Hkv, Tq, d, scaling, nullptr, nullptr, nullptr,
                                     nullptr, nullptr, 0, 0, 32, 32, k_exact, v_exact, q_dtype, cap_e, n_exact, exact_pos,
                                     q_pos, out, q_dtype, workspace, ex_floats, nullptr, 0, 0.0f, 0, 1, stream);
      if (rc != KVQ_OK) return rc;
    }
    const int64_t nrow = B * Hkv * S_ex * R;
    p.ex_o = workspace;
    p.ex_m = workspace + nrow * 128;
    p.ex_l = p.ex_m + nrow;
    p.S_ex = (int)S_ex;
  }
  float* tw = workspace + ex_floats;
  const int64_t trow = B * Hkv * static_cast<int64_t>(S) * R;
  p.ws_o = tw;
  p.ws_m = tw + trow * 128;
  p.ws_l = p.ws_m + trow;
  p.S_all = S;
  p.n_split = S;
  const int bh_pad = (p.BH + 7) / 8 * 8;
  const size_t split_smem = std::max<size_t>(
      (R * kDD + kDWaves * (2 * R * kBqStride + R * 16) + kDWaves * R * 19) * sizeof(float) + 12 * 64 * 16 + kDK * kDB * 4,
      (kDWaves * R * kDD + kDWaves * 2 * R) * sizeof(float));
  if (S > 0 && (phases & 1) && pairs) {
    if (q_dtype == KVQ_F16)
      hipLaunchKernelGGL((dct_pair_split<KVQ_F16>), dim3(static_cast<unsigned>(S) * bh_pad), dim3(kDThreads), kPairSmem, s, p);
    else
      hipLaunchKernelGGL((dct_pair_split<KVQ_BF16>), dim3(static_cast<unsigned>(S) * bh_pad), dim3(kDThreads), kPairSmem, s, p);
    KVQ_LAUNCH_CHECK("kvq_dct_decode(pair split)");
  } else if (S > 0 && (phases & 1)) {
#define KVQ_DCT_SPLIT(R_, DT_) \
    hipLaunchKernelGGL((dct_split<R_, DT_>), dim3(static_cast<unsigned>(S) * bh_pad), dim3(kDThreads), split_smem, s, p)
#define KVQ_DCT_R(DT_)                                   \
    switch (R) {                                         \
      case 1: KVQ_DCT_SPLIT(1, DT_); break;              \
      case 2: KVQ_DCT_SPLIT(2, DT_); break;              \
      case 4: KVQ_DCT_SPLIT(4, DT_); break;              \
      default: KVQ_DCT_SPLIT(8, DT_); break;             \
    }
    switch (q_dtype) {
      case KVQ_F32: KVQ_DCT_R(KVQ_F32) break;
      case KVQ_F16: KVQ_DCT_R(KVQ_F16) break;
      default: KVQ_DCT_R(KVQ_BF16) break;
    }
#undef KVQ_DCT_R
#undef KVQ_DCT_SPLIT
    KVQ_LAUNCH_CHECK("kvq_dct_decode(split)");
  }
  if (phases & 2) {
    MergeArgs ma{p.ws_o, p.ws_m, p.ws_l, p.S_all, p.ex_o, p.ex_m, p.ex_l, p.S_ex,
                 p.Hq, p.Hkv, p.Tq, p.rep, p.R_real, p.out, nullptr, ExactArgs{}};
    if (ex_merge)
      ma.ex = ExactArgs{q, q_sb, q_sh, q_st, p.qscale, k_exact, v_exact, cap_e, static_cast<int>(n_exact), exact_pos, q_pos};
    const int rc = launch_merge_rows(ma, R, p.BH, q_dtype, s);
    if (rc != KVQ_OK) return rc;
  }
  return KVQ_OK;
}
