// Mixed-width KIVI cache (C3): every 64-token block of a (b, h) has its own code width b in
// {2, 4, 8}; inside the block the codes and fp16 metadata are kivi_quant's (STRATA_KV.py:826-856)
// at that width with group 32 (keys per channel over the block's two 32-token groups, values per
// token over four 32-channel groups).  One launch decodes all widths.
//
// Storage: one flat byte buffer.  The blocks of (b, h) occupy a contiguous region starting at
// 2 KiB unit bh_base[bh], ordered by width (8-bit blocks, then 4-bit, then 2-bit; token order
// within a width).  A block of width b takes (b + 1) units:
//   0                 key rows, planar (pack_planar layout, STRATA_KV.py:1171-1182), 64 x 16b bytes
//   1024 b            value tiles of the block's two 32-token chunks, 512 b bytes each
//   2048 b            key scales sc[2][128] fp16, then key zeros lo[2][128] fp16
//   2048 b + 1024     value (scale, zero) per chunk: word [group 4][lane group 4][slot 8], scale in
//                     the low half, zero in the high half (slot j of lane group g = token
//                     slot_token(g, j) of the chunk)
// Offset table: blk_off[bh][blk] (units from bh_base, token order) and blk_bits[bh][blk]; the
// decode reads the per-(b, h) segment table seg[bh] = {bh_base, n8, n4, n2}.
//
// Decode: as the packed 4-bit kernel (scales folded into the query per key group, the zero
// through a virtual k-step, value scales into the probabilities, zero term summed per group),
// with the width-generic operand unpacking: a wavefront takes a range of the (b, h)'s blocks
// balanced by bytes and runs the 8-, 4- and 2-bit parts of it with one specialised loop each.
#include "common.hpp"
#include "mfma_common.hpp"
#include "partials.hpp"
#include "widths.hpp"

// Build-time switches: KVQ_MIXED_CLASSES 1 lets a plan that is exactly one round of blocks be
// class-major with splits sized by dispatch class, weights KVQ_MIXED_W0 : W1 : W2 (see
// class_block_of); 0 keeps the plain mapping and equal splits.  Weights measured at C3: 180 : 92 :
// 50 gives a 33.6 us step, 165 : 95 : 55 33.9, 150 : 100 : 62 34.6, 190 : 88 : 45 35.1.
#ifndef KVQ_MIXED_CLASSES
#define KVQ_MIXED_CLASSES 1
#endif
#ifndef KVQ_MIXED_W0
#define KVQ_MIXED_W0 180
#endif
#ifndef KVQ_MIXED_W1
#define KVQ_MIXED_W1 92
#endif
#ifndef KVQ_MIXED_W2
#define KVQ_MIXED_W2 50
#endif

namespace kvq {
namespace {

constexpr int kMD = 128;
constexpr int kMThreads = 256;
constexpr int kMWaves = 4;
constexpr int kUnit = 2048;

__device__ __forceinline__ float m_as_stored(float x) {
  x = fminf(fmaxf(x, -65504.0f), 65504.0f);
  return f16_to_f32(f32_to_f16(x));
}
__device__ __forceinline__ int m_code(float x, float lo, float sc, int qmax) {
  const float t = rintf(__fdiv_rn(__fsub_rn(x, lo), sc));
  return static_cast<int>(fminf(fmaxf(t, 0.0f), static_cast<float>(qmax)));
}

// One workgroup per (block, b*h): kivi_quant of the block's keys and values at its width.
template <int DT>
__global__ __launch_bounds__(kMThreads) void mixed_encode_kernel(const void* __restrict__ k, const void* __restrict__ v,
                                                                 int64_t x_bh, const uint8_t* __restrict__ blk_bits,
                                                                 const int32_t* __restrict__ blk_off,
                                                                 const int64_t* __restrict__ bh_base, int nb,
                                                                 uint8_t* __restrict__ buf) {
  __shared__ uint8_t ck[64][kMD];
  __shared__ uint8_t cv[64][kMD];
  const int blk = blockIdx.x, bh = blockIdx.y;
  const int64_t bi = static_cast<int64_t>(bh) * nb + blk;
  const int bits = blk_bits[bi];
  const int qmax = (1 << bits) - 1;
  uint8_t* seg = buf + (bh_base[bh] + blk_off[bi]) * kUnit;
  const int64_t x0 = static_cast<int64_t>(bh) * x_bh + static_cast<int64_t>(blk) * 64 * kMD;
  const int tid = threadIdx.x;
  uint16_t* kmeta = reinterpret_cast<uint16_t*>(seg + 2048 * bits);
  uint32_t* vmeta = reinterpret_cast<uint32_t*>(seg + 2048 * bits + 1024);
  {
    // keys: thread (group grp, channel c) over tokens 32 grp .. 32 grp + 31
    const int c = tid & 127, grp = tid >> 7;
    float mn = INFINITY, mx = -INFINITY;
    for (int t = 0; t < 32; ++t) {
      const float x = load_as_f32<DT>(k, x0 + static_cast<int64_t>(32 * grp + t) * kMD + c);
      mn = fminf(mn, x);
      mx = fmaxf(mx, x);
    }
    const float lo = m_as_stored(mn);
    const float sc = fmaxf(m_as_stored(__fdiv_rn(__fsub_rn(mx, lo), static_cast<float>(qmax))), 5.9604644775390625e-08f);
    kmeta[grp * kMD + c] = f32_to_f16(sc);
    kmeta[256 + grp * kMD + c] = f32_to_f16(lo);
    for (int t = 0; t < 32; ++t) {
      const float x = load_as_f32<DT>(k, x0 + static_cast<int64_t>(32 * grp + t) * kMD + c);
      ck[32 * grp + t][c] = static_cast<uint8_t>(m_code(x, lo, sc, qmax));
    }
  }
  {
    // values: thread (token t, channel group gv) over channels 32 gv .. 32 gv + 31
    const int t = tid >> 2, gv = tid & 3;
    const int64_t ro = x0 + static_cast<int64_t>(t) * kMD + 32 * gv;
    float mn = INFINITY, mx = -INFINITY;
    for (int j = 0; j < 32; ++j) {
      const float x = load_as_f32<DT>(v, ro + j);
      mn = fminf(mn, x);
      mx = fmaxf(mx, x);
    }
    const float lo = m_as_stored(mn);
    const float sc = fmaxf(m_as_stored(__fdiv_rn(__fsub_rn(mx, lo), static_cast<float>(qmax))), 5.9604644775390625e-08f);
    for (int j = 0; j < 32; ++j) cv[t][32 * gv + j] = static_cast<uint8_t>(m_code(load_as_f32<DT>(v, ro + j), lo, sc, qmax));
    const int cc = t >> 5, tl = t & 31;
    const int g = (tl & 15) >> 2, slot = 4 * (tl >> 4) + (tl & 3);
    vmeta[cc * 128 + gv * 32 + g * 8 + slot] =
        static_cast<uint32_t>(f32_to_f16(sc)) | (static_cast<uint32_t>(f32_to_f16(lo)) << 16);
  }
  __syncthreads();
  // key rows, planar: byte i of a row holds coordinates i + p * 16b in bits [p b, (p + 1) b)
  const int rb = 16 * bits;
  uint32_t* krow = reinterpret_cast<uint32_t*>(seg);
  for (int wi = tid; wi < 256 * bits; wi += kMThreads) {
    const int t = wi / (4 * bits), wr = wi % (4 * bits);
    uint32_t word = 0;
    for (int bb = 0; bb < 4; ++bb) {
      const int i = 4 * wr + bb;
      uint32_t byte = 0;
      for (int p = 0; p < 8 / bits; ++p) byte |= static_cast<uint32_t>(ck[t][p * rb + i]) << (p * bits);
      word |= byte << (8 * bb);
    }
    krow[wi] = word;
  }
  uint32_t* vt = reinterpret_cast<uint32_t*>(seg + 1024 * bits);
  for (int wi = tid; wi < 256 * bits; wi += kMThreads) {
    const int cc = wi / (128 * bits), w = wi % (128 * bits);
    auto code_at = [&](int slot, int g, int ch) -> uint32_t {
      return static_cast<uint32_t>(cv[32 * cc + slot_token(g, slot)][ch]);
    };
    vt[wi] = vtile_word(bits, w, code_at);
  }
}

// ---------------------------------------------------------------------------------------------
// decode

struct MixedParams {
  const void* q;
  int64_t q_sb, q_sh, q_st;
  int Hq, Hkv, Tq, rep, R_real, BH;
  float qscale;
  const uint8_t* buf;
  const int64_t* seg;               // (BH, 4): base unit, n8, n4, n2
  int n_split;
  int split_classes;                // > 0: class-major blocks, splits sized by dispatch class
  float* ws_o;
  float* ws_m;
  float* ws_l;
};

// LO (fp32 output): p * scale enters the PV product as hi + lo fp16 parts, two column variants
// per channel group; 16-bit outputs take the single fp16 rounding (relative error 2^-12 per
// term, below the output's own rounding), one column per group.
template <int R, bool LO>
struct MixedGeom {
  static constexpr int VPB = 16 / R;               // PV columns per row: (group[, hi/lo]) variants
  static constexpr int GPB = LO ? VPB / 2 : VPB;   // channel groups per PV B operand
  static constexpr int NB = (4 + GPB - 1) / GPB;   // PV B operands (4 groups of 32 channels)
};

template <int R, bool LO>
struct MixedState {
  f32x4 acc[8];
  float m_run, la;
  float Z[MixedGeom<R, LO>::NB];
};

struct MixedLane {
  int l, g, n, r_n, hl_qk, gcl, hl_pv, ci, ck;
};

// Blocks [kb0, kb1) of one width segment starting at byte seg_so of the (b, h) region.
template <int BITS, int R, bool LO>
__device__ __forceinline__ void mixed_run(MixedState<R, LO>& st, const MixedLane& L, const float (*qs)[kMD], uint32_t* bq,
                                          uint32_t* bv, __amdgpu_buffer_rsrc_t rs, uint32_t seg_so, int kb0, int kb1) {
  using Geo = MixedGeom<R, LO>;
  constexpr int NB = Geo::NB, GPB = Geo::GPB;
  constexpr int RB = 16 * BITS;                    // bytes per planar key row
  constexpr int SEG = (BITS + 1) * kUnit;
  constexpr int NCLS = BITS == 2 ? 4 : (BITS == 4 ? 2 : 1);
  const int g = L.g, n = L.n, l = L.l;
  const int c0 = key_channel<BITS>(g, L.ci, 2 * L.ck);
  const int c1 = key_channel<BITS>(g, L.ci, 2 * L.ck + 1);
  // element pair (2ck, 2ck+1) carries 2^code_shift: its query operand takes 2^(4 - code_shift),
  // so every key product carries 2^-20
  const float kinv = static_cast<float>(1 << (6 - code_shift<BITS>(2 * L.ck))) * 0.25f;
  const int vo_k = n * RB + g * 4 * BITS;
  int vo_m[NB];
#pragma unroll
  for (int bb = 0; bb < NB; ++bb) {
    const int gc = bb * GPB + L.gcl;
    vo_m[bb] = (gc < 4 ? gc : 0) * 128 + g * 32;
  }
  struct Chunk {
    uint32_t kw[2][BITS];
    uint32_t vw[2 * BITS];
    u32x4 mw[NB][2];
    uint32_t ks0, ks1, kl0, kl1;
  };
  const int c_last = 2 * kb1 - 1;
  auto load_chunk = [&](int cix, Chunk& c) {
    cix = min(cix, c_last);
    const int kb = cix >> 1, cc = cix & 1;
    const uint32_t so = seg_so + static_cast<uint32_t>(kb) * SEG;
    const int so_k = __builtin_amdgcn_readfirstlane(so + cc * 32 * RB);
#pragma unroll
    for (int tau = 0; tau < 2; ++tau) {
      const int vo = vo_k + tau * 16 * RB;
      if constexpr (BITS == 2) {
        const auto x = __builtin_amdgcn_raw_buffer_load_b64(rs, vo, so_k, 2);
        c.kw[tau][0] = x[0];
        c.kw[tau][1] = x[1];
      } else {
#pragma unroll
        for (int i = 0; i < BITS / 4; ++i) {
          const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rs, vo + 16 * i, so_k, 2);
#pragma unroll
          for (int k = 0; k < 4; ++k) c.kw[tau][4 * i + k] = x[k];
        }
      }
    }
    const int so_v = __builtin_amdgcn_readfirstlane(so + 1024 * BITS + cc * 512 * BITS);
#pragma unroll
    for (int i = 0; i < BITS / 2; ++i) {
      const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rs, l * 16 + 1024 * i, so_v, 2);
#pragma unroll
      for (int k = 0; k < 4; ++k) c.vw[4 * i + k] = x[k];
    }
    const int so_vm = __builtin_amdgcn_readfirstlane(so + 2048 * BITS + 1024 + cc * 512);
#pragma unroll
    for (int bb = 0; bb < NB; ++bb) {
      c.mw[bb][0] = __builtin_amdgcn_raw_buffer_load_b128(rs, vo_m[bb], so_vm, 2);
      c.mw[bb][1] = __builtin_amdgcn_raw_buffer_load_b128(rs, vo_m[bb] + 16, so_vm, 2);
    }
    const int so_km = __builtin_amdgcn_readfirstlane(so + 2048 * BITS + cc * 256);
    c.ks0 = __builtin_amdgcn_raw_buffer_load_b16(rs, c0 * 2, so_km, 0);
    c.ks1 = __builtin_amdgcn_raw_buffer_load_b16(rs, c1 * 2, so_km, 0);
    c.kl0 = __builtin_amdgcn_raw_buffer_load_b16(rs, 512 + c0 * 2, so_km, 0);
    c.kl1 = __builtin_amdgcn_raw_buffer_load_b16(rs, 512 + c1 * 2, so_km, 0);
  };

  constexpr float kTwo20 = 1048576.0f;
  constexpr float kLazy = 4.0f;
  const half8 tiny = as_half8(u32x4{0x00100010u, 0x00100010u, 0x00100010u, 0x00100010u});   // 2^-20
  const half2v hl_neg = L.hl_pv ? half2v{static_cast<_Float16>(-1.0f), static_cast<_Float16>(-1.0f)}
                                : half2v{static_cast<_Float16>(0.0f), static_cast<_Float16>(0.0f)};
  const u32x4* bq_src = reinterpret_cast<const u32x4*>(bq + (2 * L.r_n + L.hl_qk) * kBqStride + g * 16);
  const u32x4* bv_src = reinterpret_cast<const u32x4*>(bv + L.r_n * 16 + g * 4);
  // probability and zero-point sums per code-factor class, folded into the state at the end
  float lc[NCLS], zc[NCLS][NB];
#pragma unroll
  for (int k = 0; k < NCLS; ++k) {
    lc[k] = 0.0f;
#pragma unroll
    for (int bb = 0; bb < NB; ++bb) zc[k][bb] = 0.0f;
  }
  auto cls = [](int j) -> int { return BITS == 2 ? (j >> 1) : (BITS == 4 ? ((j >> 1) & 1) : 0); };

  auto step = [&](const Chunk& c) {
    // ---- the chunk is one key group: B operand q * sc (hi / lo) and the bias q . lo ----
    wave_lds_fence();
    {
      const float sc0 = h2f(c.ks0, 0), sc1 = h2f(c.ks1, 0);
      const float lo0 = h2f(c.kl0, 0), lo1 = h2f(c.kl1, 0);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float qa = qs[r][c0], qb = qs[r][c1];
        const float x0 = qa * kinv * sc0, x1 = qb * kinv * sc1;
        const _Float16 h0 = static_cast<_Float16>(x0), h1 = static_cast<_Float16>(x1);
        bq[(2 * r) * kBqStride + l] = pack_h2(h0, h1);
        bq[(2 * r + 1) * kBqStride + l] = pack_h2(static_cast<_Float16>(x0 - static_cast<float>(h0)),
                                           static_cast<_Float16>(x1 - static_cast<float>(h1)));
        float P = qa * lo0 + qb * lo1;
        P += dpp<kQuadSwap1>(P);
        P += dpp<kQuadSwap2>(P);
        if (L.ck == 0) {
          const _Float16 ph = static_cast<_Float16>(P);
          bv[r * 16 + g * 4 + L.ci] = pack_h2(ph, static_cast<_Float16>(P - static_cast<float>(ph)));
        }
      }
    }
    wave_lds_fence();
    half8 bqk[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) bqk[i] = as_half8(bq_src[i]);
    u32x4 bvr = *bv_src;
    if (L.hl_qk) bvr = u32x4{0u, 0u, 0u, 0u};
    const half8 bvirt = as_half8(bvr);
    // ---- logits (2^-20 units) ----
    float s[8];
#pragma unroll
    for (int tau = 0; tau < 2; ++tau) {
      f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        half8 a;
        if constexpr (BITS == 4) a = unpack4(c.kw[tau][w]);
        else if constexpr (BITS == 8) a = unpack8(c.kw[tau][2 * w], c.kw[tau][2 * w + 1]);
        else a = unpack2((w & 1) ? (c.kw[tau][w >> 1] >> 8) : c.kw[tau][w >> 1]);
        d = mfma(a, bqk[w], d);
      }
      d = mfma(tiny, bvirt, d);
#pragma unroll
      for (int i = 0; i < 4; ++i) s[4 * tau + i] = d[i] + dpp<kRowRor + R>(d[i]);
    }
    // ---- online softmax (base 2), lazy maximum ----
    float lm = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
    if (__any(lm * kTwo20 > st.m_run + kLazy)) {
      const float m_new = fmaxf(st.m_run, xmax32(xmax16(lm)) * kTwo20);
      const float alpha = __builtin_amdgcn_exp2f(st.m_run - m_new);
#pragma unroll
      for (int k = 0; k < 8; ++k) st.acc[k] *= alpha;
#pragma unroll
      for (int bb = 0; bb < NB; ++bb) st.Z[bb] *= alpha;
      st.la *= alpha;
#pragma unroll
      for (int k = 0; k < NCLS; ++k) {
        lc[k] *= alpha;
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) zc[k][bb] *= alpha;
      }
      st.m_run = m_new;
    }
    // slot j's value code carries 2^code_shift(j): its probability is taken divided by it
    float pr[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      pr[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j], kTwo20, -(st.m_run + static_cast<float>(code_shift<BITS>(j)))));
#pragma unroll
    for (int j = 0; j < 8; ++j) lc[cls(j)] += pr[j];
    half8 bp[NB];
#pragma unroll
    for (int bb = 0; bb < NB; ++bb) {
      uint32_t words[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int j0 = 2 * jj, j1 = 2 * jj + 1;
        const half2v m0 = h2(c.mw[bb][j0 >> 2][j0 & 3]);          // (scale, zero) of slot j0
        const half2v m1 = h2(c.mw[bb][j1 >> 2][j1 & 3]);
        const half2v hi = half2v{static_cast<_Float16>(__builtin_fmaf(pr[j0], static_cast<float>(m0[0]), 0.0f)),
                                 static_cast<_Float16>(__builtin_fmaf(pr[j1], static_cast<float>(m1[0]), 0.0f))};
        if constexpr (LO) {
          const half2v cn = hi * hl_neg;
          const half2v val = half2v{static_cast<_Float16>(__builtin_fmaf(pr[j0], static_cast<float>(m0[0]), static_cast<float>(cn[0]))),
                                    static_cast<_Float16>(__builtin_fmaf(pr[j1], static_cast<float>(m1[0]), static_cast<float>(cn[1])))};
          words[jj] = w2(val);
        } else {
          words[jj] = w2(hi);
        }
        zc[cls(j0)][bb] = __builtin_fmaf(pr[j0], static_cast<float>(m0[1]), zc[cls(j0)][bb]);
        zc[cls(j1)][bb] = __builtin_fmaf(pr[j1], static_cast<float>(m1[1]), zc[cls(j1)][bb]);
      }
      bp[bb] = as_half8(u32x4{words[0], words[1], words[2], words[3]});
    }
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
      half8 a;
      if constexpr (BITS == 4) a = unpack4(c.vw[blk]);
      else if constexpr (BITS == 8) a = unpack8(c.vw[(blk >> 1) * 4 + (blk & 1) * 2], c.vw[(blk >> 1) * 4 + (blk & 1) * 2 + 1]);
      else a = unpack2((blk & 1) ? (c.vw[blk >> 1] >> 8) : c.vw[blk >> 1]);
      st.acc[blk] = mfma(a, bp[(blk >> 1) / GPB], st.acc[blk]);
    }
  };

  {
    Chunk ca, cb_;
    const int c_first = 2 * kb0;
    load_chunk(c_first, ca);
    for (int ci = c_first;; ci += 2) {
      load_chunk(ci + 1, cb_);
      step(ca);
      if (ci + 1 > c_last) break;
      load_chunk(ci + 2, ca);
      step(cb_);
      if (ci + 2 > c_last) break;
    }
  }
#pragma unroll
  for (int k = 0; k < NCLS; ++k) {
    const float f = static_cast<float>(1 << (BITS == 2 ? 2 * k : 4 * k));
    st.la = __builtin_fmaf(lc[k], f, st.la);
#pragma unroll
    for (int bb = 0; bb < NB; ++bb) st.Z[bb] = __builtin_fmaf(zc[k][bb], f, st.Z[bb]);
  }
}

// first block (storage order) whose start, in 2 KiB units, is >= c
__device__ __forceinline__ int mixed_first_block(int64_t c, int n8, int n4, int n2) {
  if (c <= 9LL * n8) return static_cast<int>((c + 8) / 9);
  c -= 9LL * n8;
  if (c <= 5LL * n4) return n8 + static_cast<int>((c + 4) / 5);
  c -= 5LL * n4;
  return n8 + n4 + static_cast<int>(min<int64_t>((c + 2) / 3, n2));
}

template <int R, int DT>
__device__ void mixed_block(const MixedParams& p, int bh, int sidx, float* smem) {
  constexpr bool LO = DT == KVQ_F32;
  using Geo = MixedGeom<R, LO>;
  constexpr int NB = Geo::NB, GPB = Geo::GPB;
  const int b = bh / p.Hkv, h = bh % p.Hkv;
  float (*qs)[kMD] = reinterpret_cast<float (*)[kMD]>(smem);
  uint32_t* bq_all = reinterpret_cast<uint32_t*>(smem + R * kMD);    // [wave][2R][64]
  uint32_t* bv_all = bq_all + kMWaves * 2 * R * kBqStride;                  // [wave][R][16]
  for (int idx = threadIdx.x; idx < R * kMD; idx += kMThreads) {
    const int r = idx / kMD, c = idx % kMD;
    float x = 0.0f;
    if (r < p.R_real) {
      const int hq = h * p.rep + r / p.Tq, t = r % p.Tq;
      x = load_as_f32<DT>(p.q, static_cast<int64_t>(b) * p.q_sb + static_cast<int64_t>(hq) * p.q_sh +
                                   static_cast<int64_t>(t) * p.q_st + c) * p.qscale;
    }
    qs[r][c] = x;
  }
  __syncthreads();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  MixedLane L;
  L.l = threadIdx.x % 64;
  L.g = L.l >> 4;
  L.n = L.l & 15;
  L.r_n = L.n % R;
  L.hl_qk = (L.n / R) & 1;
  const int v_pv = L.n / R;
  L.gcl = LO ? (v_pv >> 1) : v_pv;
  L.hl_pv = LO ? (v_pv & 1) : 0;
  L.ci = (L.l >> 2) & 3;
  L.ck = L.l & 3;
  uint32_t* bq = bq_all + wave * 2 * R * kBqStride;
  uint32_t* bv = bv_all + wave * R * 16;

  const int64_t base = p.seg[bh * 4];
  const int n8 = static_cast<int>(p.seg[bh * 4 + 1]);
  const int n4 = static_cast<int>(p.seg[bh * 4 + 2]);
  const int n2 = static_cast<int>(p.seg[bh * 4 + 3]);
  const int64_t C = 9LL * n8 + 5LL * n4 + 3LL * n2;
  // the split's share of the (b, h)'s cost units (by its dispatch class's weight when the plan has
  // classes), a quarter of it per wavefront
  const int64_t cwt = class_weight_before(p.n_split, p.n_split, p.split_classes, KVQ_MIXED_W0, KVQ_MIXED_W1, KVQ_MIXED_W2);
  const int64_t sc0 = C * class_weight_before(sidx, p.n_split, p.split_classes, KVQ_MIXED_W0, KVQ_MIXED_W1, KVQ_MIXED_W2) / cwt;
  const int64_t sc1 = C * class_weight_before(sidx + 1, p.n_split, p.split_classes, KVQ_MIXED_W0, KVQ_MIXED_W1, KVQ_MIXED_W2) / cwt;
  const int i0 = mixed_first_block(sc0 + (sc1 - sc0) * wave / kMWaves, n8, n4, n2);
  const int i1 = mixed_first_block(sc0 + (sc1 - sc0) * (wave + 1) / kMWaves, n8, n4, n2);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.buf + base * kUnit, static_cast<uint32_t>(C * kUnit));

  MixedState<R, LO> st;
#pragma unroll
  for (int k = 0; k < 8; ++k) st.acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
  st.m_run = -INFINITY;
  st.la = 0.0f;
#pragma unroll
  for (int bb = 0; bb < NB; ++bb) st.Z[bb] = 0.0f;
  {
    const int a = i0, e = min(i1, n8);
    if (a < e) mixed_run<8, R, LO>(st, L, qs, bq, bv, rs, 0u, a, e);
  }
  {
    const int a = max(i0, n8) - n8, e = min(i1, n8 + n4) - n8;
    if (a < e) mixed_run<4, R, LO>(st, L, qs, bq, bv, rs, static_cast<uint32_t>(9 * n8) * kUnit, a, e);
  }
  {
    const int a = max(i0, n8 + n4) - (n8 + n4), e = i1 - (n8 + n4);
    if (a < e) mixed_run<2, R, LO>(st, L, qs, bq, bv, rs, static_cast<uint32_t>(9 * n8 + 5 * n4) * kUnit, a, e);
  }

  // ---- wavefront epilogue (as the packed 4-bit kernel) ----
  const float l_run = xsum32(xsum16(st.la));
  float Z[NB];
#pragma unroll
  for (int k = 0; k < NB; ++k) Z[k] = xsum32(xsum16(st.Z[k]));
  __syncthreads();
  float* red_o = smem;                            // [wave][R][d]
  float* red_ml = smem + kMWaves * R * kMD;       // [wave][2][R]
  constexpr float kTwo24 = 16777216.0f;
#pragma unroll
  for (int blk = 0; blk < 8; ++blk) {
    const int gcb = blk >> 1;
    const bool mine = (!LO || L.hl_pv == 1) && (gcb % GPB) == L.gcl;
    const float Zv = Z[gcb / GPB];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float a = st.acc[blk][i];
      if constexpr (LO) a += dpp<kRowShr + R>(st.acc[blk][i]);
      if (mine) red_o[(wave * R + L.r_n) * kMD + 16 * blk + 4 * L.g + i] = __builtin_fmaf(a, kTwo24, Zv);
    }
  }
  if (L.g == 0 && L.n < R) {
    red_ml[(wave * 2 + 0) * R + L.n] = st.m_run;
    red_ml[(wave * 2 + 1) * R + L.n] = l_run;
  }
  __syncthreads();
  const int64_t po = static_cast<int64_t>(bh) * p.n_split + sidx;
  for (int idx = threadIdx.x; idx < p.R_real * kMD; idx += kMThreads) {
    const int r = idx / kMD, c = idx % kMD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kMWaves; ++w) M = fmaxf(M, red_ml[(w * 2) * R + r]);
    float O = 0.0f, Lsum = 0.0f;
#pragma unroll
    for (int w = 0; w < kMWaves; ++w) {
      const float mw_ = red_ml[(w * 2) * R + r];
      const float wgt = (mw_ == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw_ - M);
      O += wgt * red_o[(w * R + r) * kMD + c];
      Lsum += wgt * red_ml[(w * 2 + 1) * R + r];
    }
    p.ws_o[(po * R + r) * kMD + c] = O;
    if (c == 0) {
      p.ws_m[po * R + r] = M;
      p.ws_l[po * R + r] = Lsum;
    }
  }
}

// waves per SIMD the split kernel's registers target: 3 where that fits without spilling in the
// loop (16-bit output, R <= 4), else 2; KVQ_MIXED_WAVES overrides it at build time
#ifndef KVQ_MIXED_WAVES
#define KVQ_MIXED_WAVES 0
#endif
template <int R, int DT>
constexpr int mixed_waves() {
  return KVQ_MIXED_WAVES > 0 ? KVQ_MIXED_WAVES : ((DT != KVQ_F32 && R <= 4) ? 3 : 2);
}

template <int R, int DT>
__global__ __launch_bounds__(kMThreads) __attribute__((amdgpu_waves_per_eu(mixed_waves<R, DT>())))
void mixed_split(MixedParams p) {
  extern __shared__ float smem[];
  int bh, sidx;
  class_block_of(blockIdx.x, p.n_split, p.split_classes, &bh, &sidx);
  if (bh < p.BH) mixed_block<R, DT>(p, bh, sidx, smem);
}


}  // namespace
}  // namespace kvq

using namespace kvq;

extern "C" int kvq_mixed_encode(const void* k, const void* v, int dtype, int64_t BH, int64_t nb, int64_t d,
                                int64_t x_bh, const uint8_t* blk_bits, const int32_t* blk_off, const int64_t* bh_base,
                                uint8_t* buf, void* stream) {
  KVQ_REQUIRE(valid_dtype(dtype), "kvq_mixed_encode: bad dtype");
  KVQ_REQUIRE(d == kMD, "kvq_mixed_encode: head_dim must be 128");
  KVQ_REQUIRE(BH >= 0 && nb >= 0 && x_bh >= nb * 64 * d, "kvq_mixed_encode: bad shape");
  if (BH == 0 || nb == 0) return KVQ_OK;
  KVQ_REQUIRE(k && v && blk_bits && blk_off && bh_base && buf, "kvq_mixed_encode: null pointer");
  KVQ_REQUIRE(nb < 65536 && BH < 65536, "kvq_mixed_encode: too many blocks");
  hipStream_t s = static_cast<hipStream_t>(stream);
  KVQ_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((mixed_encode_kernel<DT_>), dim3(static_cast<unsigned>(nb), static_cast<unsigned>(BH)),
                                               dim3(kMThreads), 0, s, k, v, x_bh, blk_bits, blk_off, bh_base,
                                               static_cast<int>(nb), buf));
  KVQ_LAUNCH_CHECK("kvq_mixed_encode");
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
int64_t mixed_ws_parts(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t nb, int64_t n_exact, int64_t* ex_floats,
                       int* S) {
  // resident blocks per CU = waves per SIMD of the variant (one wavefront of each block per SIMD);
  // a plan as fast as the best that is exactly one round of class-major blocks is preferred
  const int64_t Rr = kvq::pow2_rows((Hq / Hkv) * Tq);
  const int res = (Rr <= 4) ? 3 : 2;
  *S = nb > 0 ? kvq::plan_block_splits(B * Hkv, nb, res, 4) : 0;
  if (*S > 0 && KVQ_MIXED_CLASSES != 0 && (B * Hkv) % 8 == 0) {
    const int64_t s_cls = 3LL * kvq::kCUsPerXcd * 8 / (B * Hkv);
    const int64_t slots = 256LL * res;
    auto cost = [&](int64_t sv) { return ((B * Hkv * sv + slots - 1) / slots) * ((nb + 4 * sv - 1) / (4 * sv) + 4); };
    if (s_cls >= 1 && s_cls <= (nb + 3) / 4 && kvq::split_classes(B * Hkv, s_cls, res) > 0 && cost(s_cls) <= cost(*S))
      *S = static_cast<int>(s_cls);
  }
  *ex_floats = (n_exact > 0 && !kvq::exact_in_merge(n_exact))
                   ? kvq_kivi_decode_workspace(B, Hq, Hkv, Tq, 128, 0, n_exact, 32, 32, 0) : 0;
  const int64_t R = kvq::pow2_rows((Hq / Hkv) * Tq);
  return *ex_floats + B * Hkv * static_cast<int64_t>(*S) * R * (128 + 2);
}
}  // namespace

extern "C" int64_t kvq_mixed_decode_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d, int64_t nb,
                                              int64_t n_exact) {
  if (d != 128 || B <= 0 || Hkv <= 0 || Hq % Hkv != 0 || Tq <= 0 || nb < 0 || n_exact < 0) return -1;
  int64_t ex;
  int S;
  return mixed_ws_parts(B, Hq, Hkv, Tq, nb, n_exact, &ex, &S);
}

extern "C" int kvq_mixed_decode(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st, int64_t B,
                                int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d, float scaling, const uint8_t* buf,
                                const int64_t* seg, int64_t nb, const void* k_exact, const void* v_exact,
                                int64_t cap_e, int64_t n_exact, const int64_t* exact_pos, const int64_t* q_pos,
                                void* out, float* workspace, int64_t workspace_floats, int phases, void* stream) {
  KVQ_REQUIRE(phases >= 1 && phases <= 3, "kvq_mixed_decode: phases must be 1, 2 or 3");
  KVQ_REQUIRE(d == kMD, "kvq_mixed_decode: head_dim must be 128");
  KVQ_REQUIRE(valid_dtype(q_dtype), "kvq_mixed_decode: bad dtype");
  KVQ_REQUIRE(B > 0 && Hkv > 0 && Hq % Hkv == 0 && Tq > 0, "kvq_mixed_decode: bad head counts");
  const int64_t R_real = (Hq / Hkv) * Tq;
  KVQ_REQUIRE(R_real <= 8, "kvq_mixed_decode: rep*Tq must be <= 8");
  KVQ_REQUIRE(nb >= 0 && nb < 65536, "kvq_mixed_decode: bad block count");
  KVQ_REQUIRE(nb == 0 || (buf && seg), "kvq_mixed_decode: null coded cache");
  KVQ_REQUIRE(nb + n_exact > 0, "kvq_mixed_decode: empty cache");
  KVQ_REQUIRE(q && out && workspace, "kvq_mixed_decode: null q / out / workspace");
  int64_t ex_floats;
  int S;
  const int64_t need = mixed_ws_parts(B, Hq, Hkv, Tq, nb, n_exact, &ex_floats, &S);
  KVQ_REQUIRE(workspace_floats >= need, "kvq_mixed_decode: workspace too small (%lld < %lld floats)",
              (long long)workspace_floats, (long long)need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int R = pow2_rows(R_real);
  MergeArgs ma{};
  ma.Hq = (int)Hq; ma.Hkv = (int)Hkv; ma.Tq = (int)Tq; ma.rep = (int)(Hq / Hkv); ma.R_real = (int)R_real;
  ma.out = out;
  if (exact_in_merge(n_exact)) {
    ma.ex = ExactArgs{q, q_sb, q_sh, q_st, scaling * 1.4426950408889634f, k_exact, v_exact, cap_e,
                      static_cast<int>(n_exact), exact_pos, q_pos};
  } else if (n_exact > 0) {
    if (phases & 1) {
      const int rc = kvq_kivi_decode(q, q_dtype, q_sb, q_sh, q_st, B, Hq, Hkv, Tq, d, scaling, nullptr, nullptr, nullptr,
                                     nullptr, nullptr, 0, 0, 32, 32, k_exact, v_exact, q_dtype, cap_e, n_exact, exact_pos,
                                     q_pos, out, q_dtype, workspace, ex_floats, nullptr, 0, 0.0f, 0, 1, stream);
      if (rc != KVQ_OK) return rc;
    }
    int ex_rows = 0;
    const int64_t S_ex = plan_exact_blocks(B * Hkv, n_exact, &ex_rows);
    const int64_t nrow = B * Hkv * S_ex * R;
    ma.ex_o = workspace;
    ma.ex_m = workspace + nrow * 128;
    ma.ex_l = ma.ex_m + nrow;
    ma.S_ex = (int)S_ex;
  }
  MixedParams p{};
  p.q = q; p.q_sb = q_sb; p.q_sh = q_sh; p.q_st = q_st;
  p.Hq = (int)Hq; p.Hkv = (int)Hkv; p.Tq = (int)Tq; p.rep = (int)(Hq / Hkv); p.R_real = (int)R_real;
  p.BH = (int)(B * Hkv);
  p.qscale = scaling * 1.4426950408889634f;
  p.buf = buf; p.seg = seg; p.n_split = S;
  p.split_classes = KVQ_MIXED_CLASSES != 0 ? split_classes(B * Hkv, S, (pow2_rows(R_real) <= 4 && q_dtype != KVQ_F32) ? 3 : 2) : 0;
  float* tw = workspace + ex_floats;
  const int64_t trow = B * Hkv * static_cast<int64_t>(S) * R;
  p.ws_o = tw;
  p.ws_m = tw + trow * 128;
  p.ws_l = p.ws_m + trow;
  ma.ws_o = p.ws_o; ma.ws_m = p.ws_m; ma.ws_l = p.ws_l; ma.S = S;
  const int bh_pad = (p.BH + 7) / 8 * 8;
  const size_t split_smem = std::max<size_t>((R * kMD + kMWaves * (2 * R * kBqStride + R * 16)) * sizeof(float),
                                             (kMWaves * R * kMD + kMWaves * 2 * R) * sizeof(float));
  if (S > 0 && (phases & 1)) {
#define KVQ_MX_SPLIT(R_, DT_) \
    hipLaunchKernelGGL((mixed_split<R_, DT_>), dim3(static_cast<unsigned>(S) * bh_pad), dim3(kMThreads), split_smem, s, p)
#define KVQ_MX_R(DT_)                                    \
    switch (R) {                                         \
      case 1: KVQ_MX_SPLIT(1, DT_); break;               \
      case 2: KVQ_MX_SPLIT(2, DT_); break;               \
      case 4: KVQ_MX_SPLIT(4, DT_); break;               \
      default: KVQ_MX_SPLIT(8, DT_); break;              \
    }
    switch (q_dtype) {
      case KVQ_F32: KVQ_MX_R(KVQ_F32) break;
      case KVQ_F16: KVQ_MX_R(KVQ_F16) break;
      default: KVQ_MX_R(KVQ_BF16) break;
    }
#undef KVQ_MX_R
#undef KVQ_MX_SPLIT
    KVQ_LAUNCH_CHECK("kvq_mixed_decode(split)");
  }
  if (phases & 2) {
    const int rc = launch_merge_rows(ma, R, p.BH, q_dtype, s);
    if (rc != KVQ_OK) return rc;
  }
  return KVQ_OK;
}
