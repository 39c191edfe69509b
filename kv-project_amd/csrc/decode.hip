// Split-K flash decoding over a packed 4-bit KIVI cache (gfx950, v_mfma_f32_16x16x32_f16).
//
// What it computes (one decode step, one layer): for every (b, KV head h) and every query row
// r of that head (R = rep*Tq rows, GQA order of STRATA_KV.py:527-529), softmax attention over
//   * n_q packed tokens: keys  k[t,c] = code*sc[g,c] + lo[g,c]   (per channel, 64/32-token groups)
//                        values v[t,c] = code*sv[t,gc] + lv[t,gc] (per token, channel groups)
//   * n_exact exact rows (the residual window), read in their storage dtype,
// exactly the attention chunked_attention computes over KIVI token entries (STRATA_KV.py:641-675,
// 801-823) but without ever materialising k or v: scales are folded into the query per key
// group and into the probabilities per token (the affine identity of STRATA_KV.py:1419/1427-1435
// applied per channel / per channel group).
//
// Work decomposition.  Grid (n_exact_wg + n_split, B*Hkv), 256 threads = 4 wavefronts.
//   blockIdx.x <  n_exact_wg : exact rows [512*x, 512*x+512), plain fp32 VALU.
//   blockIdx.x >= n_exact_wg : packed split s, tokens [s*ST, (s+1)*ST), one contiguous quarter
//                              per wavefront; every wavefront streams 32-token chunks.
// Each block writes one flash-decoding partial (m, l, acc) per row (base-2 logits); a second
// kernel merges the partials exactly (log-sum-exp) and writes the output.
//
// Matrix-core mapping of one 32-token chunk (lane l, lane group g = l/16, column n = l%16):
//   QK : two 16x16x32 tiles per chunk, M = 16 tokens, N = 16 columns, K = 128 channels in four
//        k-steps + one "virtual" k-step.  A = key codes: lane l loads the 16 bytes of token
//        l%16 at byte 16g of its packed row (channels 32g..32g+31); word i is k-step i.  B =
//        scaled query: column n holds row n%R, hi part (n/R even) or lo part (n/R odd) of the
//        fp32 value q*scale*sc split into two fp16 (hi + lo = the fp32 value to ~2^-22), so the
//        product keeps fp32-level accuracy on fp16 matrix cores.  Output lane l, register i:
//        token 4g+i of the tile, column n; adding the partner column (row_ror:R) gives the full
//        logit in every lane of row n%R.
//   PV : per 16-channel block one 16x16x32 MFMA, M = 16 channels, N = 16 columns, K = 32
//        tokens.  A = value codes from the tile layout (word = 8 tokens of one channel).  B =
//        p * sv (hi/lo split, one column pair per (row, channel group)); the token "slots"
//        j = 0..7 of lane group g are exactly the tokens the QK output left in that lane
//        (4g+i of tile 0, then of tile 1), so probabilities never leave their lane.
//   Codes become fp16 operands with one and-or each: 0x6400|c is the fp16 value 1024+c, and
//   the high nibble of a byte masked in place is 1024+16c (its operand column is pre-divided by
//   16).  The constant 1024 is cancelled exactly with the sums of the B operands actually used.
#include <algorithm>

#include "common.hpp"

namespace kvq {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kD = 128;            // head_dim supported by the matrix-core path
constexpr int kExactRows = 512;    // exact rows per exact-row block
constexpr int kThreads = 256;
constexpr int kWaves = 4;

// Channel of slot s within an 8-channel k-slice of the packed key row (see header comment).
__device__ __constant__ int kCos[8] = {1, 5, 0, 4, 3, 7, 2, 6};

struct DecodeParams {
  const void* q;
  int64_t q_sb, q_sh, q_st;
  int Hq, Hkv, Tq, rep, R_real;
  float qscale;                       // scaling * log2(e)
  const uint8_t* kc;
  const uint16_t* k_lo;
  const uint16_t* k_sc;
  const uint8_t* vc;
  const uint16_t* vmeta;
  int64_t cap_t;
  int n_q, group_k, group_v, ngv;
  const void* k_exact;
  const void* v_exact;
  int64_t cap_e;
  int n_exact;
  const int64_t* exact_pos;
  const int64_t* q_pos;
  float* ws_m;
  float* ws_l;
  float* ws_o;
  int n_exact_wg, n_split, split_tokens, S1;
  int BH;
  void* out;
};

__device__ __forceinline__ half8 as_half8(u32x4 v) { return __builtin_bit_cast(half8, v); }

// 8 nibbles -> 8 fp16 operands, slot order (nib0, nib4 | 16*nib1, 16*nib5 | nib2, nib6 |
// 16*nib3, 16*nib7), each value offset by 1024.
__device__ __forceinline__ half8 unpack4(uint32_t w) {
  const uint32_t M = 0x64006400u;
  const uint32_t w8 = w >> 8;
  u32x4 r;
  r[0] = (w & 0x000F000Fu) | M;
  r[1] = (w & 0x00F000F0u) | M;
  r[2] = (w8 & 0x000F000Fu) | M;
  r[3] = (w8 & 0x00F000F0u) | M;
  return as_half8(r);
}

__device__ __forceinline__ f32x4 mfma(half8 a, half8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}
constexpr int kRowShr = 0x110;     // row_shr:k  (lane i reads lane i-k of its row of 16)
constexpr int kRowRor = 0x120;     // row_ror:k
constexpr int kQuadSwap1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kQuadSwap2 = 0x4E;   // quad_perm [2,3,0,1]

__device__ __forceinline__ uint32_t pack_h2(_Float16 a, _Float16 b) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, a)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b)) << 16);
}

__device__ __forceinline__ float h2f(uint32_t w, int hi) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(hi ? (w >> 16) : (w & 0xffffu))));
}

__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Row r of KV head h is (query head h*rep + r/Tq, position t = r%Tq).
__device__ __forceinline__ int64_t q_offset(const DecodeParams& p, int b, int h, int r) {
  const int hq = h * p.rep + r / p.Tq;
  const int t = r % p.Tq;
  return static_cast<int64_t>(b) * p.q_sb + static_cast<int64_t>(hq) * p.q_sh +
         static_cast<int64_t>(t) * p.q_st;
}

template <int R, int DT>
__device__ void load_q_rows(const DecodeParams& p, int b, int h, float (*qs)[kD]) {
  for (int idx = threadIdx.x; idx < R * kD; idx += kThreads) {
    const int r = idx / kD, c = idx % kD;
    float v = 0.0f;
    if (r < p.R_real) v = load_as_f32<DT>(p.q, q_offset(p, b, h, r) + c) * p.qscale;
    qs[r][c] = v;
  }
}

// ---------------------------------------------------------------------------------------------
// exact rows: plain fp32 attention over rows [e0, e1) of the residual buffer
template <int R, int DT>
__device__ void exact_block(const DecodeParams& p, int bh, int sidx, float* smem) {
  const int b = bh / p.Hkv, h = bh % p.Hkv;
  float (*qs)[kD] = reinterpret_cast<float (*)[kD]>(smem);
  float* sl = smem + R * kD;                        // logits / probabilities [R][kExactRows]
  float* stat = sl + R * kExactRows;                // m[R], l[R]
  load_q_rows<R, DT>(p, b, h, qs);
  __syncthreads();
  const int e0 = sidx * kExactRows;
  const int ne = min(kExactRows, p.n_exact - e0);
  const int64_t kbase = static_cast<int64_t>(bh) * p.cap_e * kD;
  for (int idx = threadIdx.x; idx < p.R_real * ne; idx += kThreads) {
    const int r = idx / ne, i = idx % ne;
    const int e = e0 + i;
    bool vis = true;
    if (p.exact_pos != nullptr && p.q_pos != nullptr) vis = p.exact_pos[e] <= p.q_pos[r % p.Tq];
    float acc = 0.0f;
    if (vis) {
      const int64_t ro = kbase + static_cast<int64_t>(e) * kD;
#pragma unroll 8
      for (int c = 0; c < kD; ++c) acc += qs[r][c] * load_as_f32<DT>(p.k_exact, ro + c);
    }
    sl[r * kExactRows + i] = vis ? acc : -INFINITY;
  }
  __syncthreads();
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  for (int r = wave; r < p.R_real; r += kWaves) {
    float mx = -INFINITY;
    for (int i = lane; i < ne; i += 64) mx = fmaxf(mx, sl[r * kExactRows + i]);
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    float sum = 0.0f;
    for (int i = lane; i < ne; i += 64) {
      const float s = sl[r * kExactRows + i];
      const float e = (mx == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(s - mx);
      sl[r * kExactRows + i] = e;
      sum += e;
    }
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
    if (lane == 0) {
      stat[r] = mx;
      stat[R + r] = sum;
    }
  }
  __syncthreads();
  const int64_t po = static_cast<int64_t>(bh) * p.S1 + sidx;
  for (int idx = threadIdx.x; idx < p.R_real * kD; idx += kThreads) {
    const int r = idx / kD, c = idx % kD;
    float acc = 0.0f;
    for (int i = 0; i < ne; ++i)
      acc += sl[r * kExactRows + i] * load_as_f32<DT>(p.v_exact, kbase + static_cast<int64_t>(e0 + i) * kD + c);
    p.ws_o[(po * R + r) * kD + c] = acc;
    if (c == 0) {
      p.ws_m[po * R + r] = stat[r];
      p.ws_l[po * R + r] = stat[R + r];
    }
  }
}

// ---------------------------------------------------------------------------------------------
// packed split: 4 wavefronts, each streaming its quarter of the split in 32-token chunks
template <int R, int GV, int DT>
__device__ void packed_block(const DecodeParams& p, int bh, int sidx, float* smem) {
  constexpr int VPB = 16 / R;                       // PV columns per row: (group, hi/lo) variants
  constexpr int GPB = VPB / 2;                      // channel groups per PV B operand
  constexpr int NGV = kD / GV;                      // channel groups of a value row
  constexpr int NB = (NGV + GPB - 1) / GPB;         // PV B operands
  const int b = bh / p.Hkv, h = bh % p.Hkv;
  float (*qs)[kD] = reinterpret_cast<float (*)[kD]>(smem);
  uint32_t* bq_all = reinterpret_cast<uint32_t*>(smem + R * kD);   // [wave][2R][64]
  uint32_t* bv_all = bq_all + kWaves * 2 * R * 64;                  // [wave][R][16]
  load_q_rows<R, DT>(p, b, h, qs);
  __syncthreads();

  const int wave = threadIdx.x / 64;
  const int l = threadIdx.x % 64;
  const int g = l >> 4, n = l & 15;
  const int r_n = n % R;
  const int hl_qk = (n / R) & 1;
  const int v_pv = n / R;
  const int gcl = v_pv >> 1, hl_pv = v_pv & 1;
  // cooperative operand preparation: this lane owns channels c0, c1 (slots 2ck, 2ck+1 of k-step ci)
  const int ci = (l >> 2) & 3, ck = l & 3;
  const int c0 = 32 * g + 8 * ci + kCos[2 * ck];
  const int c1 = 32 * g + 8 * ci + kCos[2 * ck + 1];
  const float kinv = (ck & 1) ? 0.0625f : 1.0f;    // high-nibble slots carry 16*code
  uint32_t* bq = bq_all + wave * 2 * R * 64;
  uint32_t* bv = bv_all + wave * R * 16;

  const int ST = p.split_tokens;
  const int WT = ST / kWaves;
  const int s_begin = (sidx - p.n_exact_wg) * ST;
  const int t0 = s_begin + wave * WT;
  const int t1 = min(t0 + WT, p.n_q);
  const int G = p.group_k;

  const uint8_t* kc = p.kc + static_cast<int64_t>(bh) * p.cap_t * (kD / 2);
  const uint8_t* vc = p.vc + static_cast<int64_t>(bh) * p.cap_t * (kD / 2);
  const uint16_t* vm = p.vmeta + static_cast<int64_t>(bh) * (p.cap_t / 32) * NGV * 64;
  const int64_t kmeta_bh = static_cast<int64_t>(bh) * (p.cap_t / G) * kD;

  f32x4 acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;
  float S[NB], Z[NB];
#pragma unroll
  for (int k = 0; k < NB; ++k) S[k] = Z[k] = 0.0f;

  float qa[R], qb[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    qa[r] = qs[r][c0];
    qb[r] = qs[r][c1];
  }
  const half8 ones = as_half8(u32x4{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u});

  // ---- software pipeline: the loads of chunk cb+32 are in flight while chunk cb computes ----
  struct Chunk {
    u32x4 kw[2], vw[2];
    u32x4 mw[NB][2];
    uint32_t ks, kl;                               // key scale / lo pairs of (c0, c1), group start only
  };
  auto load_chunk = [&](int cb, Chunk& c) {
#pragma unroll
    for (int tau = 0; tau < 2; ++tau)
      c.kw[tau] = *reinterpret_cast<const u32x4*>(kc + static_cast<int64_t>(cb + 16 * tau + n) * (kD / 2) + 16 * g);
    const uint8_t* vchunk = vc + static_cast<int64_t>(cb / 32) * (16 * kD);
#pragma unroll
    for (int qq = 0; qq < 2; ++qq) c.vw[qq] = *reinterpret_cast<const u32x4*>(vchunk + qq * 1024 + l * 16);
#pragma unroll
    for (int bb = 0; bb < NB; ++bb) {
      const int gc = bb * GPB + gcl;
      const uint16_t* src = vm + (static_cast<int64_t>(cb / 32) * NGV + (gc < NGV ? gc : 0)) * 64 + g * 16;
      c.mw[bb][0] = *reinterpret_cast<const u32x4*>(src);
      c.mw[bb][1] = *reinterpret_cast<const u32x4*>(src + 8);
    }
    if ((cb - t0) % G == 0) {
      const int64_t mo = kmeta_bh + static_cast<int64_t>(cb / G) * kD;
      c.ks = static_cast<uint32_t>(p.k_sc[mo + c0]) | (static_cast<uint32_t>(p.k_sc[mo + c1]) << 16);
      c.kl = static_cast<uint32_t>(p.k_lo[mo + c0]) | (static_cast<uint32_t>(p.k_lo[mo + c1]) << 16);
    }
  };

  half8 bqk[4];
  half8 bvirt;
  Chunk cur, nxt;
  if (t0 < t1) load_chunk(t0, nxt);
  for (int cb = t0; cb < t1; cb += 32) {
    cur = nxt;
    if (cb + 32 < t1) load_chunk(cb + 32, nxt);
    if ((cb - t0) % G == 0) {
      // ---- per key group: B operand of the scaled query and the logit correction ----
      const float sc0 = h2f(cur.ks, 0) * kinv, sc1 = h2f(cur.ks, 1) * kinv;
      const float lo0 = h2f(cur.kl, 0), lo1 = h2f(cur.kl, 1);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float x0 = qa[r] * sc0, x1 = qb[r] * sc1;
        const _Float16 h0 = static_cast<_Float16>(x0), h1 = static_cast<_Float16>(x1);
        const _Float16 e0 = static_cast<_Float16>(x0 - static_cast<float>(h0));
        const _Float16 e1 = static_cast<_Float16>(x1 - static_cast<float>(h1));
        bq[(2 * r) * 64 + l] = pack_h2(h0, h1);
        bq[(2 * r + 1) * 64 + l] = pack_h2(e0, e1);
        // bias q.lo minus the 1024 offset carried by every A operand element
        float P = qa[r] * lo0 + qb[r] * lo1 -
                  1024.0f * ((static_cast<float>(h0) + static_cast<float>(h1)) +
                             (static_cast<float>(e0) + static_cast<float>(e1)));
        P += dpp<kQuadSwap1>(P);
        P += dpp<kQuadSwap2>(P);
        if (ck == 0) {
          const _Float16 ph = static_cast<_Float16>(P);
          const _Float16 pl = static_cast<_Float16>(P - static_cast<float>(ph));
          bv[r * 16 + g * 4 + ci] = pack_h2(ph, pl);
        }
      }
      wave_lds_fence();
      const u32x4* src = reinterpret_cast<const u32x4*>(bq + (2 * r_n + hl_qk) * 64 + g * 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) bqk[i] = as_half8(src[i]);
      u32x4 bvr = *reinterpret_cast<const u32x4*>(bv + r_n * 16 + g * 4);
      if (hl_qk) bvr = u32x4{0u, 0u, 0u, 0u};
      bvirt = as_half8(bvr);
      wave_lds_fence();
    }
    // ---- logits ----
    float s[8];
#pragma unroll
    for (int tau = 0; tau < 2; ++tau) {
      f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 4; ++i) d = mfma(unpack4(cur.kw[tau][i]), bqk[i], d);
      d = mfma(ones, bvirt, d);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float full = d[i] + dpp<kRowRor + R>(d[i]);
        const int tok = cb + 16 * tau + 4 * g + i;
        s[4 * tau + i] = tok < t1 ? full : -INFINITY;
      }
    }
    // ---- online softmax (base 2) ----
    float cm = s[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) cm = fmaxf(cm, s[j]);
    cm = fmaxf(cm, __shfl_xor(cm, 16, 64));
    cm = fmaxf(cm, __shfl_xor(cm, 32, 64));
    const float m_new = fmaxf(m_run, cm);
    if (__any(m_new > m_run)) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[k] *= alpha;
      l_run *= alpha;
#pragma unroll
      for (int k = 0; k < NB; ++k) {
        S[k] *= alpha;
        Z[k] *= alpha;
      }
      m_run = m_new;
    }
    float pr[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      pr[j] = __builtin_amdgcn_exp2f(s[j] - m_run);
      l_run += pr[j];
    }
    // ---- PV operands: p * sv, hi/lo split; sums of the operands for the 1024 offset ----
    half8 bp[NB];
#pragma unroll
    for (int bb = 0; bb < NB; ++bb) {
      const int gc = bb * GPB + gcl;
      const bool gvalid = gc < NGV;
      uint32_t words[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        _Float16 hv[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int j = 2 * jj + e;
          const uint32_t mword = cur.mw[bb][j >> 2][j & 3];
          const float sv = h2f(mword, 0), lv = h2f(mword, 1);
          const float kv = ((j & 3) >= 2) ? 0.0625f : 1.0f;
          const float x = gvalid ? pr[j] * sv * kv : 0.0f;
          const _Float16 hx = static_cast<_Float16>(x);
          const _Float16 val = hl_pv ? static_cast<_Float16>(x - static_cast<float>(hx)) : hx;
          hv[e] = val;
          S[bb] += static_cast<float>(val);
          Z[bb] += gvalid ? pr[j] * lv : 0.0f;
        }
        words[jj] = pack_h2(hv[0], hv[1]);
      }
      bp[bb] = as_half8(u32x4{words[0], words[1], words[2], words[3]});
    }
    // ---- PV ----
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
      const int gcb = (16 * blk) / GV;
      acc[blk] = mfma(unpack4(cur.vw[blk >> 2][blk & 3]), bp[gcb / GPB], acc[blk]);
    }
  }

  // ---- wavefront epilogue: row sums over lane groups, hi+lo columns, offset and zero terms ----
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    S[k] += __shfl_xor(S[k], 16, 64);
    S[k] += __shfl_xor(S[k], 32, 64);
    Z[k] += __shfl_xor(Z[k], 16, 64);
    Z[k] += __shfl_xor(Z[k], 32, 64);
    S[k] += dpp<kRowShr + R>(S[k]);            // lo column (v odd) gets its hi partner
  }
  __syncthreads();                               // q rows / operand scratch no longer needed
  float* red_o = smem;                           // [wave][R][kD]
  float* red_ml = smem + kWaves * R * kD;        // [wave][2][R]
#pragma unroll
  for (int blk = 0; blk < 8; ++blk) {
    const int gcb = (16 * blk) / GV;
    const bool mine = hl_pv == 1 && (gcb % GPB) == gcl;
    const float Sb = S[gcb / GPB], Zb = Z[gcb / GPB];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = acc[blk][i] + dpp<kRowShr + R>(acc[blk][i]);
      if (mine) red_o[(wave * R + r_n) * kD + 16 * blk + 4 * g + i] = a - 1024.0f * Sb + Zb;
    }
  }
  if (g == 0 && n < R) {
    red_ml[(wave * 2 + 0) * R + n] = m_run;
    red_ml[(wave * 2 + 1) * R + n] = l_run;
  }
  __syncthreads();
  const int64_t po = static_cast<int64_t>(bh) * p.S1 + sidx;
  for (int idx = threadIdx.x; idx < p.R_real * kD; idx += kThreads) {
    const int r = idx / kD, c = idx % kD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, red_ml[(w * 2) * R + r]);
    float O = 0.0f, L = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float mw_ = red_ml[(w * 2) * R + r];
      const float wgt = (mw_ == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw_ - M);
      O += wgt * red_o[(w * R + r) * kD + c];
      L += wgt * red_ml[(w * 2 + 1) * R + r];
    }
    p.ws_o[(po * R + r) * kD + c] = O;
    if (c == 0) {
      p.ws_m[po * R + r] = M;
      p.ws_l[po * R + r] = L;
    }
  }
}

// exact log-sum-exp merge of the S1 partials of (b, h) and the output write
template <int R, int DT>
__device__ void merge_bh(const DecodeParams& p, int bh, float* smem) {
  const int b = bh / p.Hkv, h = bh % p.Hkv;
  float* wgt = smem;                             // [S1][R]
  float* tot = smem + p.S1 * R;                  // L[R]
  const int64_t pb = static_cast<int64_t>(bh) * p.S1;
  if (threadIdx.x < R) {
    const int r = threadIdx.x;
    float M = -INFINITY;
    for (int s = 0; s < p.S1; ++s) M = fmaxf(M, p.ws_m[(pb + s) * R + r]);
    float L = 0.0f;
    for (int s = 0; s < p.S1; ++s) {
      const float m = p.ws_m[(pb + s) * R + r];
      const float w = (m == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m - M);
      wgt[s * R + r] = w;
      L += w * p.ws_l[(pb + s) * R + r];
    }
    tot[r] = L;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < p.R_real * kD; idx += kThreads) {
    const int r = idx / kD, c = idx % kD;
    float O = 0.0f;
    for (int s = 0; s < p.S1; ++s) O += wgt[s * R + r] * p.ws_o[((pb + s) * R + r) * kD + c];
    const int hq = h * p.rep + r / p.Tq, t = r % p.Tq;
    const int64_t o = ((static_cast<int64_t>(b) * p.Tq + t) * p.Hq + hq) * kD + c;
    store_from_f32<DT>(p.out, o, O / tot[r]);
  }
}

// One block per (b, h, split).  Blocks are dispatched round-robin over the 8 XCDs by linear id,
// so id -> (xcd = id % 8, k = id / 8) -> bh = xcd + 8*(k / S1), split = k % S1 keeps every
// split of one (b, h) on one XCD (its query rows and key metadata are read through one L2).
template <int R, int GV, int DT>
__global__ __launch_bounds__(kThreads) void kivi_decode_split(DecodeParams p) {
  extern __shared__ float smem[];
  const int id = blockIdx.x;
  const int k = id / 8;
  const int bh = id % 8 + 8 * (k / p.S1);
  const int sidx = k % p.S1;
  if (bh >= p.BH) return;
  if (sidx < p.n_exact_wg) exact_block<R, DT>(p, bh, sidx, smem);
  else packed_block<R, GV, DT>(p, bh, sidx, smem);
}

template <int R, int DT>
__global__ __launch_bounds__(kThreads) void kivi_decode_merge(DecodeParams p) {
  extern __shared__ float smem[];
  merge_bh<R, DT>(p, blockIdx.x, smem);
}

template <int R, int GV, int DT>
int launch(DecodeParams& p, int phases, hipStream_t stream) {
  const size_t exact_smem = (R * kD + R * kExactRows + 2 * R) * sizeof(float);
  const size_t packed_smem = std::max<size_t>((R * kD) * sizeof(float) + kWaves * (2 * R * 64 + R * 16) * 4,
                                              (kWaves * R * kD + kWaves * 2 * R) * sizeof(float));
  const size_t msmem = (static_cast<size_t>(p.S1) * R + R) * sizeof(float);
  const size_t smem = std::max({exact_smem, packed_smem, msmem});
  const int bh_pad = (p.BH + 7) / 8 * 8;
  const dim3 grid(static_cast<unsigned>(p.S1) * bh_pad);
  if (phases & 1) {
    hipLaunchKernelGGL((kivi_decode_split<R, GV, DT>), grid, dim3(kThreads), smem, stream, p);
    KVQ_LAUNCH_CHECK("kvq_kivi_decode(split)");
  }
  if (phases & 2) {
    hipLaunchKernelGGL((kivi_decode_merge<R, DT>), dim3(p.BH), dim3(kThreads), msmem, stream, p);
    KVQ_LAUNCH_CHECK("kvq_kivi_decode(merge)");
  }
  return KVQ_OK;
}

inline int pow2_rows(int64_t r) {
  int R = 1;
  while (R < r) R <<= 1;
  return R;
}

struct SplitPlan {
  int n_exact_wg, n_split, split_tokens, S1, R;
};

inline SplitPlan plan_split(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t n_q,
                            int64_t n_exact, int64_t split_tokens, int group_k) {
  SplitPlan sp;
  sp.R = pow2_rows((Hq / Hkv) * Tq);
  const int64_t unit = kWaves * std::max<int64_t>(group_k, 32);
  int64_t st = split_tokens;
  if (st <= 0) {
    const int64_t target = 1024;                         // ~4 blocks per CU on 256 CUs
    const int64_t per = (n_q * B * Hkv + target - 1) / target;
    st = std::max<int64_t>(unit, (per + unit - 1) / unit * unit);
  } else {
    st = (st + unit - 1) / unit * unit;
  }
  sp.split_tokens = static_cast<int>(st);
  sp.n_split = static_cast<int>((n_q + st - 1) / st);
  sp.n_exact_wg = static_cast<int>((n_exact + kExactRows - 1) / kExactRows);
  sp.S1 = sp.n_exact_wg + sp.n_split;
  return sp;
}

}  // namespace
}  // namespace kvq

using namespace kvq;

extern "C" int64_t kvq_kivi_decode_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq,
                                             int64_t d, int64_t n_q, int64_t n_exact,
                                             int group_k, int64_t split_tokens) {
  if (d != kD || B <= 0 || Hkv <= 0 || Hq % Hkv != 0 || Tq <= 0 || group_k <= 0) return -1;
  const SplitPlan sp = plan_split(B, Hq, Hkv, Tq, n_q, n_exact, split_tokens, group_k);
  return B * Hkv * static_cast<int64_t>(sp.S1) * sp.R * (kD + 2);
}

extern "C" int kvq_kivi_decode(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st,
                               int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d,
                               float scaling, const uint8_t* kc, const uint16_t* k_lo,
                               const uint16_t* k_sc, const uint8_t* vc, const uint16_t* vmeta,
                               int64_t cap_t, int64_t n_q, int group_k, int group_v,
                               const void* k_exact, const void* v_exact, int exact_dtype,
                               int64_t cap_e, int64_t n_exact, const int64_t* exact_pos,
                               const int64_t* q_pos, void* out, int out_dtype, float* workspace,
                               int64_t workspace_floats, int64_t split_tokens, int phases,
                               void* stream) {
  KVQ_REQUIRE(phases >= 1 && phases <= 3, "kvq_kivi_decode: phases must be 1, 2 or 3");
  KVQ_REQUIRE(d == kD, "kvq_kivi_decode: head_dim must be 128 (got %lld)", (long long)d);
  KVQ_REQUIRE(valid_dtype(q_dtype) && q_dtype == exact_dtype && q_dtype == out_dtype,
              "kvq_kivi_decode: q, exact rows and output must share one dtype");
  KVQ_REQUIRE(B > 0 && Hkv > 0 && Hq % Hkv == 0 && Tq > 0, "kvq_kivi_decode: bad head counts");
  const int64_t R_real = (Hq / Hkv) * Tq;
  KVQ_REQUIRE(R_real <= 8, "kvq_kivi_decode: rep*Tq must be <= 8 (got %lld)", (long long)R_real);
  KVQ_REQUIRE(group_k % 32 == 0 && group_k > 0, "kvq_kivi_decode: group_k must be a multiple of 32");
  KVQ_REQUIRE(group_v == 32 || group_v == 64 || group_v == 128, "kvq_kivi_decode: group_v in {32,64,128}");
  KVQ_REQUIRE(cap_t % group_k == 0 && cap_t % 32 == 0 && n_q >= 0 && n_q <= cap_t,
              "kvq_kivi_decode: cap_t must be a multiple of group_k and 32, 0 <= n_q <= cap_t");
  KVQ_REQUIRE(n_exact >= 0 && n_exact <= cap_e && n_exact <= 128 * kExactRows,
              "kvq_kivi_decode: bad n_exact");
  KVQ_REQUIRE(n_q + n_exact > 0, "kvq_kivi_decode: empty cache");
  KVQ_REQUIRE(n_q == 0 || (kc && k_lo && k_sc && vc && vmeta), "kvq_kivi_decode: null packed cache");
  KVQ_REQUIRE(n_exact == 0 || (k_exact && v_exact), "kvq_kivi_decode: null exact rows");
  KVQ_REQUIRE(q && out && workspace, "kvq_kivi_decode: null q/out/workspace");
  KVQ_REQUIRE((exact_pos == nullptr) == (q_pos == nullptr), "kvq_kivi_decode: exact_pos and q_pos go together");
  KVQ_REQUIRE(n_q < (1LL << 31) && B * Hkv < 65536, "kvq_kivi_decode: sizes out of range");
  const SplitPlan sp = plan_split(B, Hq, Hkv, Tq, n_q, n_exact, split_tokens, group_k);
  const int64_t need = B * Hkv * static_cast<int64_t>(sp.S1) * sp.R * (kD + 2);
  KVQ_REQUIRE(static_cast<int64_t>(sp.S1) * R_real <= 16384, "kvq_kivi_decode: too many splits");
  KVQ_REQUIRE(workspace_floats >= need, "kvq_kivi_decode: workspace too small (%lld < %lld floats)",
              (long long)workspace_floats, (long long)need);
  DecodeParams p{};
  p.q = q;
  p.q_sb = q_sb; p.q_sh = q_sh; p.q_st = q_st;
  p.Hq = (int)Hq; p.Hkv = (int)Hkv; p.Tq = (int)Tq; p.rep = (int)(Hq / Hkv); p.R_real = (int)R_real;
  p.qscale = scaling * kLog2e;
  p.kc = kc; p.k_lo = k_lo; p.k_sc = k_sc; p.vc = vc; p.vmeta = vmeta;
  p.cap_t = cap_t; p.n_q = (int)n_q; p.group_k = group_k; p.group_v = group_v; p.ngv = (int)(kD / group_v);
  p.k_exact = k_exact; p.v_exact = v_exact; p.cap_e = cap_e; p.n_exact = (int)n_exact;
  p.exact_pos = exact_pos; p.q_pos = q_pos;
  const int64_t nrow = B * Hkv * static_cast<int64_t>(sp.S1) * sp.R;
  p.ws_o = workspace;
  p.ws_m = workspace + nrow * kD;
  p.ws_l = p.ws_m + nrow;
  p.BH = static_cast<int>(B * Hkv);
  p.n_exact_wg = sp.n_exact_wg; p.n_split = sp.n_split; p.split_tokens = sp.split_tokens; p.S1 = sp.S1;
  p.out = out;
  hipStream_t s = static_cast<hipStream_t>(stream);
#define KVQ_GV(R_, DT_)                                                             \
  switch (group_v) {                                                                \
    case 32: return launch<R_, 32, DT_>(p, phases, s);                             \
    case 64: return launch<R_, 64, DT_>(p, phases, s);                             \
    default: return launch<R_, 128, DT_>(p, phases, s);                            \
  }
#define KVQ_R(DT_)                                                                  \
  switch (sp.R) {                                                                   \
    case 1: KVQ_GV(1, DT_)                                                          \
    case 2: KVQ_GV(2, DT_)                                                          \
    case 4: KVQ_GV(4, DT_)                                                          \
    default: KVQ_GV(8, DT_)                                                         \
  }
  switch (q_dtype) {
    case KVQ_F32: KVQ_R(KVQ_F32)
    case KVQ_F16: KVQ_R(KVQ_F16)
    default: KVQ_R(KVQ_BF16)
  }
#undef KVQ_R
#undef KVQ_GV
}
