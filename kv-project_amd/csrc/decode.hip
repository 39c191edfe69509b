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
// Work decomposition.  One launch of 256-thread blocks (4 wavefronts), XCD-aware over (b, h):
//   packed split s of (b, h): a contiguous share of the tokens (equal, or weighted by the
//                             block's dispatch class when the plan is one full round), one
//                             contiguous quarter of it per wavefront; every wavefront streams
//                             32-token chunks.
//   exact window: with a one-round class plan, exact-row blocks of the same launch dispatched
//                 after the packed blocks (they run on the slots the first class leaves free);
//                 otherwise up to kFusedExact rows per packed split are attended by the packed
//                 blocks themselves (fp32 VALU, staged in LDS with the query rows, after the
//                 stream), longer windows of up to kExactInMerge rows by the merge, longer still
//                 by exact-row blocks (streaming, about one round of them) of a launch of their
//                 own after the packed blocks.
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
//   Codes become fp16 operands with one and each: a nibble masked in place is the fp16 subnormal
//   c*2^-24 (low nibble) or 16c*2^-24 (high nibble, its operand column pre-divided by 16); the
//   matrix core keeps subnormal inputs, so codes enter exactly and no offset has to be cancelled.
#include <atomic>
#include <mutex>
#include <algorithm>

#include "common.hpp"
#include "mfma_common.hpp"
#include "partials.hpp"

namespace kvq {
namespace {


// Build-time switches of the split kernel (defaults are the tuned values):
//   KVQ_WAVES       waves per SIMD the register allocation targets (0: per-variant default)
//   KVQ_SCORE_SPLITS splits of the score pass per split of the decode (its registers allow more
//                   resident blocks)
//   KVQ_LOAD_AUX    cache-policy bits of the streaming code/metadata loads (gfx950: 1 = sc0,
//                   2 = nt, 16 = sc1).  Default nt: every code byte is read once per launch, so
//                   marking it non-temporal keeps it from displacing reused lines (measured ~4%
//                   faster on the 16x32x32768 workload than the default policy)
#ifndef KVQ_WAVES
#define KVQ_WAVES 0
#endif
#ifndef KVQ_SCORE_SPLITS
#define KVQ_SCORE_SPLITS 2
#endif
#ifndef KVQ_LOAD_AUX
#define KVQ_LOAD_AUX 2
#endif
//   KVQ_CLASSES     1: plans that are one full round of packed blocks map them class-major and
//                   size the splits by dispatch class (see class_weight)
#ifndef KVQ_CLASSES
#define KVQ_CLASSES 1
#endif

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kD = 128;            // head_dim supported by the matrix-core path
// A window of at most kFusedExact rows per packed split is attended by the packed blocks
// themselves: each stages its share in LDS together with the query rows and folds it into its
// partial as one more wavefront state, so the window adds neither blocks nor merge work.
constexpr int kFusedExact = 32;
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
  float* row_ml;                      // per (b, h, row): global max (log2 units) and sum of exp2
  float* scores;                      // score pass: (BH, scores_bh) accumulated probabilities
  int64_t scores_bh;
  float score_weight;
  float* spill;                       // scored step: the split's logits (BH, spill_bh), or null
  int64_t spill_bh;
  float* ws_o;
  int n_exact_wg, n_split, split_tokens, S1;
  int split_classes;                  // > 0: class-major split mapping and class-weighted splits
  int exact_inline;                   // exact-row blocks dispatched after the packed blocks of the split
  int fused_per;                      // exact rows each packed split attends itself (0: none)
  int exact_rows;                     // rows of each exact-row block
  int BH;
  void* out;
  int ex_po0;                         // partial index of exact-row block 0 (after the retained-row blocks)
  const int32_t* ret_idx;             // retained decode: (BH, ret_bh) positions into the packed rows
  int64_t ret_bh;
  int n_ret;                          // retained positions per (b, h)
  int ret_wg;                         // retained-row blocks per (b, h)
};

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
// exact rows: fp32 attention over rows [e0, e1) of the residual buffer (e0 = sidx * exact_rows)

constexpr float kRowLazy = 4.0f;

// One row of a lane group (16 lanes, 8 channels each) into the group's base-2 online softmax of
// every query row r whose bit is set in `vis`: the logit's 16-lane sum, a lazy maximum (rescaled
// only when a logit exceeds it by more than kRowLazy), the probability-weighted values.
template <int R>
__device__ __forceinline__ void attend_row(const float (&qv)[R][8], const float (&kx)[8], const float (&vx)[8],
                                           uint32_t vis, float (&m)[R], float (&l)[R], float (&o)[R][8]) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) s = __builtin_fmaf(qv[r][k], kx[k], s);
    s = row_sum16(s);
    if (!((vis >> r) & 1u)) s = -INFINITY;
    if (s > m[r] + kRowLazy) {                       // m[r] = -inf: first visible row
      const float a = __builtin_amdgcn_exp2f(m[r] - s);
      l[r] *= a;
#pragma unroll
      for (int k = 0; k < 8; ++k) o[r][k] *= a;
      m[r] = s;
    }
    const float pr = s == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s - m[r]);
    l[r] += pr;
#pragma unroll
    for (int k = 0; k < 8; ++k) o[r][k] = __builtin_fmaf(pr, vx[k], o[r][k]);
  }
}

// The 16 lane-group states of a block meet (shuffles within a wavefront, then the wavefronts in
// LDS) and the block's partial (m, l, o) of each real query row is written at partial index po.
template <int R>
__device__ __forceinline__ void rows_epilogue(const DecodeParams& p, int64_t po, float (&m)[R], float (&l)[R],
                                              float (&o)[R][8], float* red_o, float* red_ml, int wave, int lane,
                                              int j, int part) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float M = m[r];
    M = xmax32(xmax16(M));
    const float w = m[r] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m[r] - M);
    float L = l[r] * w;
    L = xsum32(xsum16(L));
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      float t = o[r][k] * w;
      t = xsum32(xsum16(t));
      if (j == 0) red_o[(wave * R + r) * kD + 8 * part + k] = t;
    }
    if (lane == 0) {
      red_ml[(wave * 2) * R + r] = M;
      red_ml[(wave * 2 + 1) * R + r] = L;
    }
  }
  __syncthreads();
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

// Partial (m, l, o) of exact-row block `sidx`.  Each wavefront streams a contiguous quarter of the
// block's rows, four at a time: lane group j = lane / 16 takes one row, 8 channels per lane
// (coalesced 16-byte loads, kept raw until used), the loads of the next three row quads in flight
// while one is computed.  Every lane group keeps its own base-2 online softmax per query row; the
// 16 states of the block are merged at the end.  The partial goes to index ex_po0 + sidx of the
// (b, h)'s S1 partials.
template <int R, int DT>
__device__ void exact_block(const DecodeParams& p, int bh, int sidx, float* smem) {
  const int b = bh / p.Hkv, h = bh % p.Hkv;
  float (*qs)[kD] = reinterpret_cast<float (*)[kD]>(smem);
  float* red_o = smem + R * kD;                     // [wave][R][kD]
  float* red_ml = red_o + kWaves * R * kD;          // [wave][2][R]
  const int e0 = sidx * p.exact_rows;
  const int e1 = min(e0 + p.exact_rows, p.n_exact);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
  const int j = lane >> 4, part = lane & 15;       // row slot of 4, 8-channel slice of 16
  const int w0 = e0 + (e1 - e0) * wave / kWaves, w1 = e0 + (e1 - e0) * (wave + 1) / kWaves;
  const int64_t kbase = static_cast<int64_t>(bh) * p.cap_e * kD;
  const bool masked = p.exact_pos != nullptr && p.q_pos != nullptr;
  float qv[R][8];                                   // scaled query rows (set once they are staged)
  int64_t qp[R];
  float m[R], l[R], o[R][8];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) o[r][k] = 0.0f;
  }
  constexpr int kW = DT == KVQ_F32 ? 2 : 1;          // 16-byte words of 8 channels
  struct Rows {
    u32x4 kw[kW], vw[kW];
    int64_t pos;
  };
  // loads of row i (clamped to the wavefront's last row, so every load is unconditional)
  auto load_rows = [&](int i, Rows& x) {
    i = min(i, w1 - 1);
    const int64_t off = (kbase + static_cast<int64_t>(i) * kD + 8 * part) * (DT == KVQ_F32 ? 4 : 2);
    const u32x4* kp = reinterpret_cast<const u32x4*>(static_cast<const uint8_t*>(p.k_exact) + off);
    const u32x4* vp = reinterpret_cast<const u32x4*>(static_cast<const uint8_t*>(p.v_exact) + off);
#pragma unroll
    for (int w = 0; w < kW; ++w) {            // streamed once: non-temporal
      x.kw[w] = __builtin_nontemporal_load(kp + w);
      x.vw[w] = __builtin_nontemporal_load(vp + w);
    }
    x.pos = masked ? p.exact_pos[i] : 0;
  };
  auto to_f32 = [&](const u32x4 (&w)[kW], float (&x)[8]) {
    if constexpr (DT == KVQ_F32) {
#pragma unroll
      for (int k = 0; k < 8; ++k) x[k] = __uint_as_float(w[k / 4][k % 4]);
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint16_t lo = static_cast<uint16_t>(w[0][k] & 0xffffu), hi = static_cast<uint16_t>(w[0][k] >> 16);
        x[2 * k] = DT == KVQ_F16 ? f16_to_f32(lo) : bf16_to_f32(lo);
        x[2 * k + 1] = DT == KVQ_F16 ? f16_to_f32(hi) : bf16_to_f32(hi);
      }
    }
  };
  auto attend = [&](int i, const Rows& x) {
    float kx[8], vx[8];
    to_f32(x.kw, kx);
    to_f32(x.vw, vx);
    uint32_t vis = 0u;
#pragma unroll
    for (int r = 0; r < R; ++r) vis |= (i < w1 && !(masked && x.pos > qp[r])) ? (1u << r) : 0u;
    attend_row<R>(qv, kx, vx, vis, m, l, o);
  };
  // the first four row quads of the wavefront go out before the query rows are staged, so the
  // block waits for one round of loads, not two
  Rows x0, x1, x2, x3;
  if (w0 < w1) {
    load_rows(w0 + j, x0);
    load_rows(w0 + 4 + j, x1);
    load_rows(w0 + 8 + j, x2);
    load_rows(w0 + 12 + j, x3);
  }
  load_q_rows<R, DT>(p, b, h, qs);
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int k = 0; k < 8; ++k) qv[r][k] = qs[r][8 * part + k];
#pragma unroll
  for (int r = 0; r < R; ++r) qp[r] = masked ? p.q_pos[r % p.Tq] : 0;
  if (w0 < w1) {
    for (int i0 = w0;; i0 += 16) {
      if (i0 != w0) load_rows(i0 + 12 + j, x3);
      attend(i0 + j, x0);
      if (i0 + 4 >= w1) break;
      load_rows(i0 + 16 + j, x0);
      attend(i0 + 4 + j, x1);
      if (i0 + 8 >= w1) break;
      load_rows(i0 + 20 + j, x1);
      attend(i0 + 8 + j, x2);
      if (i0 + 12 >= w1) break;
      load_rows(i0 + 24 + j, x2);
      attend(i0 + 12 + j, x3);
      if (i0 + 16 >= w1) break;
    }
  }
  rows_epilogue<R>(p, static_cast<int64_t>(bh) * p.S1 + p.ex_po0 + sidx, m, l, o, red_o, red_ml, wave, lane, j,
                   part);
}

// Partial of retained-row block `sidx`: rows [sidx * exact_rows, ...) of the (b, h)'s retained
// positions ret_idx, read straight from the packed cache and dequantised in registers exactly as
// kivi_quant's xhat (code * scale + lo in fp32: two roundings, STRATA_KV.py:855) -- the eviction
// path's decode over the kept tokens without writing them out first.  Lane group j takes a token,
// lane `part` its channels 8 part .. 8 part + 7: the key codes' 4 bytes of the token's pack_codes
// row, the 16 bytes of key scale and zero of those channels in the token's key group, the token's
// 8 words of the value tile (one per channel: 8 tokens of a channel each) and its (scale, lo) word
// of the channel group.  A position outside [0, n_q) counts as a masked row (its loads read
// position 0).  The wavefront's indices are loaded first; each row quad's loads depend on them
// only.
__device__ __constant__ int kNibbleOfSlotD[8] = {0, 4, 1, 5, 2, 6, 3, 7};

template <int R, int DT>
__device__ void retained_block(const DecodeParams& p, int bh, int sidx, float* smem) {
  const int b = bh / p.Hkv, h = bh % p.Hkv;
  float (*qs)[kD] = reinterpret_cast<float (*)[kD]>(smem);
  float* red_o = smem + R * kD;
  float* red_ml = red_o + kWaves * R * kD;
  const int e0 = sidx * p.exact_rows;
  const int e1 = min(e0 + p.exact_rows, p.n_ret);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
  const int j = lane >> 4, part = lane & 15;
  const int w0 = e0 + (e1 - e0) * wave / kWaves, w1 = e0 + (e1 - e0) * (wave + 1) / kWaves;
  const int G = p.group_k;
  const int ngv = kD / p.group_v;
  const int32_t* ridx = p.ret_idx + static_cast<int64_t>(bh) * p.ret_bh;
  const uint8_t* kc = p.kc + static_cast<int64_t>(bh) * p.cap_t * (kD / 2);
  const uint16_t* ksc = p.k_sc + static_cast<int64_t>(bh) * (p.cap_t / G) * kD;
  const uint16_t* klo = p.k_lo + static_cast<int64_t>(bh) * (p.cap_t / G) * kD;
  const uint8_t* vc = p.vc + static_cast<int64_t>(bh) * p.cap_t * (kD / 2);
  const uint16_t* vm = p.vmeta + static_cast<int64_t>(bh) * (p.cap_t / 32) * ngv * 64;
  float qv[R][8];
  float m[R], l[R], o[R][8];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) o[r][k] = 0.0f;
  }
  struct Tok {
    uint32_t kw, vw[8], vmw;
    uint4 sc4, lo4;
    int t;                                       // the position, or -1 for a masked row
  };
  // the positions of this wavefront's rows, lane group j holding rows w0 + j + 4 u
  constexpr int kMaxU = 16;                      // rows per lane group held in registers (64 per wavefront)
  auto pos_of = [&](int i) -> int {
    if (i >= w1) return -1;
    const int t = ridx[i];
    return (t >= 0 && t < p.n_q) ? t : -1;
  };
  auto load_tok = [&](int t, Tok& x) {
    x.t = t;
    const int tt = t < 0 ? 0 : t;
    x.kw = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(kc + static_cast<int64_t>(tt) * (kD / 2) + 4 * part));
    const int64_t km = static_cast<int64_t>(tt / G) * kD + 8 * part;
    x.sc4 = *reinterpret_cast<const uint4*>(ksc + km);
    x.lo4 = *reinterpret_cast<const uint4*>(klo + km);
    const int chunk = tt / 32, u = tt % 32;
    const int g = (u % 16) / 4, jj = 4 * (u / 16) + (u % 4);
    const int blk = part / 2;
    const uint32_t* tile = reinterpret_cast<const uint32_t*>(vc + static_cast<int64_t>(chunk) * 16 * kD) +
                           (blk / 4) * 256 + (16 * g + 8 * (part % 2)) * 4 + (blk % 4);
#pragma unroll
    for (int e = 0; e < 8; ++e) x.vw[e] = tile[4 * e];
    x.vmw = *reinterpret_cast<const uint32_t*>(vm + ((static_cast<int64_t>(chunk) * ngv + (8 * part) / p.group_v) * 64 +
                                                      (8 * g + jj) * 2));
  };
  auto attend = [&](const Tok& x) {
    float kx[8], vx[8];
    const uint32_t scw[4] = {x.sc4.x, x.sc4.y, x.sc4.z, x.sc4.w}, low[4] = {x.lo4.x, x.lo4.y, x.lo4.z, x.lo4.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t byte = (x.kw >> (8 * (k / 2))) & 0xffu;
      const int code = (k & 1) ? static_cast<int>(byte & 15u) : static_cast<int>(byte >> 4);
      const float sc = f16_to_f32(static_cast<uint16_t>(scw[k / 2] >> (16 * (k & 1))));
      const float lo = f16_to_f32(static_cast<uint16_t>(low[k / 2] >> (16 * (k & 1))));
      kx[k] = __fadd_rn(__fmul_rn(static_cast<float>(code), sc), lo);
    }
    const int u = (x.t < 0 ? 0 : x.t) % 32;
    const int jj = 4 * (u / 16) + (u % 4);
    const int shift = 4 * kNibbleOfSlotD[jj];
    const float sv = f16_to_f32(static_cast<uint16_t>(x.vmw & 0xffffu));
    const float lv = f16_to_f32(static_cast<uint16_t>(x.vmw >> 16));
#pragma unroll
    for (int e = 0; e < 8; ++e) vx[e] = __fadd_rn(__fmul_rn(static_cast<float>((x.vw[e] >> shift) & 15u), sv), lv);
    attend_row<R>(qv, kx, vx, x.t >= 0 ? 0xffffffffu : 0u, m, l, o);
  };
  const int n_u = w0 < w1 ? (w1 - w0 + 3) / 4 : 0;     // row quads of the wavefront
  int tpos[kMaxU];
#pragma unroll
  for (int u = 0; u < kMaxU; ++u) tpos[u] = u < n_u ? pos_of(w0 + 4 * u + j) : -1;
  Tok x0, x1;
  if (n_u > 0) load_tok(tpos[0], x0);
  load_q_rows<R, DT>(p, b, h, qs);
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int k = 0; k < 8; ++k) qv[r][k] = qs[r][8 * part + k];
#pragma unroll
  for (int u = 0; u < kMaxU; u += 2) {
    if (u >= n_u) break;
    if (u + 1 < n_u) load_tok(tpos[u + 1], x1);
    attend(x0);
    if (u + 1 >= n_u) break;
    if (u + 2 < n_u) load_tok(tpos[u + 2], x0);
    attend(x1);
  }
  rows_epilogue<R>(p, static_cast<int64_t>(bh) * p.S1 + sidx, m, l, o, red_o, red_ml, wave, lane, j, part);
}

// ---------------------------------------------------------------------------------------------
// packed split: 4 wavefronts, each streaming its quarter of the split in 32-token chunks
// MODE 0: flash-decoding partials of this split.  MODE 1: the score pass of the eviction path --
// the same logits, normalised by the row's global (max, sum) from the merge, summed over the rows
// of the KV head and accumulated into the scores row (no value work).  MODE 2: the partials, and
// every logit of the split spilled (chunk-local layout, see spill_index) for score_from_logits,
// which then needs neither the keys nor their metadata again.
// LDS of a packed block (floats): query rows + per-wavefront operand scratch, reused by the
// wavefront partials of the epilogue; the fused exact-row region follows it.
template <int R>
constexpr int packed_lds_floats() {
  constexpr int loop = R * kD + kWaves * (2 * R * kBqStride + R * 16);
  constexpr int epi = kWaves * R * kD + kWaves * 2 * R;
  return loop > epi ? loop : epi;
}
template <int R, int DT>
constexpr int fused_lds_floats() {
  constexpr int esz = DT == KVQ_F32 ? 4 : 2;
  static_assert(R * kD <= kFusedExact * kD * esz / 4, "value sums must fit over the staged keys");
  return 2 * kFusedExact * kD * esz / 4 + R * kFusedExact + R + 2 * R;   // keys, values, logits, masks, stats
}

// Dispatch-class weights of the packed split (see class_block_of): fitted on the 8B-shape layer
// from the classes' measured stream times (the youngest class still finishes last, since it
// issues only when the older ones wait)
#ifndef KVQ_CLASS_W
#define KVQ_CLASS_W 141, 98, 68
#endif
constexpr int kClassW[3] = {KVQ_CLASS_W};
constexpr int kClassW0 = kClassW[0], kClassW1 = kClassW[1], kClassW2 = kClassW[2];
__device__ __forceinline__ int64_t split_weight_before(const DecodeParams& p, int s) {
  return class_weight_before(s, p.n_split, p.split_classes, kClassW0, kClassW1, kClassW2);
}
__device__ __forceinline__ void packed_block_of(const DecodeParams& p, int id, int n_split, int* bh, int* sidx) {
  class_block_of(id, n_split, p.split_classes, bh, sidx);
}

template <int R, int GV, int DT, int MODE>
__device__ void packed_block(const DecodeParams& p, int bh, int sidx, float* smem) {
  // fp32 output: p * sv enters the PV product as hi + lo fp16 parts (two column variants per
  // group); 16-bit outputs take the single fp16 rounding (relative error 2^-12 per term, far
  // below the output's own rounding), one column per group
  constexpr bool LO = DT == KVQ_F32;
  constexpr int VPB = 16 / R;                       // PV columns per row: (group[, hi/lo]) variants
  constexpr int GPB = LO ? VPB / 2 : VPB;           // channel groups per PV B operand
  constexpr int NGV = kD / GV;                      // channel groups of a value row
  constexpr int NB = (NGV + GPB - 1) / GPB;         // PV B operands
  const int b = bh / p.Hkv, h = bh % p.Hkv;
  float (*qs)[kD] = reinterpret_cast<float (*)[kD]>(smem);
  uint32_t* bq_all = reinterpret_cast<uint32_t*>(smem + R * kD);   // [wave][2R][64]
  uint32_t* bv_all = bq_all + kWaves * 2 * R * kBqStride;                  // [wave][R][16]

  // fused exact rows [fe0, fe0 + fne) of the window: raw rows staged in LDS (their loads are in
  // flight together with the query rows'), visibility of row i to query row r in bit i of emask[r]
  constexpr int kEsz = DT == KVQ_F32 ? 4 : 2;
  constexpr int kRowU4 = kD * kEsz / 16;                       // 16-byte words of one row
  constexpr int kExU4 = kFusedExact * kRowU4 / kThreads;       // words per thread and tensor
  static_assert(kFusedExact * kRowU4 % kThreads == 0, "fused rows must spread evenly");
  u32x4* const ek4 = reinterpret_cast<u32x4*>(smem + packed_lds_floats<R>());
  u32x4* const ev4 = ek4 + kFusedExact * kRowU4;
  float* const esl = reinterpret_cast<float*>(ev4 + kFusedExact * kRowU4);   // [R][kFusedExact]
  uint32_t* const emask = reinterpret_cast<uint32_t*>(esl + R * kFusedExact);
  float* const estat = reinterpret_cast<float*>(emask + R);                   // row max [R], sum [R]
  float* const eo = reinterpret_cast<float*>(ek4);                            // [R][kD] value sums
  int fe0 = 0, fne = 0;
  constexpr bool SCORE = MODE == 1;
  if constexpr (!SCORE) {
    if (p.fused_per > 0) {
      fe0 = min(sidx * p.fused_per, p.n_exact);
      fne = min(p.fused_per, p.n_exact - fe0);
    }
  }

  // wave index made explicitly uniform: every token offset derived from it lives in SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const int l = threadIdx.x % 64;
  const int g = l >> 4, n = l & 15;
  const int r_n = n % R;
  const int hl_qk = (n / R) & 1;
  const int v_pv = n / R;
  const int gcl = LO ? (v_pv >> 1) : v_pv, hl_pv = LO ? (v_pv & 1) : 0;
  // cooperative operand preparation: this lane owns channels c0, c1 (slots 2ck, 2ck+1 of k-step ci)
  const int ci = (l >> 2) & 3, ck = l & 3;
  const int c0 = 32 * g + 8 * ci + kCos[2 * ck];
  const int c1 = 32 * g + 8 * ci + kCos[2 * ck + 1];
  // key slots of high nibbles carry 16*code: their query operand is q*scale, the low-nibble
  // slots' is 16*q*scale, so every product is 16 * code * q*scale * 2^-24 and the fp16 low part
  // of the operand stays out of the subnormal range
  const float kinv = (ck & 1) ? 1.0f : 16.0f;
  uint32_t* bq = bq_all + wave * 2 * R * kBqStride;
  uint32_t* bv = bv_all + wave * R * 16;

  // wavefront `wave` of split sidx takes a quarter of the split's share of the NC 32-token chunks
  // (a range may start inside a key group)
  const int G = p.group_k;
  const int NC = (p.n_q + 31) / 32;
  const int64_t cwt = split_weight_before(p, p.n_split);
  const int64_t sc0 = NC * split_weight_before(p, sidx) / cwt;       // the split's chunks [sc0, sc1)
  const int64_t sc1 = NC * split_weight_before(p, sidx + 1) / cwt;
  const int t0 = 32 * static_cast<int>(sc0 + (sc1 - sc0) * wave / kWaves);
  const int t1 = min(32 * static_cast<int>(sc0 + (sc1 - sc0) * (wave + 1) / kWaves), p.n_q);
  // start of this wavefront's last chunk: loads past it are clamped onto it (they then hit in
  // cache), so every load of the pipeline is unconditional and the wait before each chunk's
  // compute counts exactly the loads issued after that chunk's
  const int t_last = t0 < t1 ? t0 + ((t1 - 1 - t0) & ~31) : t0;

  // buffer resources over this (b, h)'s slices; chunk advance goes in the scalar offset
  const uint32_t code_bytes = static_cast<uint32_t>(p.cap_t) * (kD / 2);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(p.kc + static_cast<int64_t>(bh) * p.cap_t * (kD / 2), code_bytes);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.vc + static_cast<int64_t>(bh) * p.cap_t * (kD / 2), code_bytes);
  const uint32_t vm_bytes = static_cast<uint32_t>(p.cap_t / 32) * NGV * 128;
  const __amdgpu_buffer_rsrc_t rm =
      make_rsrc(p.vmeta + static_cast<int64_t>(bh) * (p.cap_t / 32) * NGV * 64, vm_bytes);
  const uint32_t km_bytes = static_cast<uint32_t>(p.cap_t / G) * kD * 2;
  const __amdgpu_buffer_rsrc_t rks = make_rsrc(p.k_sc + static_cast<int64_t>(bh) * (p.cap_t / G) * kD, km_bytes);
  const __amdgpu_buffer_rsrc_t rkl = make_rsrc(p.k_lo + static_cast<int64_t>(bh) * (p.cap_t / G) * kD, km_bytes);
  const int vo_k = n * (kD / 2) + 16 * g;           // token n of a 16-token tile, channels 32g..32g+31
  const int vo_v = l * 16;
  int vo_m[NB];
#pragma unroll
  for (int bb = 0; bb < NB; ++bb) {
    const int gc = bb * GPB + gcl;
    vo_m[bb] = ((gc < NGV ? gc : 0) * 64 + g * 16) * 2;
  }

  // A nibble masked in place is an fp16 subnormal: c * 2^-24 (low nibble) or 16c * 2^-24 (high
  // nibble), exact, so every code becomes a matrix-core operand with one and.  Key products carry
  // the common factor 2^-20 (see kinv), removed once from the logits; value products carry 2^-24,
  // removed once from the value sums.
  auto unpack = [&](uint32_t w) -> half8 {
    const uint32_t w8 = w >> 8;
    u32x4 r;
    r[0] = w & 0x000F000Fu;
    r[1] = w & 0x00F000F0u;
    r[2] = w8 & 0x000F000Fu;
    r[3] = w8 & 0x00F000F0u;
    return as_half8(r);
  };
  constexpr float kTwo24 = 16777216.0f;
  constexpr float kTwo20 = 1048576.0f;              // logit = 2^20 * matrix-core sum
  constexpr float kLazy = 4.0f;

  // one 32-token chunk of this wavefront: key rows, value tile, value metadata, and the key
  // scale / zero of channels (c0, c1) of the chunk's key group (used when the chunk starts one)
  struct Chunk {
    u32x4 kw[2], vw[2];
    u32x4 mw[NB][2];
    uint32_t ks0, ks1, kl0, kl1;
    uint32_t sc;                                     // score pass: the token's score so far
  };
  // score pass: token of this lane's score slot (lane n < 8 of lane group g carries slot n) and
  // a buffer over the (b, h) scores row (reads past n_q are zero)
  const int sc_tok = 16 * ((n & 7) >> 2) + 4 * g + (n & 3);
  const __amdgpu_buffer_rsrc_t rsc = make_rsrc(SCORE ? p.scores + static_cast<int64_t>(bh) * p.scores_bh : p.ws_o,
                                               SCORE ? static_cast<uint32_t>(p.n_q) * 4u : 0u);
  auto load_chunk = [&](int cb, Chunk& c) {
    cb = min(cb, t_last);
    // scalar offsets: uniform by construction (readfirstlane keeps them out of waterfall loops)
    const int so = __builtin_amdgcn_readfirstlane(cb * (kD / 2));   // key rows and value tiles alike
    c.kw[0] = __builtin_amdgcn_raw_buffer_load_b128(rk, vo_k, so, KVQ_LOAD_AUX);
    c.kw[1] = __builtin_amdgcn_raw_buffer_load_b128(rk, vo_k + 16 * (kD / 2), so, KVQ_LOAD_AUX);
    if constexpr (!SCORE) {
      c.vw[0] = __builtin_amdgcn_raw_buffer_load_b128(rv, vo_v, so, KVQ_LOAD_AUX);
      c.vw[1] = __builtin_amdgcn_raw_buffer_load_b128(rv, vo_v + 1024, so, KVQ_LOAD_AUX);
      const int som = __builtin_amdgcn_readfirstlane((cb / 32) * NGV * 128);
#pragma unroll
      for (int bb = 0; bb < NB; ++bb) {
        c.mw[bb][0] = __builtin_amdgcn_raw_buffer_load_b128(rm, vo_m[bb], som, KVQ_LOAD_AUX);
        c.mw[bb][1] = __builtin_amdgcn_raw_buffer_load_b128(rm, vo_m[bb] + 16, som, KVQ_LOAD_AUX);
      }
    }
    const int sok = __builtin_amdgcn_readfirstlane((cb / G) * kD * 2);
    c.ks0 = __builtin_amdgcn_raw_buffer_load_b16(rks, c0 * 2, sok, 0);
    c.ks1 = __builtin_amdgcn_raw_buffer_load_b16(rks, c1 * 2, sok, 0);
    c.kl0 = __builtin_amdgcn_raw_buffer_load_b16(rkl, c0 * 2, sok, 0);
    c.kl1 = __builtin_amdgcn_raw_buffer_load_b16(rkl, c1 * 2, sok, 0);
    if constexpr (SCORE) c.sc = __builtin_amdgcn_raw_buffer_load_b32(rsc, (cb + sc_tok) * 4, 0, 0);
  };

  f32x4 acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
  // probability sums and zero-point sums, split by slot scale: slots 2,3,6,7 hold p/16
  float m_run = -INFINITY, la = 0.0f, lb = 0.0f;
  float Za[NB], Zb[NB];
#pragma unroll
  for (int k = 0; k < NB; ++k) Za[k] = Zb[k] = 0.0f;
  const half8 tiny = as_half8(u32x4{0x00100010u, 0x00100010u, 0x00100010u, 0x00100010u});   // 2^-20
  const half2v hl_neg = hl_pv ? half2v{static_cast<_Float16>(-1.0f), static_cast<_Float16>(-1.0f)}
                              : half2v{static_cast<_Float16>(0.0f), static_cast<_Float16>(0.0f)};
  const u32x4* bq_src = reinterpret_cast<const u32x4*>(bq + (2 * r_n + hl_qk) * kBqStride + g * 16);
  const u32x4* bv_src = reinterpret_cast<const u32x4*>(bv + r_n * 16 + g * 4);
  half8 bqk[4];                                      // query operand of the current key group
  half8 bvirt;
  // score pass: this lane's row statistics (padded rows contribute nothing)
  float score_m = 0.0f, score_il = 0.0f;
  float* score_row = nullptr;
  if constexpr (SCORE) {
    const int64_t ri = (static_cast<int64_t>(bh) * R + r_n) * 2;
    score_m = r_n < p.R_real ? p.row_ml[ri] : 0.0f;
    score_il = r_n < p.R_real ? 1.0f / p.row_ml[ri + 1] : 0.0f;
    score_row = p.scores + static_cast<int64_t>(bh) * p.scores_bh;
  }

  auto step = [&](int cb, const Chunk& c) {
    if (cb % G == 0 || cb == t0) {
      wave_lds_fence();                              // previous group's operand reads are done
      // ---- per key group: B operand of the scaled query and the logit correction ----
      const _Float16 sc0 = __builtin_bit_cast(_Float16, static_cast<uint16_t>(c.ks0));
      const _Float16 sc1 = __builtin_bit_cast(_Float16, static_cast<uint16_t>(c.ks1));
      const _Float16 lo0 = __builtin_bit_cast(_Float16, static_cast<uint16_t>(c.kl0));
      const _Float16 lo1 = __builtin_bit_cast(_Float16, static_cast<uint16_t>(c.kl1));
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float qa = qs[r][c0], qb = qs[r][c1];
        const float qak = qa * kinv, qbk = qb * kinv;
        // hi part: the rounded product; lo part: the product's exact residual (one fma), so the
        // split is the same in every instantiation whatever the optimiser shares between them
        const _Float16 h0 = static_cast<_Float16>(qak * static_cast<float>(sc0));
        const _Float16 h1 = static_cast<_Float16>(qbk * static_cast<float>(sc1));
        const _Float16 e0 = static_cast<_Float16>(__builtin_fmaf(qak, static_cast<float>(sc0), -static_cast<float>(h0)));
        const _Float16 e1 = static_cast<_Float16>(__builtin_fmaf(qbk, static_cast<float>(sc1), -static_cast<float>(h1)));
        bq[(2 * r) * kBqStride + l] = pack_h2(h0, h1);
        bq[(2 * r + 1) * kBqStride + l] = pack_h2(e0, e1);
        // logit bias q.lo of this key group (added through the virtual k-step)
        float P = __builtin_fmaf(qa, static_cast<float>(lo0), __fmul_rn(qb, static_cast<float>(lo1)));
        P += dpp<kQuadSwap1>(P);
        P += dpp<kQuadSwap2>(P);
        if (ck == 0) {
          const _Float16 ph = static_cast<_Float16>(P);
          const _Float16 pl = static_cast<_Float16>(P - static_cast<float>(ph));
          bv[r * 16 + g * 4 + ci] = pack_h2(ph, pl);
        }
      }
      wave_lds_fence();
#pragma unroll
      for (int i = 0; i < 4; ++i) bqk[i] = as_half8(bq_src[i]);
      u32x4 bvr = *bv_src;
      if (hl_qk) bvr = u32x4{0u, 0u, 0u, 0u};
      bvirt = as_half8(bvr);
    }
    // ---- logits ----
    float s[8];
#pragma unroll
    for (int tau = 0; tau < 2; ++tau) {
      f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 4; ++i) d = mfma(unpack(c.kw[tau][i]), bqk[i], d);
      d = mfma(tiny, bvirt, d);
#pragma unroll
      for (int i = 0; i < 4; ++i) s[4 * tau + i] = d[i] + dpp<kRowRor + R>(d[i]);   // 2^-20 * logit
    }
    if (cb + 32 > t1) {                              // last chunk of the range: mask past t1
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (cb + 16 * (j >> 2) + 4 * g + (j & 3) >= t1) s[j] = -INFINITY;
    }
    if constexpr (MODE == 2) {
      // logits (log2 units) of this chunk: lane (g, n < R) writes its 8 tokens of row n as two
      // 16-byte stores, [chunk][g][row][j], token cb + 16 (j >> 2) + 4 g + (j & 3)
      if (n < R) {
        float4* sp = reinterpret_cast<float4*>(p.spill + static_cast<int64_t>(bh) * p.spill_bh +
                                               (static_cast<int64_t>(cb / 32) * 4 * R + g * R + n) * 8);
        sp[0] = make_float4(s[0] * kTwo20, s[1] * kTwo20, s[2] * kTwo20, s[3] * kTwo20);
        sp[1] = make_float4(s[4] * kTwo20, s[5] * kTwo20, s[6] * kTwo20, s[7] * kTwo20);
      }
    }
    if constexpr (SCORE) {
      // every product rounded before the cross-lane sums (no contraction into the row pairs' adds,
      // which would round the lanes of a pair differently); score_from_logits computes the same
#pragma clang fp contract(off)
      // probability of each (row, token) under the row's global softmax, summed over the rows
      // of this KV head (lanes n = 0 .. R-1 hold rows 0 .. R-1 of one column variant)
      float x[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j], kTwo20, -score_m)) * score_il;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if constexpr (R >= 2) x[j] += dpp<kQuadSwap1>(x[j]);
        if constexpr (R >= 4) x[j] += dpp<kQuadSwap2>(x[j]);
        if constexpr (R >= 8) x[j] += __shfl_xor(x[j], 4, 64);
      }
      // every lane of group g now holds the row sums of its 8 slots: lane n < 8 adds slot n to
      // the token's score, read with the chunk's loads (each token belongs to one wavefront of
      // the launch, so a plain read-add-write is exact); the 32 tokens go out as one store
      float v = x[0];
#pragma unroll
      for (int j = 1; j < 8; ++j) v = (n == j) ? x[j] : v;
      const int tok = cb + sc_tok;
      if (n < 8 && tok < t1) score_row[tok] = __builtin_fmaf(p.score_weight, v, __uint_as_float(c.sc));
      return;
    }
    // ---- online softmax (base 2) with a lazy maximum: probabilities are taken against the running
    // maximum m_run as long as no logit exceeds it by more than kLazy (p <= 2^kLazy = 16, so
    // p * scale stays far inside fp16 range); only then is the exact chunk maximum reduced across
    // lanes and everything rescaled.  The first chunk always takes this path (m_run = -inf).
    float lm = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
    if (__any(lm * kTwo20 > m_run + kLazy)) {
      const float cm = xmax32(xmax16(lm)) * kTwo20;
      const float m_new = fmaxf(m_run, cm);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[k] *= alpha;
#pragma unroll
      for (int k = 0; k < NB; ++k) {
        Za[k] *= alpha;
        Zb[k] *= alpha;
      }
      la *= alpha;
      lb *= alpha;
      m_run = m_new;
    }
    // slots 2,3,6,7 (tile registers 2,3) carry p/16: their value codes are 16x (high nibbles)
    const float m4 = m_run + 4.0f;
    float pr[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) pr[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j], kTwo20, -(((j & 3) >= 2) ? m4 : m_run)));
    la += (pr[0] + pr[1]) + (pr[4] + pr[5]);
    lb += (pr[2] + pr[3]) + (pr[6] + pr[7]);
    // ---- PV operands p * sv (hi part, or lo part = p*sv - hi), zero-point sums ----
    half8 bp[NB];
#pragma unroll
    for (int bb = 0; bb < NB; ++bb) {
      uint32_t words[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int j0 = 2 * jj, j1 = 2 * jj + 1;
        const half2v m0 = h2(c.mw[bb][j0 >> 2][j0 & 3]);          // (sv, lv) of slot j0
        const half2v m1 = h2(c.mw[bb][j1 >> 2][j1 & 3]);
        // hi = fp16(p * sv) rounded once from the exact product (a mixed-precision fma each);
        // lo = fp16(p * sv - hi), again from the exact product
        const half2v hi = half2v{static_cast<_Float16>(__builtin_fmaf(pr[j0], static_cast<float>(m0[0]), 0.0f)),
                                 static_cast<_Float16>(__builtin_fmaf(pr[j1], static_cast<float>(m1[0]), 0.0f))};
        if constexpr (LO) {
          const half2v cn = hi * hl_neg;                                // 0 (hi lanes) or -hi (lo lanes)
          const half2v val = half2v{static_cast<_Float16>(__builtin_fmaf(pr[j0], static_cast<float>(m0[0]), static_cast<float>(cn[0]))),
                                    static_cast<_Float16>(__builtin_fmaf(pr[j1], static_cast<float>(m1[0]), static_cast<float>(cn[1])))};
          words[jj] = w2(val);
        } else {
          words[jj] = w2(hi);
        }
        float& z = ((j0 & 3) >= 2) ? Zb[bb] : Za[bb];
        z = __builtin_fmaf(pr[j0], static_cast<float>(m0[1]), z);
        z = __builtin_fmaf(pr[j1], static_cast<float>(m1[1]), z);
      }
      bp[bb] = as_half8(u32x4{words[0], words[1], words[2], words[3]});
    }
    // ---- PV ----
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
      const int gcb = (16 * blk) / GV;
      acc[blk] = mfma(unpack(c.vw[blk >> 2][blk & 3]), bp[gcb / GPB], acc[blk]);
    }
  };

  // ---- software pipeline over chunks: two register buffers used in turn; the load of the next
  // chunk is always issued (clamped) before the current chunk is computed ----
  u32x4 ekr[kExU4], evr[kExU4];
  if (fne > 0) {
    const int64_t row0 = static_cast<int64_t>(bh) * p.cap_e + fe0;
    const u32x4* gk = reinterpret_cast<const u32x4*>(static_cast<const uint8_t*>(p.k_exact) + row0 * kD * kEsz);
    const u32x4* gv = reinterpret_cast<const u32x4*>(static_cast<const uint8_t*>(p.v_exact) + row0 * kD * kEsz);
#pragma unroll
    for (int u = 0; u < kExU4; ++u) {
      const int w = threadIdx.x + kThreads * u;
      if (w < fne * kRowU4) {
        ekr[u] = gk[w];
        evr[u] = gv[w];
      }
    }
  }
  // the query rows (scaled) into registers, then the first chunk's loads, then the LDS stores:
  // the staging waits for the query and window rows only
  constexpr int kQPer = (R * kD + kThreads - 1) / kThreads;
  float qv[kQPer];
#pragma unroll
  for (int e = 0; e < kQPer; ++e) {
    const int idx = threadIdx.x + kThreads * e;
    const int r = idx / kD, c = idx % kD;
    qv[e] = (idx < R * kD && r < p.R_real) ? load_as_f32<DT>(p.q, q_offset(p, b, h, r) + c) * p.qscale : 0.0f;
  }
  Chunk ca, cb_;
  if (t0 < t1) load_chunk(t0, ca);
#pragma unroll
  for (int e = 0; e < kQPer; ++e) {
    const int idx = threadIdx.x + kThreads * e;
    if (idx < R * kD) qs[idx / kD][idx % kD] = qv[e];
  }
  if (fne > 0) {
#pragma unroll
    for (int u = 0; u < kExU4; ++u) {
      const int w = threadIdx.x + kThreads * u;
      if (w < fne * kRowU4) {
        ek4[w] = ekr[u];
        ev4[w] = evr[u];
      }
    }
    if (threadIdx.x < 64) {
      const int i = threadIdx.x;
      const bool masked = p.exact_pos != nullptr && p.q_pos != nullptr;
      const int64_t ep = (masked && i < fne) ? p.exact_pos[fe0 + i] : 0;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const bool vis = i < fne && (!masked || ep <= p.q_pos[r % p.Tq]);
        const uint64_t bal = __ballot(vis);
        if (i == 0) emask[r] = static_cast<uint32_t>(bal);
      }
    }
  }
  block_lds_barrier();                             // the first chunk's loads stay in flight
  if (t0 < t1) {
    for (int cb = t0;; cb += 64) {
      load_chunk(cb + 32, cb_);
      step(cb, ca);
      if (cb + 32 >= t1) break;
      load_chunk(cb + 64, ca);
      step(cb + 32, cb_);
      if (cb + 64 >= t1) break;
    }
  }

  // ---- fused exact rows, after the stream (a block dispatched early does this while later
  // blocks stream; one in the last class with its CU to itself): logits of rows 16u + 4*wave + g
  // (16 lanes per row, 8 channels per lane; rows past fne are computed, not stored), then each
  // row's maximum, sum and value sums, left in LDS for the epilogue ----
  if (fne > 0) {
    const void* ek_lds = ek4;
#pragma unroll
    for (int u = 0; u < kFusedExact / 16; ++u) {
      const int i = 16 * u + 4 * wave + g;
      float kx[8];
      load8<DT>(ek_lds, static_cast<int64_t>(i) * kD + 8 * n, kx);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float d = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) d = __builtin_fmaf(qs[r][8 * n + k], kx[k], d);
        d = row_sum16(d);
        if (n == 0 && i < fne) esl[r * kFusedExact + i] = ((emask[r] >> i) & 1u) ? d : -INFINITY;
      }
    }
    block_lds_barrier();                           // logits complete; key rows no longer read
    const void* ev_lds = ev4;
    for (int idx = threadIdx.x; idx < p.R_real * kD; idx += kThreads) {
      const int r = idx / kD, c = idx % kD;
      // every logit of the row and every value of channel c read before any use (rows past fne
      // hold stale data: masked by selects)
      float sl[kFusedExact], vv[kFusedExact];
#pragma unroll
      for (int i = 0; i < kFusedExact; i += 4) {
        const float4 x = *reinterpret_cast<const float4*>(&esl[r * kFusedExact + i]);
        sl[i] = x.x; sl[i + 1] = x.y; sl[i + 2] = x.z; sl[i + 3] = x.w;
      }
#pragma unroll
      for (int i = 0; i < kFusedExact; ++i) vv[i] = load_as_f32<DT>(ev_lds, static_cast<int64_t>(i) * kD + c);
      float me = -INFINITY, le = 0.0f, oe = 0.0f;
#pragma unroll
      for (int i = 0; i < kFusedExact; ++i) me = fmaxf(me, i < fne ? sl[i] : -INFINITY);
      if (me != -INFINITY) {
#pragma unroll
        for (int i = 0; i < kFusedExact; ++i) {
          const float pr = i < fne ? __builtin_amdgcn_exp2f(sl[i] - me) : 0.0f;
          le += pr;
          oe = __builtin_fmaf(pr, i < fne ? vv[i] : 0.0f, oe);
        }
      }
      eo[idx] = oe;
      if (c == 0) {
        estat[r] = me;
        estat[R + r] = le;
      }
    }
  }
  if constexpr (SCORE) return;
  // ---- wavefront epilogue: row sums over lane groups, hi+lo columns, offset and zero terms ----
  const float l_run = xsum32(xsum16(la + 16.0f * lb));
  float Z[NB];
#pragma unroll
  for (int k = 0; k < NB; ++k) Z[k] = xsum32(xsum16(Za[k] + 16.0f * Zb[k]));
  __syncthreads();                               // q rows / operand scratch no longer needed
  float* red_o = smem;                           // [wave][R][kD]
  float* red_ml = smem + kWaves * R * kD;        // [wave][2][R]
#pragma unroll
  for (int blk = 0; blk < 8; ++blk) {
    const int gcb = (16 * blk) / GV;
    const bool mine = (!LO || hl_pv == 1) && (gcb % GPB) == gcl;
    const float Zv = Z[gcb / GPB];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float a = acc[blk][i];
      if constexpr (LO) a += dpp<kRowShr + R>(acc[blk][i]);            // hi + lo columns
      if (mine) red_o[(wave * R + r_n) * kD + 16 * blk + 4 * g + i] = __builtin_fmaf(a, kTwo24, Zv);
    }
  }
  if (g == 0 && n < R) {
    red_ml[(wave * 2 + 0) * R + n] = m_run;
    red_ml[(wave * 2 + 1) * R + n] = l_run;
  }
  __syncthreads();
  const int64_t po = static_cast<int64_t>(bh) * p.S1 + p.n_exact_wg + sidx;
  for (int idx = threadIdx.x; idx < p.R_real * kD; idx += kThreads) {
    const int r = idx / kD, c = idx % kD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, red_ml[(w * 2) * R + r]);
    // the fused exact rows' own state (me, le, oe) joins the wavefronts'
    float me = -INFINITY, le = 0.0f, oe = 0.0f;
    if (fne > 0) {
      me = estat[r];
      le = estat[R + r];
      oe = eo[idx];
      M = fmaxf(M, me);
    }
    float O = 0.0f, L = 0.0f;
    if (me != -INFINITY) {
      const float we = __builtin_amdgcn_exp2f(me - M);
      O = we * oe;
      L = we * le;
    }
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


// Exact-row block e of a split launch (dispatched after the packed blocks, so the blocks of the
// window run on CU slots the first packed blocks to finish leave free): same XCD-aware mapping.
template <int R, int DT>
__device__ __forceinline__ void exact_block_of(const DecodeParams& p, int e, float* smem) {
  const int k = e / 8;
  const int bh = e % 8 + 8 * (k / p.n_exact_wg);
  if (bh < p.BH && k / p.n_exact_wg < (p.BH + 7) / 8) exact_block<R, DT>(p, bh, k % p.n_exact_wg, smem);
}

// One block per (b, h, split).  Blocks are dispatched round-robin over the 8 XCDs by linear id,
// so id -> (xcd = id % 8, k = id / 8) -> bh = xcd + 8*(k / S1), split = k % S1 keeps every
// split of one (b, h) on one XCD (its query rows and key metadata are read through one L2).
// Waves per SIMD the register allocation targets: 3 where the loop fits 168 VGPRs without
// spilling (one PV operand, <= 4 rows), 2 otherwise.
template <int R, int GV>
constexpr int split_waves() {
  constexpr int NB = ((kD / GV) + (8 / R) - 1) / (8 / R);
  return KVQ_WAVES > 0 ? KVQ_WAVES : ((NB == 1 && R <= 4) ? 3 : 2);
}

template <int R, int GV, int DT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(split_waves<R, GV>())))
void kivi_decode_split(DecodeParams p) {
  extern __shared__ float smem[];
  const int bh_pad = (p.BH + 7) / 8 * 8;
  const int n_packed = p.n_split * bh_pad;
  const int id = blockIdx.x;
  if (id < n_packed) {
    int bh, sidx;
    packed_block_of(p, id, p.n_split, &bh, &sidx);
    if (bh < p.BH) packed_block<R, GV, DT, 0>(p, bh, sidx, smem);
  } else {
    exact_block_of<R, DT>(p, id - n_packed, smem);
  }
}

// The split of a scored step: partials as kivi_decode_split, and its logits spilled.
template <int R, int GV, int DT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(split_waves<R, GV>())))
void kivi_decode_split_spill(DecodeParams p) {
  extern __shared__ float smem[];
  const int bh_pad = (p.BH + 7) / 8 * 8;
  const int id = blockIdx.x;
  if (id < p.n_split * bh_pad) {
    int bh, sidx;
    packed_block_of(p, id, p.n_split, &bh, &sidx);
    if (bh < p.BH) packed_block<R, GV, DT, 2>(p, bh, sidx, smem);
  } else {
    exact_block_of<R, DT>(p, id - p.n_split * bh_pad, smem);
  }
}

// Scores of a scored step from the spilled logits.  One thread per (chunk, lane group g) of one
// (b, h): the 8 tokens 4g + 0..3 and 16 + 4g + 0..3 of the chunk (two runs of 4 in the scores row,
// 16-byte loads and stores), their R rows' logits as 2R 16-byte loads.  p = sum over the rows r of
// exp2(logit - M_r) / L_r in the score pass's order and roundings (rows paired as its quad swaps
// pair them, every product rounded), score += weight * p.  The keys are not read again.
template <int R>
__global__ __launch_bounds__(256) void score_from_logits(DecodeParams p) {
#pragma clang fp contract(off)
  const int nc = (p.n_q + 31) / 32;
  const int per_bh = (nc + 63) / 64;
  const int bh = blockIdx.x / per_bh;
  const int c = (blockIdx.x % per_bh) * 64 + threadIdx.x / 4;
  const int g = threadIdx.x % 4;
  if (bh >= p.BH || c >= nc) return;
  float M[R], IL[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t ri = (static_cast<int64_t>(bh) * R + r) * 2;
    M[r] = r < p.R_real ? p.row_ml[ri] : 0.0f;
    IL[r] = r < p.R_real ? 1.0f / p.row_ml[ri + 1] : 0.0f;
  }
  const float4* lg = reinterpret_cast<const float4*>(p.spill + static_cast<int64_t>(bh) * p.spill_bh +
                                                     (static_cast<int64_t>(c) * 4 * R + g * R) * 8);
  float4 L[R][2];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    L[r][0] = lg[2 * r];
    L[r][1] = lg[2 * r + 1];
  }
  float* row = p.scores + static_cast<int64_t>(bh) * p.scores_bh + c * 32 + 4 * g;
  const int left = p.n_q - (c * 32 + 4 * g);             // tokens of this thread's first run left in the row
#pragma unroll
  for (int h = 0; h < 2; ++h) {                          // run h: tokens 16 h + 4 g + 0..3 = slots 4 h .. 4 h + 3
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float x[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float4 q = L[r][h];
        const float lgt = i == 0 ? q.x : i == 1 ? q.y : i == 2 ? q.z : q.w;
        x[r] = __builtin_amdgcn_exp2f(lgt - M[r]) * IL[r];
      }
      if constexpr (R == 1) v[i] = x[0];
      else if constexpr (R == 2) v[i] = x[0] + x[1];
      else if constexpr (R == 4) v[i] = (x[0] + x[1]) + (x[2] + x[3]);
      else v[i] = ((x[0] + x[1]) + (x[2] + x[3])) + ((x[4] + x[5]) + (x[6] + x[7]));
    }
    float* sc = row + 16 * h;
    const int n = left - 16 * h;                         // valid tokens of this run
    if (n >= 4 && p.scores_bh % 4 == 0 && reinterpret_cast<uintptr_t>(p.scores) % 16 == 0) {
      float4 o = *reinterpret_cast<const float4*>(sc);
      o.x = __builtin_fmaf(p.score_weight, v[0], o.x);
      o.y = __builtin_fmaf(p.score_weight, v[1], o.y);
      o.z = __builtin_fmaf(p.score_weight, v[2], o.z);
      o.w = __builtin_fmaf(p.score_weight, v[3], o.w);
      *reinterpret_cast<float4*>(sc) = o;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (i < n) sc[i] = __builtin_fmaf(p.score_weight, v[i], sc[i]);
    }
  }
}

// Exact-row blocks (windows attended neither by the packed splits nor by the merge): their own
// launch, so their registers do not bound the packed kernel's occupancy; same XCD-aware mapping.
template <int R, int DT>
__global__ __launch_bounds__(kThreads) void kivi_decode_exact(DecodeParams p) {
  extern __shared__ float smem[];
  const int k = blockIdx.x / 8;
  const int bh = blockIdx.x % 8 + 8 * (k / p.n_exact_wg);
  if (bh < p.BH) exact_block<R, DT>(p, bh, k % p.n_exact_wg, smem);
}

// Retained decode of the eviction path: the retained-row blocks of every (b, h), then its exact-row
// blocks (the window), S1 = ret_wg + n_exact_wg partials per (b, h); XCD-aware as the exact launch.
template <int R, int DT>
__global__ __launch_bounds__(kThreads) void kivi_decode_retained(DecodeParams p) {
  extern __shared__ float smem[];
  const int k = blockIdx.x / 8;
  const int bh = blockIdx.x % 8 + 8 * (k / p.S1);
  const int s = k % p.S1;
  if (bh >= p.BH) return;
  if (s < p.ret_wg) retained_block<R, DT>(p, bh, s, smem);
  else exact_block<R, DT>(p, bh, s - p.ret_wg, smem);
}

// Score pass of the eviction path: packed blocks only, same split grid and mapping.
template <int R, int GV, int DT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(split_waves<R, GV>())))
void kivi_score_split(DecodeParams p) {
  extern __shared__ float smem[];
  int bh, sidx;
  packed_block_of(p, blockIdx.x, p.n_split, &bh, &sidx);
  if (bh < p.BH) packed_block<R, GV, DT, 1>(p, bh, sidx, smem);
}

template <int R, int GV, int DT>
int launch(DecodeParams& p, int phases, hipStream_t stream) {
  const size_t exact_smem = (R * kD + kWaves * R * kD + kWaves * 2 * R) * sizeof(float);
  const size_t packed_smem = packed_lds_floats<R>() * sizeof(float);
  const size_t fused_smem = p.fused_per > 0 ? fused_lds_floats<R, DT>() * sizeof(float) : 0;
  const int bh_pad = (p.BH + 7) / 8 * 8;
  if ((phases & 1) && p.n_split > 0) {
    const unsigned blocks = static_cast<unsigned>(p.n_split + (p.exact_inline ? p.n_exact_wg : 0)) * bh_pad;
    const size_t smem = std::max(packed_smem + fused_smem, p.exact_inline ? exact_smem : 0);
    if (p.spill != nullptr)
      hipLaunchKernelGGL((kivi_decode_split_spill<R, GV, DT>), dim3(blocks), dim3(kThreads), smem, stream, p);
    else
      hipLaunchKernelGGL((kivi_decode_split<R, GV, DT>), dim3(blocks), dim3(kThreads), smem, stream, p);
    KVQ_LAUNCH_CHECK("kvq_kivi_decode(split)");
  }
  if ((phases & 1) && p.n_exact_wg > 0 && !p.exact_inline) {
    hipLaunchKernelGGL((kivi_decode_exact<R, DT>), dim3(static_cast<unsigned>(p.n_exact_wg) * bh_pad),
                       dim3(kThreads), exact_smem, stream, p);
    KVQ_LAUNCH_CHECK("kvq_kivi_decode(exact)");
  }
  if (phases & 2) {
    MergeArgs ma{};
    ma.ws_o = p.ws_o; ma.ws_m = p.ws_m; ma.ws_l = p.ws_l; ma.S = p.S1;
    ma.Hq = p.Hq; ma.Hkv = p.Hkv; ma.Tq = p.Tq; ma.rep = p.rep; ma.R_real = p.R_real;
    ma.out = p.out; ma.row_ml = p.row_ml;
    if (p.fused_per == 0 && p.n_exact_wg == 0 && p.n_exact > 0)
      ma.ex = ExactArgs{p.q, p.q_sb, p.q_sh, p.q_st, p.qscale, p.k_exact, p.v_exact, p.cap_e, p.n_exact,
                        p.exact_pos, p.q_pos};
    const int rc = launch_merge_rows(ma, R, p.BH, DT, stream);
    if (rc != KVQ_OK) return rc;
  }
  if ((phases & 4) && p.scores != nullptr && p.n_split > 0 && p.spill != nullptr) {
    const int per_bh = ((p.n_q + 31) / 32 + 63) / 64;
    hipLaunchKernelGGL((score_from_logits<R>), dim3(static_cast<unsigned>(per_bh) * p.BH), dim3(256), 0, stream, p);
    KVQ_LAUNCH_CHECK("kvq_kivi_decode(score)");
  } else if ((phases & 4) && p.scores != nullptr && p.n_split > 0) {
    // the score pass writes no partials, so its split count is its own: its registers allow
    // twice the decode's resident blocks, so twice the splits (at least one chunk per wavefront)
    DecodeParams ps = p;
    const int nc = (p.n_q + 31) / 32;
    ps.n_split = std::max(1, std::min(KVQ_SCORE_SPLITS * p.n_split, (nc + kWaves - 1) / kWaves));
    ps.split_classes = 0;
    hipLaunchKernelGGL((kivi_score_split<R, GV, DT>), dim3(static_cast<unsigned>(ps.n_split) * bh_pad),
                       dim3(kThreads), packed_smem, stream, ps);
    KVQ_LAUNCH_CHECK("kvq_kivi_decode(score)");
  }
  return KVQ_OK;
}

struct SplitPlan {
  int n_exact_wg, n_split, split_tokens, S1, R, fused_per, exact_rows, classes, exact_inline;
};

constexpr int kCUs = 256;          // MI355X compute units
constexpr int64_t kBlockCost = 1024;

inline SplitPlan plan_split(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t n_q,
                            int64_t n_exact, int64_t split_tokens, int /*group_k*/, int group_v) {
  SplitPlan sp;
  sp.R = pow2_rows((Hq / Hkv) * Tq);
  // blocks resident per CU = waves per SIMD of the variant (one wavefront of each block per SIMD)
  int resident_blocks = 2;
  switch (sp.R) {
    case 1: resident_blocks = group_v == 128 ? split_waves<1, 128>() : group_v == 64 ? split_waves<1, 64>() : split_waves<1, 32>(); break;
    case 2: resident_blocks = group_v == 128 ? split_waves<2, 128>() : group_v == 64 ? split_waves<2, 64>() : split_waves<2, 32>(); break;
    case 4: resident_blocks = group_v == 128 ? split_waves<4, 128>() : group_v == 64 ? split_waves<4, 64>() : split_waves<4, 32>(); break;
    default: resident_blocks = group_v == 128 ? split_waves<8, 128>() : group_v == 64 ? split_waves<8, 64>() : split_waves<8, 32>(); break;
  }
  const int64_t nc = (n_q + 31) / 32;                   // 32-token chunks per (b, h)
  int64_t ns = 0;
  if (nc > 0 && split_tokens > 0) {
    ns = (n_q + split_tokens - 1) / split_tokens;
  } else if (nc > 0) {
    // Fewest rounds of resident blocks times (chunks of the longest wavefront + a fixed per-block
    // cost of kBlockCost tokens: query load, operand set-up, partial write, one more merge
    // input): blocks of one launch run in ceil(blocks / slots) rounds.  Ties go to fewer splits.
    const int64_t bh = B * Hkv;
    const int64_t slots = static_cast<int64_t>(kCUs) * resident_blocks;
    int64_t best_cost = 0;
    for (int64_t cand = 1; cand <= std::min<int64_t>((nc + kWaves - 1) / kWaves, 512); ++cand) {
      const int64_t per_wave = (nc + cand * kWaves - 1) / (cand * kWaves);
      const int64_t rounds = (bh * cand + slots - 1) / slots;
      const int64_t cost = rounds * (32 * per_wave * kWaves + kBlockCost);
      if (ns == 0 || cost < best_cost) {
        ns = cand;
        best_cost = cost;
      }
    }
  }
  // every wavefront gets at least one chunk
  ns = std::min<int64_t>(ns, (nc + kWaves - 1) / kWaves);
  sp.n_split = static_cast<int>(ns);
  sp.split_tokens = ns > 0 ? static_cast<int>((n_q + ns - 1) / ns) : 0;
  // class-weighted splits: the packed blocks are exactly one round of 3 per CU, every (b, h)
  // with the same number of splits in each class
  const int64_t bhn = B * Hkv;
  sp.classes = KVQ_CLASSES != 0 ? split_classes(bhn, ns, resident_blocks) : 0;
  // exact window: in the packed splits (at most kFusedExact rows each), else in the merge (at
  // most kExactInMerge rows), else in exact-row blocks
  const int64_t per = ns > 0 ? (n_exact + ns - 1) / ns : 0;
  sp.fused_per = (n_exact > 0 && ns > 0 && per <= kFusedExact) ? static_cast<int>(per) : 0;
  sp.exact_rows = 0;
  sp.exact_inline = 0;
  if (sp.classes > 0 && n_exact > 0) {
    // one full round of packed blocks: the window in exact-row blocks of the same launch,
    // which fill the slots of the first blocks to finish while the last class still streams
    sp.fused_per = 0;
    sp.exact_inline = 1;
    sp.n_exact_wg = plan_exact_blocks(B * Hkv, n_exact, &sp.exact_rows);
  } else {
    sp.n_exact_wg = (n_exact == 0 || sp.fused_per > 0 || exact_in_merge(n_exact))
                        ? 0 : plan_exact_blocks(B * Hkv, n_exact, &sp.exact_rows);
  }
  sp.S1 = sp.n_exact_wg + sp.n_split;
  return sp;
}

// ---- the allocation-free entry point's scratch ------------------------------------------------
// kvq_kivi_decode_noalloc keeps the split partials and row statistics (what kvq_kivi_decode keeps in
// its workspace argument) in this array.  Every GPU the library runs on holds its own copy for the
// life of the process.  In host code `scratch` names a host-side stand-in, never the device array:
// the device address of each GPU's copy comes from hipGetSymbolAddress, once per device, with that
// device current, and only that address is passed to kernels.
constexpr int64_t kScratchFloats = KVQ_NOALLOC_SCRATCH_FLOATS;      // 8 MiB per GPU
__device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::atomic<float*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of the current device's scratch (looked up on the first call on that device).
// The stream must belong to the current device: its kernels read that device's copy.
int current_scratch(void* stream, float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("kvq_kivi_decode_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    return KVQ_EHIP;
  }
  KVQ_REQUIRE(dev >= 0 && dev < kMaxDevices, "kvq_kivi_decode_noalloc: device %d out of range", dev);
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev);
    if (e != hipSuccess) {
      set_error("kvq_kivi_decode_noalloc: hipStreamGetDevice: %s", hipGetErrorString(e));
      return KVQ_EHIP;
    }
    KVQ_REQUIRE(sdev == dev, "kvq_kivi_decode_noalloc: the stream belongs to device %d but device %d is current",
                (int)sdev, dev);
  }
  float* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      void* addr = nullptr;
      e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || addr == nullptr) {
        set_error("kvq_kivi_decode_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(e));
        return KVQ_EHIP;
      }
      p = static_cast<float*>(addr);
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return KVQ_OK;
}

}  // namespace
}  // namespace kvq

using namespace kvq;

extern "C" int64_t kvq_kivi_decode_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq,
                                             int64_t d, int64_t n_q, int64_t n_exact,
                                             int group_k, int group_v, int64_t split_tokens) {
  if (d != kD || B <= 0 || Hkv <= 0 || Hq % Hkv != 0 || Tq <= 0 || group_k <= 0) return -1;
  if (group_v != 32 && group_v != 64 && group_v != 128) return -1;
  const SplitPlan sp = plan_split(B, Hq, Hkv, Tq, n_q, n_exact, split_tokens, group_k, group_v);
  return B * Hkv * (static_cast<int64_t>(sp.S1) * sp.R * (kD + 2) + 2 * sp.R);
}

// A scored step's workspace: the decode's, then its logits (32 R floats per 32-token chunk and
// (b, h)).  Given at least this much, a scored step spills its logits and scores them without
// reading the keys again; given only kvq_kivi_decode_workspace's floats, it runs the score pass.
extern "C" int64_t kvq_kivi_score_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d,
                                            int64_t n_q, int64_t n_exact, int group_k, int group_v,
                                            int64_t split_tokens) {
  const int64_t base = kvq_kivi_decode_workspace(B, Hq, Hkv, Tq, d, n_q, n_exact, group_k, group_v, split_tokens);
  if (base < 0) return base;
  const int R = pow2_rows((Hq / Hkv) * Tq);
  return (base + 3) / 4 * 4 + B * Hkv * ((n_q + 31) / 32) * 32 * R;    // logits 16-byte aligned
}

extern "C" int kvq_kivi_decode(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st,
                               int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d,
                               float scaling, const uint8_t* kc, const uint16_t* k_lo,
                               const uint16_t* k_sc, const uint8_t* vc, const uint16_t* vmeta,
                               int64_t cap_t, int64_t n_q, int group_k, int group_v,
                               const void* k_exact, const void* v_exact, int exact_dtype,
                               int64_t cap_e, int64_t n_exact, const int64_t* exact_pos,
                               const int64_t* q_pos, void* out, int out_dtype, float* workspace,
                               int64_t workspace_floats, float* scores, int64_t scores_bh,
                               float score_weight, int64_t split_tokens, int phases,
                               void* stream) {
  KVQ_REQUIRE(phases >= 1 && phases <= 7, "kvq_kivi_decode: phases must be in 1..7");
  KVQ_REQUIRE(scores == nullptr || scores_bh >= n_q, "kvq_kivi_decode: scores row stride < n_q");
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
  KVQ_REQUIRE(n_exact >= 0 && n_exact <= cap_e && n_exact <= 65536,
              "kvq_kivi_decode: bad n_exact");
  KVQ_REQUIRE(n_q + n_exact > 0, "kvq_kivi_decode: empty cache");
  KVQ_REQUIRE(n_q == 0 || (kc && k_lo && k_sc && vc && vmeta), "kvq_kivi_decode: null packed cache");
  KVQ_REQUIRE(n_exact == 0 || (k_exact && v_exact), "kvq_kivi_decode: null exact rows");
  KVQ_REQUIRE(n_exact == 0 || (reinterpret_cast<uintptr_t>(k_exact) % 16 == 0 &&
                               reinterpret_cast<uintptr_t>(v_exact) % 16 == 0),
              "kvq_kivi_decode: exact rows must be 16-byte aligned");
  KVQ_REQUIRE(q && out && workspace, "kvq_kivi_decode: null q/out/workspace");
  KVQ_REQUIRE((exact_pos == nullptr) == (q_pos == nullptr), "kvq_kivi_decode: exact_pos and q_pos go together");
  KVQ_REQUIRE(n_q < (1LL << 31) && B * Hkv < 65536, "kvq_kivi_decode: sizes out of range");
  const SplitPlan sp = plan_split(B, Hq, Hkv, Tq, n_q, n_exact, split_tokens, group_k, group_v);
  const int64_t need = B * Hkv * (static_cast<int64_t>(sp.S1) * sp.R * (kD + 2) + 2 * sp.R);
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
  p.row_ml = p.ws_l + nrow;
  p.scores = scores;
  p.scores_bh = scores_bh;
  p.score_weight = score_weight;
  // a scored step with room for its logits after the decode's workspace spills them
  const int64_t spill_bh = ((n_q + 31) / 32) * 32 * sp.R;
  const int64_t spill_off = (need + 3) / 4 * 4;
  if (scores != nullptr && n_q > 0 && workspace_floats >= spill_off + B * Hkv * spill_bh) {
    p.spill = workspace + spill_off;
    p.spill_bh = spill_bh;
  }
  p.BH = static_cast<int>(B * Hkv);
  p.n_exact_wg = sp.n_exact_wg; p.n_split = sp.n_split; p.split_tokens = sp.split_tokens; p.S1 = sp.S1;
  p.fused_per = sp.fused_per;
  p.exact_rows = sp.exact_rows;
  p.split_classes = sp.classes;
  p.exact_inline = sp.exact_inline;
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

namespace kvq {
namespace {
// Rows per block of a retained decode (one plan for the retained rows and the window: about one
// round of workgroups over the (b, h), at most 64 rows a wavefront) and the blocks of each part.
struct RetainedPlan {
  int rows, ret_wg, ex_wg, R;
};
inline RetainedPlan plan_retained(int64_t BH, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t n_ret, int64_t n_exact) {
  RetainedPlan rp;
  rp.R = pow2_rows((Hq / Hkv) * Tq);
  int rows = 0;
  plan_exact_blocks(BH, n_ret + n_exact, &rows);
  rows = std::max(16, std::min(rows, 256));
  rp.rows = rows;
  rp.ret_wg = static_cast<int>((n_ret + rows - 1) / rows);
  rp.ex_wg = static_cast<int>((n_exact + rows - 1) / rows);
  return rp;
}
}  // namespace
}  // namespace kvq

extern "C" int64_t kvq_kivi_retained_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d,
                                               int64_t n_ret, int64_t n_exact) {
  if (d != kD || B <= 0 || Hkv <= 0 || Hq % Hkv != 0 || Tq <= 0 || n_ret < 0 || n_exact < 0 || n_ret + n_exact == 0)
    return -1;
  const RetainedPlan rp = plan_retained(B * Hkv, Hq, Hkv, Tq, n_ret, n_exact);
  return B * Hkv * (static_cast<int64_t>(rp.ret_wg + rp.ex_wg) * rp.R * (kD + 2) + 2 * rp.R);
}

extern "C" int kvq_kivi_decode_retained(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st,
                                        int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d, float scaling,
                                        const uint8_t* kc, const uint16_t* k_lo, const uint16_t* k_sc,
                                        const uint8_t* vc, const uint16_t* vmeta, int64_t cap_t, int64_t n_q,
                                        int group_k, int group_v, const int32_t* idx, int64_t n_ret, int64_t idx_bh,
                                        const void* k_exact, const void* v_exact, int exact_dtype, int64_t cap_e,
                                        int64_t n_exact, const int64_t* exact_pos, const int64_t* q_pos, void* out,
                                        int out_dtype, float* workspace, int64_t workspace_floats, void* stream) {
  KVQ_REQUIRE(d == kD, "kvq_kivi_decode_retained: head_dim must be 128 (got %lld)", (long long)d);
  KVQ_REQUIRE(valid_dtype(q_dtype) && q_dtype == exact_dtype && q_dtype == out_dtype,
              "kvq_kivi_decode_retained: q, exact rows and output must share one dtype");
  KVQ_REQUIRE(B > 0 && Hkv > 0 && Hq % Hkv == 0 && Tq > 0, "kvq_kivi_decode_retained: bad head counts");
  const int64_t R_real = (Hq / Hkv) * Tq;
  KVQ_REQUIRE(R_real <= 8, "kvq_kivi_decode_retained: rep*Tq must be <= 8 (got %lld)", (long long)R_real);
  KVQ_REQUIRE(group_k % 32 == 0 && group_k > 0, "kvq_kivi_decode_retained: group_k must be a multiple of 32");
  KVQ_REQUIRE(group_v == 32 || group_v == 64 || group_v == 128, "kvq_kivi_decode_retained: group_v in {32,64,128}");
  KVQ_REQUIRE(cap_t % group_k == 0 && cap_t % 32 == 0 && n_q >= 0 && n_q <= cap_t && n_q < (1LL << 31),
              "kvq_kivi_decode_retained: cap_t must be a multiple of group_k and 32, 0 <= n_q <= cap_t");
  KVQ_REQUIRE(n_ret >= 0 && n_ret < (1LL << 31) && idx_bh >= n_ret, "kvq_kivi_decode_retained: bad retained count");
  KVQ_REQUIRE(n_exact >= 0 && n_exact <= cap_e && n_exact <= 65536, "kvq_kivi_decode_retained: bad n_exact");
  KVQ_REQUIRE(n_ret + n_exact > 0, "kvq_kivi_decode_retained: empty cache");
  KVQ_REQUIRE(n_ret == 0 || (kc && k_lo && k_sc && vc && vmeta && idx), "kvq_kivi_decode_retained: null packed cache");
  // a masked retained row still loads position 0, so a retained set needs a non-empty cache
  KVQ_REQUIRE(n_ret == 0 || cap_t >= 32, "kvq_kivi_decode_retained: retained rows over an empty packed cache");
  KVQ_REQUIRE(n_ret == 0 || (reinterpret_cast<uintptr_t>(k_lo) % 16 == 0 && reinterpret_cast<uintptr_t>(k_sc) % 16 == 0),
              "kvq_kivi_decode_retained: key metadata must be 16-byte aligned");
  KVQ_REQUIRE(n_exact == 0 || (k_exact && v_exact), "kvq_kivi_decode_retained: null exact rows");
  KVQ_REQUIRE(n_exact == 0 || (reinterpret_cast<uintptr_t>(k_exact) % 16 == 0 &&
                               reinterpret_cast<uintptr_t>(v_exact) % 16 == 0),
              "kvq_kivi_decode_retained: exact rows must be 16-byte aligned");
  KVQ_REQUIRE(q && out && workspace, "kvq_kivi_decode_retained: null q/out/workspace");
  KVQ_REQUIRE((exact_pos == nullptr) == (q_pos == nullptr), "kvq_kivi_decode_retained: exact_pos and q_pos go together");
  KVQ_REQUIRE(B * Hkv < 65536, "kvq_kivi_decode_retained: sizes out of range");
  const RetainedPlan rp = plan_retained(B * Hkv, Hq, Hkv, Tq, n_ret, n_exact);
  const int S1 = rp.ret_wg + rp.ex_wg;
  const int64_t need = B * Hkv * (static_cast<int64_t>(S1) * rp.R * (kD + 2) + 2 * rp.R);
  KVQ_REQUIRE(workspace_floats >= need, "kvq_kivi_decode_retained: workspace too small (%lld < %lld floats)",
              (long long)workspace_floats, (long long)need);
  DecodeParams p{};
  p.q = q; p.q_sb = q_sb; p.q_sh = q_sh; p.q_st = q_st;
  p.Hq = (int)Hq; p.Hkv = (int)Hkv; p.Tq = (int)Tq; p.rep = (int)(Hq / Hkv); p.R_real = (int)R_real;
  p.qscale = scaling * kLog2e;
  p.kc = kc; p.k_lo = k_lo; p.k_sc = k_sc; p.vc = vc; p.vmeta = vmeta;
  p.cap_t = cap_t; p.n_q = (int)n_q; p.group_k = group_k; p.group_v = group_v; p.ngv = (int)(kD / group_v);
  p.k_exact = k_exact; p.v_exact = v_exact; p.cap_e = cap_e; p.n_exact = (int)n_exact;
  p.exact_pos = exact_pos; p.q_pos = q_pos;
  const int64_t nrow = B * Hkv * static_cast<int64_t>(S1) * rp.R;
  p.ws_o = workspace;
  p.ws_m = workspace + nrow * kD;
  p.ws_l = p.ws_m + nrow;
  p.row_ml = p.ws_l + nrow;
  p.BH = static_cast<int>(B * Hkv);
  p.S1 = S1;
  p.exact_rows = rp.rows;
  p.ex_po0 = rp.ret_wg;
  p.ret_idx = idx; p.ret_bh = idx_bh; p.n_ret = (int)n_ret; p.ret_wg = rp.ret_wg;
  p.out = out;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int bh_pad = (p.BH + 7) / 8 * 8;
  const size_t smem = (rp.R * kD + kWaves * rp.R * kD + kWaves * 2 * rp.R) * sizeof(float);
  const dim3 grid(static_cast<unsigned>(S1) * bh_pad);
#define KVQ_RT(R_, DT_) hipLaunchKernelGGL((kivi_decode_retained<R_, DT_>), grid, dim3(kThreads), smem, s, p)
#define KVQ_RT_R(DT_)                       \
  switch (rp.R) {                           \
    case 1: KVQ_RT(1, DT_); break;          \
    case 2: KVQ_RT(2, DT_); break;          \
    case 4: KVQ_RT(4, DT_); break;          \
    default: KVQ_RT(8, DT_); break;         \
  }
  switch (q_dtype) {
    case KVQ_F32: KVQ_RT_R(KVQ_F32) break;
    case KVQ_F16: KVQ_RT_R(KVQ_F16) break;
    default: KVQ_RT_R(KVQ_BF16) break;
  }
#undef KVQ_RT_R
#undef KVQ_RT
  KVQ_LAUNCH_CHECK("kvq_kivi_decode_retained");
  MergeArgs ma{};
  ma.ws_o = p.ws_o; ma.ws_m = p.ws_m; ma.ws_l = p.ws_l; ma.S = S1;
  ma.Hq = p.Hq; ma.Hkv = p.Hkv; ma.Tq = p.Tq; ma.rep = p.rep; ma.R_real = p.R_real;
  ma.out = out; ma.row_ml = p.row_ml;
  return launch_merge_rows(ma, rp.R, p.BH, q_dtype, s);
}

extern "C" int kvq_kivi_decode_noalloc(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st,
                                       int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d,
                                       float scaling, const uint8_t* kc, const uint16_t* k_lo,
                                       const uint16_t* k_sc, const uint8_t* vc, const uint16_t* vmeta,
                                       int64_t cap_t, int64_t n_q, int group_k, int group_v,
                                       const void* k_exact, const void* v_exact, int exact_dtype,
                                       int64_t cap_e, int64_t n_exact, const int64_t* exact_pos,
                                       const int64_t* q_pos, void* out, int out_dtype, float* scores,
                                       int64_t scores_bh, float score_weight, int64_t split_tokens,
                                       int phases, void* stream) {
  // shapes the planner rejects fall through to kvq_kivi_decode, which names what is wrong
  const int64_t need = kvq_kivi_decode_workspace(B, Hq, Hkv, Tq, d, n_q, n_exact, group_k, group_v, split_tokens);
  KVQ_REQUIRE(need <= kScratchFloats,
              "kvq_kivi_decode_noalloc: this step needs %lld scratch floats, more than the static scratch of "
              "%lld (call kvq_kivi_decode with a workspace instead)", (long long)need, (long long)kScratchFloats);
  float* ws = nullptr;
  const int rc = current_scratch(stream, &ws);
  if (rc != KVQ_OK) return rc;
  return kvq_kivi_decode(q, q_dtype, q_sb, q_sh, q_st, B, Hq, Hkv, Tq, d, scaling, kc, k_lo, k_sc, vc, vmeta, cap_t,
                         n_q, group_k, group_v, k_exact, v_exact, exact_dtype, cap_e, n_exact, exact_pos, q_pos, out,
                         out_dtype, ws, kScratchFloats, scores, scores_bh, score_weight, split_tokens, phases, stream);
}
