// QUASAR compressed-domain decode (QuasarState.attend, QUASAR_KV.py:1945-1968): attention of a
// decode step over exact rows and embedded spectral codes, reading only the packed bytes.
//
// Stored code of one layer (QuasarState.__init__, 1883-1898), per side (0 = keys, 1 = values):
//   codes   one flat uint8 buffer: per step, in step order, an (Hkv, n_s, nb) block of pack_rows
//           rows (QUASAR_KV.py:1185-1190: the 8/b codes of a byte, first in the most significant
//           bits) of the step's band [a, a + w) at b bits, for the n_s most important coded tokens
//   table   int32 rows [byte offset of the step's block, n_s, nb, a, w, b, level offset]
//   levels  float32 stage codebooks, concatenated (one list for both sides)
// plus rho (Hkv, n_c) fp16 per coded token and side, the read-out matrices T_K (Hkv, d, R) float32
// and T_V^T (Hkv, R, d, transposed) fp16 -- the precision the reference stores them at -- and the
// means mu (Hkv, d) float32.  Coded token j of head h contributes
//   logit  (sum over the K steps with n_s > j of qt[band] . level[code]) rho_K[j] + q . mu_K
//   value  p_j rho_V[j] level[code] into coefficient a + i of each V step it owns,
// with qt = q T_K; the value coefficients are lifted once per query row: o += acc T_V^T + P mu_V.
//
// Launches: quasar_prologue (qt and q . mu_K, log2 units), quasar_split (coded workgroups over
// makespan-balanced token ranges, each lifting its coefficient sums by T_V into an output partial, then
// exact-row workgroups when the exact part is long), merge_rows_kernel (the shared row merge; a short
// exact part is attended there).
#include <algorithm>
#include <vector>

#include "common.hpp"
#include "mfma_common.hpp"
#include "partials.hpp"

namespace kvq {
namespace {

constexpr int kQD = 128;                  // head_dim (the decode entry point requires it)
constexpr int kQChunk = 64;               // coded tokens per wavefront iteration (lane = token)
constexpr int kQWaves = 4;
constexpr int kQThreads = 256;
constexpr int kQExRows = 128;             // exact rows per exact-row workgroup
constexpr int kQMaxR = 256;               // coefficient dimension limit (R_k, R_v <= d <= 256)
constexpr int kQMaxLevels = 256;
constexpr float kQLazy = 4.0f;
constexpr int kQRowCoef = 128;            // coefficients per query row in LDS (R_k, R_v <= d = 128)

struct QuasarParams {
  int Hkv, Hq, Tq, rep, R_real;
  int64_t n_c;
  int n_chunks;
  const float* qt;                        // [Hkv][R][Rk], log2 units
  const float* qmu;                       // [Hkv][R]
  int Rk, Rv;
  const uint8_t* kcodes;
  const uint8_t* vcodes;
  uint32_t kbytes, vbytes;                // sizes of the code buffers (buffer-resource ranges)
  const float* levels;
  int n_levels;
  const uint16_t* rho_k;                  // [Hkv][n_c] fp16
  const uint16_t* rho_v;
  const int32_t* bounds;                  // [S + 1] chunk boundaries of the coded splits
  const int32_t* slots;                   // [2][kQSlots][kQSlotInts] slot table (kvq_quasar_plan)
  int nslots_k, nslots_v;
  int S;
  float* ws_m;                            // [Hkv][S][R]
  float* ws_l;
  float* ws_o;                            // [Hkv][S][R][128]: the split's lifted output (acc T_V^T + l mu_V)
  const uint16_t* tvt;                    // [Hkv][Rv][128] read-out T_V transposed, fp16 (its stored precision)
  const float* muv;                       // [Hkv][128]
  ExactArgs ex;                           // exact rows of the split launch (ex.n rows)
  int S_ex;                               // exact-row workgroups per (h, row)
  float* ex_m;                            // [Hkv][S_ex][R]
  float* ex_l;
  float* ex_o;                            // [Hkv][S_ex][R][128]
};

// qt[h][k][r] = qscale sum_c q[c] T_K[h][c][k] (coefficient-major: the R rows of a coefficient
// side by side, so the split reads four coefficients of every row as one scalar load);
// qmu[h][r] = qscale q . mu_K[h]; padded rows r >= R_real are zero
template <int DT>
__global__ __launch_bounds__(256) void quasar_prologue(const void* __restrict__ q, int64_t q_sh, int64_t q_st, int rep,
                                                       int Tq, int R, int R_real, int d, const float* __restrict__ Tk,
                                                       const float* __restrict__ muk, int Rk, float qscale,
                                                       float* __restrict__ qt, float* __restrict__ qmu) {
  __shared__ float qs[256];
  __shared__ float red[4];
  const int h = blockIdx.x / R, r = blockIdx.x % R;
  const int tid = threadIdx.x;
  if (r >= R_real) {
    if (tid < Rk) qt[(static_cast<int64_t>(h) * Rk + tid) * R + r] = 0.0f;
    if (tid == 0) qmu[static_cast<int64_t>(h) * R + r] = 0.0f;
    return;
  }
  const int hq = h * rep + r / Tq, t = r % Tq;
  float pm = 0.0f;
  if (tid < d) {
    const float qc = load_as_f32<DT>(q, static_cast<int64_t>(hq) * q_sh + static_cast<int64_t>(t) * q_st + tid);
    qs[tid] = qc;
    pm = qc * muk[static_cast<int64_t>(h) * d + tid];
  }
  pm = wave_sum(pm);
  if ((tid & 63) == 0) red[tid >> 6] = pm;
  __syncthreads();
  if (tid < Rk) {
    // the column's d = 128 values loaded at once (one memory round trip), then the dot product in
    // channel order
    const float* col = Tk + static_cast<int64_t>(h) * d * Rk + tid;
    float cv[kQD];
#pragma unroll
    for (int c = 0; c < kQD; ++c) cv[c] = col[static_cast<int64_t>(c) * Rk];
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < kQD; ++c) acc = __builtin_fmaf(qs[c], cv[c], acc);
    qt[(static_cast<int64_t>(h) * Rk + tid) * R + r] = acc * qscale;
  }
  if (tid == 0) qmu[static_cast<int64_t>(h) * R + r] = ((red[0] + red[1]) + (red[2] + red[3])) * qscale;
}

// Code slots: the dwords of a token's rows over every step of a side, in step order (step s holds
// nb_s / 4 consecutive slots).  A side holds at most kQSlots of them (128 bytes per token: d = 128
// coefficients at 8 bits over all stages).  kvq_quasar_plan writes the slot table, int32
// [side][slot][8]: byte offset of the dword for token 0 of head 0 (step offset + 4 dw), n_s, nb,
// first coefficient of the dword, bits, level offset, first slot of the step, step index.  The
// decode walks the steps through their first slots.
constexpr int kQSlots = 32;
constexpr int kQSlotInts = 8;
constexpr int kQSideBytes = kQSlots * 256;   // one side's rows of a chunk: slot s at s * 256 bytes

typedef __attribute__((address_space(1))) void qgvoid;
typedef __attribute__((address_space(3))) void qlvoid;

// A chunk's rows of one step straight into LDS (LDS DMA: no registers held while in flight).
// Lane = token: rows of >= 16 bytes go as 16-byte pieces (piece q of every token at q * 1024,
// token t at t * 16), shorter rows as dwords (dword d at d * 256, token t at t * 4).  Tokens past
// n_s re-read the step's last row (never used).
__device__ __forceinline__ void dma_step(const uint8_t* codes, int off, int ns, int nb, int h, int tok, uint8_t* dst) {
  const uint8_t* src = codes + off + (static_cast<int64_t>(h) * ns + min(tok, ns - 1)) * nb;
  if (nb >= 16) {
    for (int q = 0; q < nb / 16; ++q)
      __builtin_amdgcn_global_load_lds((qgvoid*)(src + 16 * q), (qlvoid*)(dst + q * 1024), 16, 0, 0);
  } else {
    for (int d = 0; d < nb / 4; ++d)
      __builtin_amdgcn_global_load_lds((qgvoid*)(src + 4 * d), (qlvoid*)(dst + d * 256), 4, 0, 0);
  }
}

// wave-uniform tables read through the constant address space: scalar loads into SGPRs, which
// the FMAs take as operands directly
typedef __attribute__((address_space(4))) const float qcfloat;
typedef __attribute__((address_space(4))) const int32_t qcint;

// Scores of one K dword for this lane's token: its 32 / B codes (coefficients c0 ..), each code's
// level times qt[c][r]; qt (this head's, coefficient-major) read by scalar loads, kQG coefficients
// of every row at a time.  A scalar load's data is waited for together with the LDS lookups in
// flight (one counter), so each group of kQG codes costs one exposed wait: groups of eight halve
// them against groups of four.
constexpr int kQG = 8;
template <int R, int B>
__device__ __forceinline__ void score_word(uint32_t word, int c0, int lo, const float* lv, qcfloat* qtc,
                                           float (&sc)[R]) {
  constexpr int per = 8 / B, mask = (1 << B) - 1, cpw = 32 / B;
  constexpr int QG = cpw < kQG ? cpw : kQG;
#pragma unroll
  for (int g = 0; g < cpw / QG; ++g) {
    float l[QG];
#pragma unroll
    for (int i = 0; i < QG; ++i) {
      const int m = QG * g + i, by = m / per, k = m % per;
      l[i] = lv[lo + static_cast<int>((word >> (8 * by + (per - 1 - k) * B)) & mask)];
    }
    qcfloat* qg = qtc + (c0 + QG * g) * R;
#pragma unroll
    for (int i = 0; i < QG; ++i)
#pragma unroll
      for (int r = 0; r < R; ++r) sc[r] = __builtin_fmaf(qg[i * R + r], l[i], sc[r]);
  }
}

// Scores of one staged K step for this lane's token.
template <int R, int B>
__device__ __forceinline__ void score_step(const uint8_t* st, int nb, int a, int lo, int lane, const float* lv,
                                           qcfloat* qtc, float (&sc)[R]) {
  constexpr int cpw = 32 / B;
  if (nb >= 16) {
    for (int q = 0; q < nb / 16; ++q) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(st + q * 1024 + lane * 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) score_word<R, B>(w[i], a + (4 * q + i) * cpw, lo, lv, qtc, sc);
    }
  } else {
    for (int d = 0; d < nb / 4; ++d)
      score_word<R, B>(*reinterpret_cast<const uint32_t*>(st + d * 256 + lane * 4), a + d * cpw, lo, lv, qtc, sc);
  }
}

// Values of one staged V step on the matrix cores: acc[r][a + c] += sum_t pv[t][r] level(code(t, c))
// as D = A B per 16-coefficient tile and 32-token k-block, A = the chunk's probabilities (rows r,
// fp16 hi + lo parts), B = the levels of column c's codes (fp16 hi + lo parts from lvp), three
// products (hi hi, hi lo, lo hi).  Lane l supplies column n = l % 16 (coefficient 16 j + n: byte
// (16 j + n) / per, code position (16 j + n) % per) for the k-slots of lane group g = l / 16, which
// stand for tokens 32 kb + g + 4 i (neighbouring lane groups read neighbouring tokens: distinct
// LDS banks).  The products reduce over the tokens inside the matrix core; each tile then joins
// the wavefront's accumulator once (lanes of rows r < R, the tile's coefficients below w).
template <int R, int B>
__device__ __forceinline__ void value_step_mfma(const uint8_t* st, int nb, int a, int lo, int ns, int j0,
                                                const uint32_t* lvp, const half8 (&Ah)[2], const half8 (&Al)[2],
                                                float* accw, int lane) {
  constexpr int per = 8 / B, mask = (1 << B) - 1;
  const int w = nb * per;                                         // coefficients of the step
  const int n = lane & 15, g = lane >> 4;
  // tokens j0 + t with t >= ns - j0 own no code of this step: their probabilities drop out
  half8 Ahm[2] = {Ah[0], Ah[1]}, Alm[2] = {Al[0], Al[1]};
  const int n_own = ns - j0;
  if (n_own < kQChunk) {                                          // wave-uniform
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const bool own = 32 * kb + g + 4 * i < n_own;
        Ahm[kb][i] = own ? Ahm[kb][i] : static_cast<_Float16>(0.0f);
        Alm[kb][i] = own ? Alm[kb][i] : static_cast<_Float16>(0.0f);
      }
  }
  const int ts = nb >= 16 ? 16 : 4;                               // staged bytes per token
  for (int j = 0; j < (w + 15) / 16; ++j) {
    const int c = 16 * j + n;
    const int cc = c < w ? c : w - 1;                             // columns past w read a real byte
    const int byte = cc / per;
    const int shift = (per - 1 - cc % per) * B;
    const uint8_t* col = nb >= 16 ? st + (byte >> 4) * 1024 + (byte & 15) : st + (byte >> 2) * 256 + (byte & 3);
    f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      uint32_t pr[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t v = col[(32 * kb + g + 4 * i) * ts];
        pr[i] = lvp[lo + static_cast<int>((v >> shift) & static_cast<uint32_t>(mask))];
      }
      u32x4 bh, bl;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        bh[m] = __builtin_amdgcn_perm(pr[2 * m + 1], pr[2 * m], 0x05040100u);   // hi parts
        bl[m] = __builtin_amdgcn_perm(pr[2 * m + 1], pr[2 * m], 0x07060302u);   // lo parts
      }
      d = mfma(Ahm[kb], as_half8(bh), d);
      d = mfma(Ahm[kb], as_half8(bl), d);
      d = mfma(Alm[kb], as_half8(bh), d);
    }
    if (c < w) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * g + i;
        if (r < R) accw[r * kQRowCoef + a + c] += d[i];
      }
    }
  }
}

template <int R, int DT>
__global__ __launch_bounds__(kQThreads) __attribute__((amdgpu_waves_per_eu(3))) void quasar_split(QuasarParams p) {
  __shared__ __align__(16) uint8_t stage_all[kQWaves][1][kQSideBytes];
  __shared__ float lv[kQMaxLevels];
  __shared__ uint32_t lvp[kQMaxLevels];                           // levels as fp16 (hi, lo) pairs
  __shared__ __align__(16) float pch_all[kQWaves][kQChunk * R];
  __shared__ float acc_all[kQWaves][R * kQRowCoef];
  __shared__ int next_chunk;                                      // the split's next unclaimed chunk
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_coded_wg = p.Hkv * p.S;
  if (static_cast<int>(blockIdx.x) >= n_coded_wg) {
    // ---- exact-row workgroup: (h, row r, block eb) over rows [eb * kQExRows, ...) ----
    const int e = blockIdx.x - n_coded_wg;
    const int eb = e % p.S_ex, hr = e / p.S_ex;
    const int h = hr / p.R_real, r = hr % p.R_real;
    const int hq = h * p.rep + r / p.Tq, t = r % p.Tq;
    ExactArgs ea = p.ex;
    const int i0 = eb * kQExRows;
    ea.n = min(kQExRows, p.ex.n - i0);
    const int64_t esz = DT == KVQ_F32 ? 4 : 2;
    ea.k_exact = static_cast<const uint8_t*>(p.ex.k_exact) + static_cast<int64_t>(i0) * 128 * esz;
    ea.v_exact = static_cast<const uint8_t*>(p.ex.v_exact) + static_cast<int64_t>(i0) * 128 * esz;
    if (ea.exact_pos != nullptr) ea.exact_pos += i0;
    float* smem = reinterpret_cast<float*>(&stage_all[0][0][0]);
    float* sl = smem;                                             // [kQExRows]
    float* red = smem + kQExRows;                                 // [4]
    float4* part_o = reinterpret_cast<float4*>(smem + kQExRows + 16);   // [8][32]
    float me, le;
    float4 oe;
    const int c4 = tid % 32, part = tid / 32;
    exact_partial<DT, 128>(ea, 0, hq, t, h, sl, red, me, le, oe, c4, part);
    part_o[part * 32 + c4] = oe;
    __syncthreads();
    const int64_t pr = (static_cast<int64_t>(h) * p.S_ex + eb) * R + r;
    if (tid < 128) {
      float O = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float4 v = part_o[k * 32 + (tid >> 2)];
        O += (tid & 3) == 0 ? v.x : (tid & 3) == 1 ? v.y : (tid & 3) == 2 ? v.z : v.w;
      }
      p.ex_o[pr * 128 + tid] = O;
    }
    if (tid == 0) {
      p.ex_m[pr] = me;
      p.ex_l[pr] = le;
    }
    return;
  }
  // ---- coded workgroup: head h, split sidx ----
  const int h = blockIdx.x / p.S, sidx = blockIdx.x % p.S;
  uint8_t* stK = &stage_all[wave][0][0];                         // key rows, then value rows
  uint8_t* stV = stK;
  float* pch = pch_all[wave];
  float* accw = acc_all[wave];
  qcfloat* qtc = (qcfloat*)(p.qt + static_cast<int64_t>(h) * p.Rk * R);
  for (int i = tid; i < p.n_levels; i += kQThreads) {
    const float x = p.levels[i];
    const _Float16 hi = static_cast<_Float16>(x);
    const _Float16 lo = static_cast<_Float16>(x - static_cast<float>(hi));
    lv[i] = x;
    lvp[i] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hi)) |
             (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, lo)) << 16);
  }
  for (int i = lane; i < R * kQRowCoef; i += 64) accw[i] = 0.0f;
  if (tid == 0) next_chunk = p.bounds[sidx];
  __syncthreads();
  qcint* ks = (qcint*)p.slots;                                    // scalar loads: wave-uniform indices
  qcint* vs = ks + kQSlots * kQSlotInts;
  const int nks = p.nslots_k, nvs = p.nslots_v;
  float qmu[R];
#pragma unroll
  for (int r = 0; r < R; ++r) qmu[r] = r < p.R_real ? p.qmu[h * R + r] : 0.0f;
  float m_run[R], l_lane[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    m_run[r] = -INFINITY;
    l_lane[r] = 0.0f;
  }
  const int c_hi = p.bounds[sidx + 1];
  const uint16_t* rk = p.rho_k + static_cast<int64_t>(h) * p.n_c;
  const uint16_t* rvv = p.rho_v + static_cast<int64_t>(h) * p.n_c;
  // chunks are claimed one at a time (their costs differ: early tokens own more steps), so the
  // wavefronts of the split finish together
  for (;;) {
    int ch = 0;
    if (lane == 0) ch = atomicAdd(&next_chunk, 1);
    ch = __builtin_amdgcn_readfirstlane(ch);
    if (ch >= c_hi) break;
    const int j0 = ch * kQChunk;
    const int tok = j0 + lane;
    const bool valid = tok < p.n_c;
    // ---- every key row of the chunk's owned steps into LDS at once ----
    for (int j = 0; j < nks;) {
      qcint* sl = ks + j * kQSlotInts;
      if (sl[1] <= j0) break;                                     // steps own prefixes: n_s never grows
      dma_step(p.kcodes, sl[0], sl[1], sl[2], h, tok, stK + j * 256);
      j += sl[2] / 4;
    }
    const float rkj = valid ? f16_to_f32(rk[tok]) : 0.0f;
    const float rvj = valid ? f16_to_f32(rvv[tok]) : 0.0f;
    __builtin_amdgcn_s_waitcnt(0);                                // the wavefront's LDS DMA has landed
    // ---- scores ----
    float sc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) sc[r] = 0.0f;
    for (int j = 0; j < nks;) {
      qcint* sl = ks + j * kQSlotInts;
      const int ns = sl[1], nb = sl[2];
      if (ns <= j0) break;
      if (tok < ns) {                                             // code 0 is a level, not nothing
        switch (sl[4]) {
          case 1: score_step<R, 1>(stK + j * 256, nb, sl[3], sl[5], lane, lv, qtc, sc); break;
          case 2: score_step<R, 2>(stK + j * 256, nb, sl[3], sl[5], lane, lv, qtc, sc); break;
          case 4: score_step<R, 4>(stK + j * 256, nb, sl[3], sl[5], lane, lv, qtc, sc); break;
          default: score_step<R, 8>(stK + j * 256, nb, sl[3], sl[5], lane, lv, qtc, sc); break;
        }
      }
      j += nb / 4;
    }
    // ---- logits (log2 units), lazy online softmax ----
    float pv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float s = valid ? __builtin_fmaf(sc[r], rkj, qmu[r]) : -INFINITY;
      const float cm = wave_max(s);
      if (cm > m_run[r] + kQLazy) {                               // wave-uniform
        const float mn = fmaxf(m_run[r], cm);
        const float alpha = __builtin_amdgcn_exp2f(m_run[r] - mn);
        l_lane[r] *= alpha;
        for (int i = lane; i < p.Rv; i += 64) accw[r * kQRowCoef + i] *= alpha;
        m_run[r] = mn;
      }
      const float pr = valid ? __builtin_amdgcn_exp2f(s - m_run[r]) : 0.0f;
      l_lane[r] += pr;
      pv[r] = pr * rvj;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) pch[lane * R + r] = pv[r];
    // ---- the value rows into the same staging area (key rows consumed) ----
    wave_lds_fence();
    for (int j = 0; j < nvs;) {
      qcint* sl = vs + j * kQSlotInts;
      if (sl[1] <= j0) break;
      dma_step(p.vcodes, sl[0], sl[1], sl[2], h, tok, stV + j * 256);
      j += sl[2] / 4;
    }
    __builtin_amdgcn_s_waitcnt(0);
    // ---- values: the chunk's probabilities as the A operand (rows r = lane % 16, fp16 hi + lo),
    // then every owned step on the matrix cores ----
    half8 Ah[2], Al[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = lane & 15;
        const float x = r < R ? pch[(32 * kb + (lane >> 4) + 4 * i) * R + (r < R ? r : 0)] : 0.0f;
        const _Float16 hi = static_cast<_Float16>(x);
        Ah[kb][i] = hi;
        Al[kb][i] = static_cast<_Float16>(x - static_cast<float>(hi));
      }
    for (int j = 0; j < nvs;) {
      qcint* sl = vs + j * kQSlotInts;
      const int ns = sl[1], nb = sl[2];
      if (ns <= j0) break;
      switch (sl[4]) {
        case 1: value_step_mfma<R, 1>(stV + j * 256, nb, sl[3], sl[5], ns, j0, lvp, Ah, Al, accw, lane); break;
        case 2: value_step_mfma<R, 2>(stV + j * 256, nb, sl[3], sl[5], ns, j0, lvp, Ah, Al, accw, lane); break;
        case 4: value_step_mfma<R, 4>(stV + j * 256, nb, sl[3], sl[5], ns, j0, lvp, Ah, Al, accw, lane); break;
        default: value_step_mfma<R, 8>(stV + j * 256, nb, sl[3], sl[5], ns, j0, lvp, Ah, Al, accw, lane); break;
      }
      j += nb / 4;
    }
    wave_lds_fence();                                             // staging, pch, accw of this chunk done
  }
  // ---- epilogue: the four wavefronts' (m, l, acc) combined, lifted by T_V into this split's
  // output partial (the exact-row partials' form, so the shared row merge combines them) ----
  float* mw = &pch_all[0][0];                                     // [wave][R] maxima, then [wave][R] sums, then [R] M, [R] L
  float l_w[R];
#pragma unroll
  for (int r = 0; r < R; ++r) l_w[r] = wave_sum(l_lane[r]);
  __syncthreads();                                                // every wavefront's pch / accw / staging done
  // the head's T_V^T (fp16, Rv x 128) into the free staging area, one LDS DMA burst
  {
    uint8_t* tdst = &stage_all[0][0][0];
    const uint8_t* tsrc = reinterpret_cast<const uint8_t*>(p.tvt + static_cast<int64_t>(h) * p.Rv * 128);
    const int pieces = p.Rv * 128 * 2 / 1024;                     // 1 KB per wavefront instruction
    for (int q = wave; q < pieces; q += kQWaves)
      __builtin_amdgcn_global_load_lds((qgvoid*)(tsrc + q * 1024 + lane * 16), (qlvoid*)(tdst + q * 1024), 16, 0, 0);
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      mw[wave * R + r] = m_run[r];
      mw[kQWaves * R + wave * R + r] = l_w[r];
    }
  }
  __syncthreads();
  float* accc = mw + 16 * R;                                      // [R][kQRowCoef] combined coefficients (past mw's 10 R)
  for (int i = tid; i < R * p.Rv; i += kQThreads) {
    const int r = i / p.Rv, c = i % p.Rv;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kQWaves; ++w) M = fmaxf(M, mw[w * R + r]);
    float a = 0.0f, L = 0.0f;
#pragma unroll
    for (int w = 0; w < kQWaves; ++w) {
      const float mwr = mw[w * R + r];
      const float sc = mwr == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mwr - M);
      a = __builtin_fmaf(sc, acc_all[w][r * kQRowCoef + c], a);
      L = __builtin_fmaf(sc, mw[kQWaves * R + w * R + r], L);
    }
    accc[r * kQRowCoef + c] = a;
    if (c == 0) {
      mw[2 * kQWaves * R + r] = M;
      mw[2 * kQWaves * R + R + r] = L;
    }
  }
  __builtin_amdgcn_s_waitcnt(0);                                  // this wavefront's share of T_V^T landed
  __syncthreads();
  const int64_t pr0 = (static_cast<int64_t>(h) * p.S + sidx) * R;
  if (tid < 128) {                                                // thread = output channel
    const int c = tid;
    float o[R];
    const float mu = p.muv[static_cast<int64_t>(h) * 128 + c];
#pragma unroll
    for (int r = 0; r < R; ++r) o[r] = mw[2 * kQWaves * R + R + r] * mu;
    const uint16_t* tcol = reinterpret_cast<const uint16_t*>(&stage_all[0][0][0]) + c;
#pragma unroll 8
    for (int k = 0; k < p.Rv; ++k) {
      const float t = f16_to_f32(tcol[k * 128]);
#pragma unroll
      for (int r = 0; r < R; ++r) o[r] = __builtin_fmaf(accc[r * kQRowCoef + k], t, o[r]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) p.ws_o[(pr0 + r) * 128 + c] = o[r];
  }
  if (tid < R) {
    p.ws_m[pr0 + tid] = mw[2 * kQWaves * R + tid];
    p.ws_l[pr0 + tid] = mw[2 * kQWaves * R + R + tid];
  }
}

inline int64_t quasar_ws_floats(int64_t Hkv, int R, int64_t Rk, int64_t S, int64_t S_ex) {
  return Hkv * R * Rk + Hkv * R + 2 * Hkv * S * R + Hkv * S * R * 128 + 2 * Hkv * S_ex * R + Hkv * S_ex * R * 128;
}

// exact rows: in the merge up to kQExRows of them (one key and one value round trip there), else
// workgroups of kQExRows rows in the split launch, overlapping the coded work
inline int64_t quasar_exact_blocks(int64_t n_exact) {
  return n_exact <= kQExRows ? 0 : (n_exact + kQExRows - 1) / kQExRows;
}

}  // namespace
}  // namespace kvq

using namespace kvq;

extern "C" int kvq_quasar_plan(const int32_t* k_table, int k_steps, const int32_t* v_table, int v_steps, int64_t n_c,
                               int64_t Hkv, int max_splits, int32_t* bounds, int32_t* n_splits, int32_t* slots,
                               int32_t* n_slots) {
  KVQ_REQUIRE(n_c >= 0 && Hkv > 0 && max_splits > 0 && bounds != nullptr && n_splits != nullptr && slots != nullptr &&
                  n_slots != nullptr,
              "kvq_quasar_plan: bad arguments");
  KVQ_REQUIRE(k_steps >= 0 && v_steps >= 0 && (k_table != nullptr || k_steps == 0) && (v_table != nullptr || v_steps == 0),
              "kvq_quasar_plan: bad step tables");
  auto count_slots = [](const int32_t* tab, int steps) {
    int64_t n = 0;
    for (int s = 0; s < steps; ++s) n += tab[7 * s + 2] / 4;
    return n;
  };
  KVQ_REQUIRE(count_slots(k_table, k_steps) <= kQSlots && count_slots(v_table, v_steps) <= kQSlots,
              "kvq_quasar_plan: at most %d code bytes per token and side", 4 * kQSlots);
  for (int side = 0; side < 2; ++side) {
    const int32_t* tab = side ? v_table : k_table;
    const int steps = side ? v_steps : k_steps;
    int n = 0, prev = 0x7fffffff;
    for (int s = 0; s < steps; ++s) {
      const int32_t* row = tab + 7 * s;
      const int bits = row[5], nb = row[2];
      KVQ_REQUIRE((bits == 1 || bits == 2 || bits == 4 || bits == 8) && nb >= 4 && nb <= 64 && (nb & (nb - 1)) == 0 &&
                      nb * 8 == row[4] * bits && row[0] % 4 == 0 && row[1] >= 0 && row[1] <= n_c && row[1] <= prev,
                  "kvq_quasar_plan: step %d of side %d is not a decodable step", s, side);
      prev = row[1];
      for (int dw = 0; dw < nb / 4; ++dw, ++n) {
        int32_t* sl = slots + (side * kQSlots + n) * kQSlotInts;
        sl[0] = row[0] + 4 * dw;
        sl[1] = row[1];
        sl[2] = nb;
        sl[3] = row[3] + 4 * dw * (8 / bits);
        sl[4] = bits;
        sl[5] = row[6];
        sl[6] = s;
        sl[7] = 0;
      }
    }
    n_slots[side] = n;
  }
  const int64_t n_chunks = (n_c + kQChunk - 1) / kQChunk;
  if (n_chunks == 0) {
    bounds[0] = bounds[1] = 0;
    *n_splits = 1;
    return KVQ_OK;
  }
  // cost of chunk c: coefficients the chunk's tokens own over both sides (FMAs per query row)
  // plus a fixed per-chunk part (softmax, the row staging and its waits), measured best at 96
  // coefficients per token (6144 per chunk; 2048 / 3072 / 4096 / 8192: 74.2 / 65.7 / 64.7 / 68.3 us
  // of the split at the F2 workload against 64.5)
  std::vector<double> cost(static_cast<size_t>(n_chunks), 6144.0);
  auto add = [&](const int32_t* tab, int steps) {
    for (int s = 0; s < steps; ++s) {
      const int64_t ns = tab[7 * s + 1], w = tab[7 * s + 4];
      for (int64_t c = 0; c * kQChunk < ns && c < n_chunks; ++c)
        cost[static_cast<size_t>(c)] += static_cast<double>(std::min<int64_t>(kQChunk, ns - c * kQChunk)) * w;
    }
  };
  add(k_table, k_steps);
  add(v_table, v_steps);
  double total = 0.0, c_max = 0.0;
  for (double c : cost) {
    total += c;
    c_max = std::max(c_max, c);
  }
  // one resident round of workgroups over the heads (3 per CU), splits of 4 chunks on average at least
  const int64_t S = std::max<int64_t>(1, std::min<int64_t>({static_cast<int64_t>(max_splits), (768 + Hkv - 1) / Hkv,
                                                             (n_chunks + 3) / 4}));
  // The wavefronts of a split claim its chunks in order, each taking the next when it is free, so a
  // split's time is the makespan of that list schedule, and one full early chunk costs several
  // times a split's average share per wavefront: splits of equal cost would hand some wavefronts
  // two heavy chunks.  Contiguous splits are cut greedily under a makespan bound B (a split closes
  // before the chunk that would push its schedule past B), and B is the least bound (bisection)
  // that needs at most S splits.
  auto cut = [&](double B, int32_t* out) -> int64_t {
    int64_t ns = 0;
    int64_t c = 0;
    if (out != nullptr) out[0] = 0;
    while (c < n_chunks) {
      double fin[kQWaves] = {};
      double span = 0.0;
      int64_t e = c;
      for (; e < n_chunks; ++e) {
        int w = 0;
        for (int i = 1; i < kQWaves; ++i)
          if (fin[i] < fin[w]) w = i;
        const double f = fin[w] + cost[static_cast<size_t>(e)];
        if (e > c && std::max(span, f) > B) break;
        fin[w] = f;
        span = std::max(span, f);
      }
      ++ns;
      c = e;
      if (out != nullptr) out[ns] = static_cast<int32_t>(c);
    }
    return ns;
  };
  double lo = c_max, hi = total;
  for (int it = 0; it < 60 && hi - lo > 1e-6 * total; ++it) {
    const double mid = 0.5 * (lo + hi);
    if (cut(mid, nullptr) <= S) hi = mid;
    else lo = mid;
  }
  *n_splits = static_cast<int32_t>(cut(hi, bounds));
  return KVQ_OK;
}

extern "C" int64_t kvq_quasar_decode_workspace(int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d, int64_t R_k,
                                               int64_t n_exact, int splits) {
  if (Hkv <= 0 || Hq % Hkv != 0 || Tq <= 0 || d != 128 || R_k <= 0 || R_k > kQMaxR || n_exact < 0 || splits <= 0)
    return -1;
  const int64_t R = pow2_rows(Hq / Hkv * Tq);
  if (R > 8) return -1;
  return quasar_ws_floats(Hkv, static_cast<int>(R), R_k, splits, quasar_exact_blocks(n_exact));
}

extern "C" int kvq_quasar_decode(const void* q, int q_dtype, int64_t q_sh, int64_t q_st, int64_t Hq, int64_t Hkv,
                                 int64_t Tq, int64_t d, float scaling, const void* k_exact, const void* v_exact,
                                 int64_t cap_e, int64_t n_exact, const int64_t* exact_pos, const int64_t* q_pos,
                                 const uint8_t* k_codes, int64_t k_bytes, const uint8_t* v_codes, int64_t v_bytes,
                                 const int32_t* slots, int nslots_k,
                                 int nslots_v, const float* levels, int n_levels,
                                 const uint16_t* rho_k, const uint16_t* rho_v, int64_t n_c, const float* T_k,
                                 const uint16_t* T_v, int64_t R_k, int64_t R_v, const float* mu_k, const float* mu_v,
                                 const int32_t* bounds, int splits, void* out, float* workspace,
                                 int64_t workspace_floats, int phases, void* stream) {
  KVQ_REQUIRE(q != nullptr && out != nullptr && workspace != nullptr, "kvq_quasar_decode: null pointer");
  KVQ_REQUIRE(phases >= 1 && phases <= 7, "kvq_quasar_decode: phases is a mask of 1 (prologue), 2 (split), 4 (merge)");
  KVQ_REQUIRE(valid_dtype(q_dtype), "kvq_quasar_decode: bad dtype %d", q_dtype);
  KVQ_REQUIRE(d == 128, "kvq_quasar_decode: head_dim must be 128");
  KVQ_REQUIRE(Hkv > 0 && Hq % Hkv == 0 && Tq > 0, "kvq_quasar_decode: bad head counts");
  const int64_t R_real = Hq / Hkv * Tq;
  KVQ_REQUIRE(R_real <= 8, "kvq_quasar_decode: rep x Tq must be <= 8");
  KVQ_REQUIRE(n_exact >= 0 && n_exact <= cap_e && (n_exact == 0 || (k_exact != nullptr && v_exact != nullptr)),
              "kvq_quasar_decode: bad exact rows");
  KVQ_REQUIRE(n_exact + n_c > 0, "kvq_quasar_decode: nothing to attend");
  KVQ_REQUIRE((exact_pos == nullptr) == (q_pos == nullptr), "kvq_quasar_decode: exact_pos and q_pos go together");
  KVQ_REQUIRE(n_c >= 0 && n_c < (1LL << 31), "kvq_quasar_decode: bad n_c");
  if (n_c > 0) {
    KVQ_REQUIRE(k_codes != nullptr && v_codes != nullptr && slots != nullptr && levels != nullptr &&
                    rho_k != nullptr && rho_v != nullptr && T_k != nullptr && T_v != nullptr && mu_k != nullptr &&
                    mu_v != nullptr && bounds != nullptr,
                "kvq_quasar_decode: null code pointer");
    KVQ_REQUIRE(nslots_k > 0 && nslots_k <= kQSlots && nslots_v > 0 && nslots_v <= kQSlots && splits > 0,
                "kvq_quasar_decode: slot counts must be in [1, %d], splits > 0", kQSlots);
    KVQ_REQUIRE(R_k % 4 == 0 && R_v % 4 == 0, "kvq_quasar_decode: R_k, R_v must be multiples of 4");
    KVQ_REQUIRE(k_bytes > 0 && k_bytes < (1LL << 31) && v_bytes > 0 && v_bytes < (1LL << 31),
                "kvq_quasar_decode: code buffers must hold 1 byte .. 2 GiB");
    KVQ_REQUIRE(R_k > 0 && R_k <= d && R_v > 0 && R_v <= d, "kvq_quasar_decode: R_k, R_v must be in [1, d]");
    KVQ_REQUIRE(n_levels > 0 && n_levels <= kQMaxLevels, "kvq_quasar_decode: at most %d levels", kQMaxLevels);
  }
  const int R = pow2_rows(R_real);
  const int S = n_c > 0 ? splits : 0;
  const int64_t S_ex = quasar_exact_blocks(n_exact);
  const int64_t need = quasar_ws_floats(Hkv, R, std::max<int64_t>(R_k, 1), std::max(S, 1), S_ex);
  KVQ_REQUIRE(workspace_floats >= need, "kvq_quasar_decode: workspace of %lld floats, need %lld",
              static_cast<long long>(workspace_floats), static_cast<long long>(need));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const float qscale = scaling * 1.4426950408889634f;
  float* qt = workspace;
  float* qmu = qt + Hkv * R * std::max<int64_t>(R_k, 1);
  float* ws_m = qmu + Hkv * R;
  float* ws_l = ws_m + Hkv * std::max(S, 1) * R;
  float* ws_o = ws_l + Hkv * std::max(S, 1) * R;
  float* ex_m = ws_o + Hkv * std::max(S, 1) * R * 128;
  float* ex_l = ex_m + Hkv * S_ex * R;
  float* ex_o = ex_l + Hkv * S_ex * R;
  if (n_c > 0 && (phases & 1)) {
    KVQ_DISPATCH_DTYPE(q_dtype, hipLaunchKernelGGL((quasar_prologue<DT_>), dim3(static_cast<unsigned>(Hkv * R)), dim3(256), 0,
                                                   st, q, q_sh, q_st, static_cast<int>(Hq / Hkv), static_cast<int>(Tq), R,
                                                   static_cast<int>(R_real), static_cast<int>(d), T_k, mu_k,
                                                   static_cast<int>(R_k), qscale, qt, qmu));
    KVQ_LAUNCH_CHECK("kvq_quasar_decode(prologue)");
  }
  QuasarParams p{};
  p.Hkv = static_cast<int>(Hkv);
  p.Hq = static_cast<int>(Hq);
  p.Tq = static_cast<int>(Tq);
  p.rep = static_cast<int>(Hq / Hkv);
  p.R_real = static_cast<int>(R_real);
  p.n_c = n_c;
  p.n_chunks = static_cast<int>((n_c + kQChunk - 1) / kQChunk);
  p.qt = qt;
  p.qmu = qmu;
  p.Rk = static_cast<int>(std::max<int64_t>(R_k, 1));
  p.Rv = static_cast<int>(std::max<int64_t>(R_v, 1));
  p.kcodes = k_codes;
  p.vcodes = v_codes;
  p.kbytes = static_cast<uint32_t>(k_bytes);
  p.vbytes = static_cast<uint32_t>(v_bytes);
  p.slots = slots;
  p.nslots_k = nslots_k;
  p.nslots_v = nslots_v;
  p.levels = levels;
  p.n_levels = n_levels;
  p.rho_k = rho_k;
  p.rho_v = rho_v;
  p.bounds = bounds;
  p.S = S;
  p.ws_m = ws_m;
  p.ws_l = ws_l;
  p.ws_o = ws_o;
  p.tvt = T_v;
  p.muv = mu_v;
  p.ex = ExactArgs{q, 0, q_sh, q_st, qscale, k_exact, v_exact, cap_e, static_cast<int>(n_exact), exact_pos, q_pos};
  p.S_ex = static_cast<int>(S_ex);
  p.ex_m = ex_m;
  p.ex_l = ex_l;
  p.ex_o = ex_o;
  const int64_t n_wg = Hkv * S + Hkv * R_real * S_ex;
  const size_t lds = 0;                                           // static LDS (stage, coefficients, levels)
#define KVQ_QSPLIT(R_, DT_) hipLaunchKernelGGL((quasar_split<R_, DT_>), dim3(static_cast<unsigned>(n_wg)), dim3(kQThreads), lds, st, p)
#define KVQ_QSPLIT_R(DT_)                  \
  switch (R) {                             \
    case 1: KVQ_QSPLIT(1, DT_); break;     \
    case 2: KVQ_QSPLIT(2, DT_); break;     \
    case 4: KVQ_QSPLIT(4, DT_); break;     \
    default: KVQ_QSPLIT(8, DT_); break;    \
  }
  if ((phases & 2) && n_wg > 0) {                               // nothing to split: the merge does it all
    KVQ_DISPATCH_DTYPE(q_dtype, KVQ_QSPLIT_R(DT_));
    KVQ_LAUNCH_CHECK("kvq_quasar_decode(split)");
  }
#undef KVQ_QSPLIT_R
#undef KVQ_QSPLIT
  if (phases & 4) {                                              // the shared row merge (partials.hpp)
    MergeArgs ma{};
    ma.ws_o = ws_o;
    ma.ws_m = ws_m;
    ma.ws_l = ws_l;
    ma.S = S;
    ma.ex_o = ex_o;
    ma.ex_m = ex_m;
    ma.ex_l = ex_l;
    ma.S_ex = static_cast<int>(S_ex);
    ma.Hq = static_cast<int>(Hq);
    ma.Hkv = static_cast<int>(Hkv);
    ma.Tq = static_cast<int>(Tq);
    ma.rep = p.rep;
    ma.R_real = static_cast<int>(R_real);
    ma.out = out;
    if (S_ex == 0 && n_exact > 0) ma.ex = p.ex;                    // short exact part: attended in the merge
    const int rc = launch_merge_rows(ma, R, static_cast<int>(Hkv), q_dtype, st);
    if (rc != KVQ_OK) return rc;
  }
  return KVQ_OK;
}
