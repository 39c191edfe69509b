// Fused quantise + pack append of one decode token per sequence (streaming KIVI window).
//
// State of one layer: a ring of W exact rows (row of position p in slot p % W) and the packed
// cache (key codes in pack_codes rows, value codes in 32-token tiles, fp16 metadata).  Appending
// the token at position `pos`:
//   1. if pos >= W, token o = pos - W leaves the window: its value row is quantised per token
//      (channel groups of group_v) into the value tile and tile metadata;
//   2. if additionally o % group_k == 0, key group o / group_k (tokens o .. o+group_k-1, all in
//      the ring because W >= group_k) is quantised per channel into key rows and key metadata;
//   3. the new key/value rows are written into slot pos % W.
// Thread c owns channel c of every row it reads and writes, so the write of step 3 needs no
// barrier after the reads of steps 1-2; every independent load is issued first.
// Codes and metadata are bit-identical to kivi_quant over the whole sequence (STRATA_KV.py:
// 826-856): a key group is quantised only when complete, a value row only needs itself.  This is
// the streaming restatement of KIVIMethod's window rule (a token is read exact until it leaves
// the window, then from its codes; STRATA_KV.py:806-822).
#include "common.hpp"

namespace kvq {
namespace {

constexpr float kF16Max = 65504.0f;
constexpr float kMinScale = 5.9604644775390625e-08f;

__device__ __forceinline__ float as_stored(float x) {
  x = fminf(fmaxf(x, -kF16Max), kF16Max);
  return f16_to_f32(f32_to_f16(x));
}

__device__ __forceinline__ int quant_code(float x, float lo, float sc, int qmax) {
  float t = rintf(__fdiv_rn(__fsub_rn(x, lo), sc));
  t = fminf(fmaxf(t, 0.0f), static_cast<float>(qmax));
  return static_cast<int>(t);
}

// nibble (bit offset / 4) of the tile word that holds slot j (inverse of the tile's slot order)
__device__ __constant__ int kNibbleOfSlot[8] = {0, 4, 1, 5, 2, 6, 3, 7};

template <int DT>
__global__ void kivi_append_kernel(const void* __restrict__ k_new, const void* __restrict__ v_new,
                                   int64_t k_sb, int64_t k_sh, int64_t v_sb, int64_t v_sh, int Hkv, int d,
                                   int64_t pos, void* __restrict__ k_ring, void* __restrict__ v_ring,
                                   int64_t W, uint8_t* __restrict__ kc, uint16_t* __restrict__ k_lo,
                                   uint16_t* __restrict__ k_sc, uint8_t* __restrict__ vc,
                                   uint16_t* __restrict__ vmeta, int64_t cap_t, int group_k, int group_v) {
  extern __shared__ float red[];                  // [d] values of the leaving row
  const int bh = blockIdx.x;
  const int b = bh / Hkv, h = bh % Hkv;
  const int c = threadIdx.x;                      // thread c owns channel c of every row it touches
  const int qmax = 15;
  const int64_t ring_bh = static_cast<int64_t>(bh) * W * d;
  const int64_t slot = pos % W;                   // the new row's slot = the leaving row's slot
  const bool leaving = pos >= W;
  const int64_t o = pos - W;                      // token leaving the window (when leaving)
  // ---- every independent load first: the new rows, the leaving value row, its tile word ----
  const float kv = load_as_f32<DT>(k_new, static_cast<int64_t>(b) * k_sb + static_cast<int64_t>(h) * k_sh + c);
  const float vv = load_as_f32<DT>(v_new, static_cast<int64_t>(b) * v_sb + static_cast<int64_t>(h) * v_sh + c);
  const int64_t chunk = leaving ? o / 32 : 0;
  const int u = leaving ? static_cast<int>(o % 32) : 0;
  const int g = (u % 16) / 4, j = 4 * (u / 16) + (u % 4);
  const int blk = c / 16;
  uint32_t* word = reinterpret_cast<uint32_t*>(vc + static_cast<int64_t>(bh) * cap_t * (d / 2) + chunk * 16 * d) +
                   (blk / 4) * 256 + (16 * g + c % 16) * 4 + (blk % 4);
  float x = 0.0f;
  uint32_t wold = 0u;
  if (leaving) {
    x = load_as_f32<DT>(v_ring, ring_bh + slot * d + c);
    wold = *word;
  }
  if (leaving) {
    // ---- value row of token o, per channel group ----
    red[c] = x;
    __syncthreads();
    const int gc = c / group_v;
    float mn = INFINITY, mx = -INFINITY;
    for (int i = gc * group_v; i < (gc + 1) * group_v; ++i) {
      mn = fminf(mn, red[i]);
      mx = fmaxf(mx, red[i]);
    }
    const float lo = as_stored(mn);
    const float sc = fmaxf(as_stored(__fdiv_rn(__fsub_rn(mx, lo), static_cast<float>(qmax))), kMinScale);
    const int code = quant_code(x, lo, sc, qmax);
    const int sh = 4 * kNibbleOfSlot[j];
    *word = (wold & ~(0xfu << sh)) | (static_cast<uint32_t>(code) << sh);
    const int ngv = d / group_v;
    if (c % group_v == 0) {
      uint16_t* vm = vmeta + ((static_cast<int64_t>(bh) * (cap_t / 32) + chunk) * ngv + gc) * 64 + (8 * g + j) * 2;
      vm[0] = f32_to_f16(sc);
      vm[1] = f32_to_f16(lo);
    }
    // ---- key group starting at token o (every group_k steps): rows o .. o + group_k - 1 ----
    if (o % group_k == 0) {
      constexpr int kB = 16;                      // rows loaded together
      float kmn = INFINITY, kmx = -INFINITY;
      for (int t0 = 0; t0 < group_k; t0 += kB) {
        float kx[kB];
#pragma unroll
        for (int t = 0; t < kB; ++t) kx[t] = load_as_f32<DT>(k_ring, ring_bh + ((o + t0 + t) % W) * d + c);
#pragma unroll
        for (int t = 0; t < kB; ++t) {
          kmn = fminf(kmn, kx[t]);
          kmx = fmaxf(kmx, kx[t]);
        }
      }
      const float klo = as_stored(kmn);
      const float ksc = fmaxf(as_stored(__fdiv_rn(__fsub_rn(kmx, klo), static_cast<float>(qmax))), kMinScale);
      const int64_t mo = static_cast<int64_t>(bh) * (cap_t / group_k) * d + (o / group_k) * d + c;
      k_lo[mo] = f32_to_f16(klo);
      k_sc[mo] = f32_to_f16(ksc);
      uint8_t* rows = kc + static_cast<int64_t>(bh) * cap_t * (d / 2);
      for (int t0 = 0; t0 < group_k; t0 += kB) {
        float kx[kB];
#pragma unroll
        for (int t = 0; t < kB; ++t) kx[t] = load_as_f32<DT>(k_ring, ring_bh + ((o + t0 + t) % W) * d + c);
#pragma unroll
        for (int t = 0; t < kB; ++t) {
          const int kcode = quant_code(kx[t], klo, ksc, qmax);
          // channel c + 1's code (lanes 2i, 2i+1 are a quad-swap pair): byte = c[2i] << 4 | c[2i+1]
          const int other = __builtin_amdgcn_update_dpp(0, kcode, 0xB1, 0xF, 0xF, true);
          if ((c & 1) == 0) rows[(o + t0 + t) * (d / 2) + c / 2] = static_cast<uint8_t>((kcode << 4) | other);
        }
      }
    }
  }
  // ---- the new token into its ring slot (each thread writes the channel it alone has read) ----
  store_from_f32<DT>(k_ring, ring_bh + slot * d + c, kv);
  store_from_f32<DT>(v_ring, ring_bh + slot * d + c, vv);
}

}  // namespace
}  // namespace kvq

using namespace kvq;

extern "C" int kvq_kivi_append(const void* k_new, const void* v_new, int dtype, int64_t k_sb,
                               int64_t k_sh, int64_t v_sb, int64_t v_sh, int64_t B, int64_t Hkv,
                               int64_t d, int64_t pos, void* k_ring, void* v_ring, int64_t W,
                               uint8_t* kc, uint16_t* k_lo, uint16_t* k_sc, uint8_t* vc,
                               uint16_t* vmeta, int64_t cap_t, int group_k, int group_v,
                               void* stream) {
  KVQ_REQUIRE(valid_dtype(dtype), "kvq_kivi_append: bad dtype");
  KVQ_REQUIRE(k_new && v_new && k_ring && v_ring && kc && k_lo && k_sc && vc && vmeta,
              "kvq_kivi_append: null pointer");
  KVQ_REQUIRE(d == 128, "kvq_kivi_append: head_dim must be 128");
  KVQ_REQUIRE(group_k > 0 && group_k % 32 == 0 && W >= group_k, "kvq_kivi_append: need W >= group_k, group_k %% 32 == 0");
  KVQ_REQUIRE(group_v == 32 || group_v == 64 || group_v == 128, "kvq_kivi_append: group_v in {32,64,128}");
  KVQ_REQUIRE(pos >= 0 && cap_t % group_k == 0 && cap_t % 32 == 0, "kvq_kivi_append: bad pos / capacity");
  // token o = pos - W takes packed row o; a key group is written only when o % group_k == 0, and
  // cap_t % group_k == 0, so every o < cap_t keeps its group's rows inside the capacity
  KVQ_REQUIRE(pos < W || pos - W < cap_t, "kvq_kivi_append: packed capacity exhausted");
  KVQ_REQUIRE(B > 0 && Hkv > 0 && B * Hkv < (1LL << 31), "kvq_kivi_append: bad batch/heads");
  hipStream_t s = static_cast<hipStream_t>(stream);
  KVQ_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((kivi_append_kernel<DT_>), dim3(B * Hkv), dim3(d),
                                              d * sizeof(float), s, k_new, v_new, k_sb, k_sh, v_sb, v_sh,
                                              (int)Hkv, (int)d, pos, k_ring, v_ring, W, kc, k_lo, k_sc, vc,
                                              vmeta, cap_t, group_k, group_v));
  KVQ_LAUNCH_CHECK("kvq_kivi_append");
  return KVQ_OK;
}
