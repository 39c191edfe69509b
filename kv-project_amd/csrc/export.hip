// Wire format of a packed KIVI layer (F4: on-device byte accounting).
//
// The reference measures a KIVI cache by materialising its storage format (payload_bytes,
// STRATA_KV.py:2736-2769): pack_codes of every stored code (2728-2732), the fp16 zero points and
// scales of every group, and the live exact rows as 2-byte values; it must agree with the
// analytic bits (state_bits 773-783: 2 d (bits + 32 / group) per quantised token, 2 d 16 per exact
// row).  Exact rows are written as fp16 whatever their stored dtype, as the reference's payload does.  kvq_kivi_export writes that payload from the decode layout in one launch, section by
// section (each section (B*Hkv)-major, then token, then channel / group):
//   S1 key codes   pack_codes rows (n_q, d bits / 8) per bh
//   S2 key lo      fp16 (n_g, d) per bh, n_g = ceil(n_q / group_k)
//   S3 key scale   fp16 (n_g, d)
//   S4 value codes pack_codes rows (n_q, d bits / 8), read back from the 32-token value tiles
//   S5 value lo    fp16 (n_q, d / group_v), read back from the slot-ordered metadata tiles
//   S6 value scale fp16 (n_q, d / group_v)
//   S7 exact keys  (n_exact, d) fp16 (the reference's .half() of the stored rows), oldest first
//   S8 exact values
// so the payload's byte count is the measured cache size and its bytes are a portable copy.
#include <algorithm>

#include "common.hpp"

namespace kvq {
namespace {

struct ExportArgs {
  const uint8_t* kc;
  const uint16_t* k_lo;
  const uint16_t* k_sc;
  const uint8_t* vc;
  const uint16_t* vmeta;
  int64_t BH, cap_t, n_q, d, n_g, ngv;
  int group_k;
  const uint8_t* k_exact;
  const uint8_t* v_exact;
  int64_t cap_e, n_exact, first_slot;
  int exact_dtype;
  int64_t sec[9];                 // section starts in 2-byte units; sec[8] = total
  uint16_t* out;
};

// code (4 bits) of value channel ch of token t of bh from the value tiles (the inverse of
// kvq_v_tile: token u of a 32-token chunk sits in lane group g = (u % 16) / 4, slot j = 4 (u / 16)
// + u % 4, which the tile word of its channel holds in nibble kNibbleOfSlotE[j])
__device__ __constant__ int kNibbleOfSlotE[8] = {0, 4, 1, 5, 2, 6, 3, 7};

__device__ __forceinline__ uint32_t value_code(const ExportArgs& a, int64_t bh, int64_t t, int ch) {
  const int64_t chunk = t / 32;
  const int u = static_cast<int>(t % 32);
  const int g = (u % 16) / 4, j = 4 * (u / 16) + (u % 4);
  const int blk = ch / 16, lane = 16 * g + ch % 16;
  const uint32_t* tw = reinterpret_cast<const uint32_t*>(a.vc + bh * (a.cap_t * a.d / 2) + chunk * 16 * a.d);
  return (tw[(blk / 4) * 256 + lane * 4 + (blk % 4)] >> (4 * kNibbleOfSlotE[j])) & 0xfu;
}

__global__ __launch_bounds__(256) void kivi_export_kernel(ExportArgs a) {
  const int64_t total = a.sec[8];
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    int s = 0;
#pragma unroll
    for (int k = 1; k < 8; ++k) s += i >= a.sec[k];
    const int64_t e = i - a.sec[s];
    uint16_t v = 0;
    if (s == 0) {                                          // key code bytes 2e, 2e + 1
      const int64_t rb = a.d / 2, b = 2 * e;
      const int64_t bh = b / (a.n_q * rb), t = (b / rb) % a.n_q, o = b % rb;
      v = *reinterpret_cast<const uint16_t*>(a.kc + (bh * a.cap_t + t) * rb + o);
    } else if (s == 1 || s == 2) {                         // key lo / scale element e
      const int64_t bh = e / (a.n_g * a.d), g = (e / a.d) % a.n_g, c = e % a.d;
      v = (s == 1 ? a.k_lo : a.k_sc)[(bh * (a.cap_t / a.group_k) + g) * a.d + c];
    } else if (s == 3) {                                   // value code bytes 2e, 2e + 1: channels 4q .. 4q + 3
      const int64_t rb = a.d / 2, b = 2 * e;
      const int64_t bh = b / (a.n_q * rb), t = (b / rb) % a.n_q;
      const int ch = static_cast<int>(b % rb) * 2;
      const uint32_t b0 = (value_code(a, bh, t, ch) << 4) | value_code(a, bh, t, ch + 1);
      const uint32_t b1 = (value_code(a, bh, t, ch + 2) << 4) | value_code(a, bh, t, ch + 3);
      v = static_cast<uint16_t>(b0 | (b1 << 8));
    } else if (s == 4 || s == 5) {                         // value lo / scale of (t, group gc)
      const int64_t bh = e / (a.n_q * a.ngv), t = (e / a.ngv) % a.n_q, gc = e % a.ngv;
      const int u = static_cast<int>(t % 32);
      const int p = 8 * ((u % 16) / 4) + 4 * (u / 16) + (u % 4);
      const uint16_t* m = a.vmeta + ((bh * (a.cap_t / 32) + t / 32) * a.ngv + gc) * 64 + 2 * p;
      v = m[s == 4 ? 1 : 0];                               // tiles hold (scale, lo) pairs
    } else {                                               // exact element e as fp16 (the reference's .half())
      const int64_t bh = e / (a.n_exact * a.d), r = (e / a.d) % a.n_exact, c = e % a.d;
      const int64_t src = (bh * a.cap_e + (a.first_slot + r) % a.cap_e) * a.d + c;
      const uint8_t* base = s == 6 ? a.k_exact : a.v_exact;
      if (a.exact_dtype == KVQ_F16) v = reinterpret_cast<const uint16_t*>(base)[src];
      else if (a.exact_dtype == KVQ_BF16) v = f32_to_f16(bf16_to_f32(reinterpret_cast<const uint16_t*>(base)[src]));
      else v = f32_to_f16(reinterpret_cast<const float*>(base)[src]);
    }
    a.out[i] = v;
  }
}

void export_sections(int64_t BH, int64_t n_q, int64_t d, int64_t n_g, int64_t ngv, int64_t n_exact, int64_t (&sec)[9]) {
  const int64_t sz[8] = {BH * n_q * d / 4, BH * n_g * d, BH * n_g * d, BH * n_q * d / 4, BH * n_q * ngv, BH * n_q * ngv,
                         BH * n_exact * d, BH * n_exact * d};
  sec[0] = 0;
  for (int k = 0; k < 8; ++k) sec[k + 1] = sec[k] + sz[k];
}

}  // namespace
}  // namespace kvq

using namespace kvq;

extern "C" int64_t kvq_kivi_payload_bytes(int64_t BH, int64_t n_q, int64_t d, int group_k, int group_v, int64_t n_exact,
                                          int exact_dtype) {
  if (BH < 0 || n_q < 0 || d != 128 || group_k <= 0 || group_v <= 0 || d % group_v || n_exact < 0 ||
      !valid_dtype(exact_dtype))
    return -1;
  int64_t sec[9];
  export_sections(BH, n_q, d, (n_q + group_k - 1) / group_k, d / group_v, n_exact, sec);
  return 2 * sec[8];
}

extern "C" int kvq_kivi_export(const uint8_t* kc, const uint16_t* k_lo, const uint16_t* k_sc, const uint8_t* vc,
                               const uint16_t* vmeta, int64_t BH, int64_t cap_t, int64_t n_q, int64_t d, int group_k,
                               int group_v, const void* k_exact, const void* v_exact, int exact_dtype, int64_t cap_e,
                               int64_t n_exact, int64_t first_slot, uint8_t* out, int64_t out_bytes, void* stream) {
  KVQ_REQUIRE(d == 128, "kvq_kivi_export: head_dim must be 128 (4-bit decode layout)");
  KVQ_REQUIRE(BH >= 0 && n_q >= 0 && n_q <= cap_t && cap_t % 32 == 0 && group_k > 0 && cap_t % group_k == 0 &&
                  group_v > 0 && d % group_v == 0,
              "kvq_kivi_export: bad cache shape");
  KVQ_REQUIRE(valid_dtype(exact_dtype) && n_exact >= 0 && n_exact <= cap_e && first_slot >= 0 &&
                  (cap_e == 0 || first_slot < cap_e),
              "kvq_kivi_export: bad exact rows");
  KVQ_REQUIRE(out != nullptr && reinterpret_cast<uintptr_t>(out) % 2 == 0, "kvq_kivi_export: out must be 2-byte aligned");
  KVQ_REQUIRE((n_q == 0 || (kc && k_lo && k_sc && vc && vmeta)) && (n_exact == 0 || (k_exact && v_exact)),
              "kvq_kivi_export: null pointer");
  ExportArgs a{};
  a.kc = kc;
  a.k_lo = k_lo;
  a.k_sc = k_sc;
  a.vc = vc;
  a.vmeta = vmeta;
  a.BH = BH;
  a.cap_t = cap_t;
  a.n_q = n_q;
  a.d = d;
  a.n_g = (n_q + group_k - 1) / group_k;
  a.ngv = d / group_v;
  a.group_k = group_k;
  a.k_exact = static_cast<const uint8_t*>(k_exact);
  a.v_exact = static_cast<const uint8_t*>(v_exact);
  a.cap_e = cap_e > 0 ? cap_e : 1;
  a.n_exact = n_exact;
  a.first_slot = first_slot;
  a.exact_dtype = exact_dtype;
  export_sections(BH, n_q, d, a.n_g, a.ngv, n_exact, a.sec);
  KVQ_REQUIRE(out_bytes >= 2 * a.sec[8], "kvq_kivi_export: out holds %lld bytes, the payload is %lld",
              static_cast<long long>(out_bytes), static_cast<long long>(2 * a.sec[8]));
  a.out = reinterpret_cast<uint16_t*>(out);
  if (a.sec[8] == 0) return KVQ_OK;
  const int64_t blocks = std::min<int64_t>((a.sec[8] + 255) / 256, 4096);
  hipLaunchKernelGGL(kivi_export_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  KVQ_LAUNCH_CHECK("kvq_kivi_export");
  return KVQ_OK;
}
