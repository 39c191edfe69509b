// Code layouts of 2-, 4- and 8-bit codes shared by the width-generic decode kernels (STRATA tiers,
// mixed-width KIVI blocks): planar key rows, value tiles, and the matrix-core operand unpacking.
//
// A 32-token chunk is read by one wavefront; lane l = 16g + n.  The decode's logits leave token
// slot_token(g, j) of the chunk in slot j = 0..7 of lane group g, so the value operands are built
// with the same token order.
//
// Planar key rows (pack_planar, STRATA_KV.py:1171-1182): a row of 128 coordinates at b bits is
// 16b bytes; byte i of the row holds coordinates i + p*(16b) in bits [p*b, (p+1)*b), p < 8/b.
// A lane reads 4b bytes of a row at 4b*g; key_channel() names the coordinate each operand element
// multiplies and code_shift() the power of two its code carries in the fp16 half it is masked in.
//
// Value tiles (one per 32-token chunk, 512*b bytes), lane l = 16g + n, channel 16*blk + n:
//   4 bits: word (blk/4)*256 + l*4 + blk%4; nibble k holds slot kSlotOfNibble4[k]
//   8 bits: word (blk/2)*256 + l*4 + (blk%2)*2 + w; byte k of the lane's 8 holds slot kSlotOfByte8[k]
//   2 bits: word l*4 + blk/2; bits 2k hold slot 2(k&3) + (k>>3) of blk 2(blk/2) + ((k>>2)&1)
#pragma once
#include "common.hpp"
#include "mfma_common.hpp"

namespace kvq {
namespace {

// token of slot j of lane group g within a 32-token chunk
__device__ __forceinline__ int slot_token(int g, int j) { return 16 * (j >> 2) + 4 * g + (j & 3); }

__device__ __constant__ int kSlotOfNibble4[8] = {0, 2, 4, 6, 1, 3, 5, 7};
__device__ __constant__ int kSlotOfByte8[8] = {0, 2, 1, 3, 4, 6, 5, 7};

// Key operand element e of k-step w for lane group g: the coordinate it multiplies.
template <int BITS>
__device__ __forceinline__ int key_channel(int g, int w, int e) {
  if constexpr (BITS == 4) {
    const int byte = 16 * g + 4 * w + ((e >> 2) & 1) + 2 * (e & 1);
    return ((e >> 1) & 1) ? 64 + byte : byte;
  } else if constexpr (BITS == 8) {
    constexpr int kOff[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    return 32 * g + 8 * w + kOff[e];
  } else {
    return 32 * (e >> 1) + 8 * g + 4 * (w >> 1) + 2 * (e & 1) + (w & 1);
  }
}
// log2 of the factor the code of operand element (or value slot) e carries
template <int BITS>
__device__ __forceinline__ int code_shift(int e) {
  if constexpr (BITS == 4) return ((e >> 1) & 1) ? 4 : 0;
  else if constexpr (BITS == 8) return 0;
  else return 2 * (e >> 1);
}
template <int BITS>
constexpr int smax_shift() { return BITS == 4 ? 4 : (BITS == 8 ? 0 : 6); }

// codes masked in place are fp16 subnormals c * 2^(code_shift - 24), exact
__device__ __forceinline__ half8 unpack4(uint32_t w) {
  const uint32_t w8 = w >> 8;
  return as_half8(u32x4{w & 0x000F000Fu, w & 0x00F000F0u, w8 & 0x000F000Fu, w8 & 0x00F000F0u});
}
__device__ __forceinline__ half8 unpack8(uint32_t w0, uint32_t w1) {
  return as_half8(u32x4{w0 & 0x00FF00FFu, (w0 >> 8) & 0x00FF00FFu, w1 & 0x00FF00FFu, (w1 >> 8) & 0x00FF00FFu});
}
__device__ __forceinline__ half8 unpack2(uint32_t x) {
  return as_half8(u32x4{x & 0x00030003u, x & 0x000C000Cu, x & 0x00300030u, x & 0x00C000C0u});
}

// Word w of a value tile of `bits`-bit codes; code_at(slot, g, channel) gives the code.
template <class F>
__device__ __forceinline__ uint32_t vtile_word(int bits, int w, F code_at) {
  uint32_t word = 0;
  if (bits == 4) {
    const int blk = (w / 256) * 4 + (w % 4), l = (w % 256) / 4;
    const int g = l / 16, ch = 16 * blk + (l % 16);
    for (int k = 0; k < 8; ++k) word |= code_at(kSlotOfNibble4[k], g, ch) << (4 * k);
  } else if (bits == 8) {
    const int blk = (w / 256) * 2 + ((w % 4) / 2), l = (w % 256) / 4, half = w % 2;
    const int g = l / 16, ch = 16 * blk + (l % 16);
    for (int k = 0; k < 4; ++k) word |= code_at(kSlotOfByte8[4 * half + k], g, ch) << (8 * k);
  } else {
    const int l = w / 4, bp = w % 4;
    const int g = l / 16;
    for (int k = 0; k < 16; ++k) {
      const int blk = 2 * bp + ((k >> 2) & 1), slot = 2 * (k & 3) + (k >> 3);
      word |= code_at(slot, g, 16 * blk + (l % 16)) << (2 * k);
    }
  }
  return word;
}

}  // namespace
}  // namespace kvq
