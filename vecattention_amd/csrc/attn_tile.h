// Tile geometry and compile-time helpers shared by the MFMA attention
// kernels (attn_mfma.hip, attn_pair.hip): 64-key tiles of K and V rows in LDS
// with an XOR swizzle of their 16-byte chunks.
#pragma once
#include <type_traits>
#include <utility>

#include "lanes.h"
#include "mfma.h"

namespace va {

constexpr int kTileKeys = 64;
constexpr int kMaxSegments = 64;  // key segments of a split selection (a wave's lanes)
constexpr uint32_t kOutOfRange = 0xfffffff0u;  // voffset past every buffer's range
constexpr float kRescaleSlack = 8.f;           // log2 of the largest kept probability

typedef short s16x4_t __attribute__((ext_vector_type(4)));

// f(std::integral_constant<int, i>) for i = 0 .. N-1, in order.
template <typename F, int... I>
__device__ inline void static_for_impl(F& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ inline void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}
template <uint32_t V>
using lds_off = std::integral_constant<uint32_t, V>;

// XOR swizzle of the 16-byte chunks of tile row R.  The LDS serves 256 bytes
// per clock from 64 four-byte banks: a ds_read_b128 is served 16 lanes at a
// time, a ds_read_b64_tr_b16 32 lanes at a time.  Rows R and R + 256 / (2D)
// start on the same bank, so m = (R * 2D / 256) mod NCH numbers the rows of a
// 256-byte bank period, and the swizzle is m with its bits rotated right by
// log2(NCH) - 2:
//  - the K reads (16 consecutive rows, one logical chunk) need m -> swizzle
//    to be a bijection, which any rotation is;
//  - the V^T reads (rows R0 + j, j < 4, R0 % 4 == 0, logical chunks 4i + g,
//    g < 4) need the four rows to differ in swizzle bits 2.., which the
//    rotation gives by moving the low bits of m there.
template <int D>
__device__ inline int chunk_swizzle(int R) {
  constexpr int NCH = D / 8;
  if constexpr (NCH == 16) {
    const int m = R % 16;
    return ((m & 3) << 2) | (m >> 2);
  } else {
    static_assert(NCH == 8, "D must be 64 or 128");
    const int m = (R / 2) % 8;
    return ((m & 1) << 2) | (m >> 1);
  }
}

}  // namespace va
