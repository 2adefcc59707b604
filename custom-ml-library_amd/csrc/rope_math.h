// Interleaved-pair RoPE arithmetic shared by the RoPE kernels and the
// attention kernels that fold the rotation into their prologue / epilogue.
//
// Pair (x0, x1) = channels (2i, 2i+1) rotates by (c, s) = (cos, sin) of its
// angle, both already in the tensor dtype T, with every operation rounded to
// T as the reference's array expressions round it
// (src/tensorsmith/nn/attention.py:281-294):
//   y0 = rnd(rnd(x0 c) + rnd(-x1 s)),  y1 = rnd(rnd(x1 c) + rnd(x0 s));
// `inverse` rotates by the negative angle (the VJP).  For f32 each product
// and sum rounds on its own: contraction into a fused multiply-add (hipcc's
// default for device code) is switched off in these helpers.
#pragma once

#include <type_traits>

#include "tsattn_internal.h"

namespace tsattn {

template <typename T>
__device__ __forceinline__ T rope_mul(T a, T b) {
#pragma clang fp contract(off)
  if constexpr (std::is_same<T, float>::value) return a * b;
  else return static_cast<T>(static_cast<float>(a) * static_cast<float>(b));
}
template <typename T>
__device__ __forceinline__ T rope_add(T a, T b) {
#pragma clang fp contract(off)
  if constexpr (std::is_same<T, float>::value) return a + b;
  else return static_cast<T>(static_cast<float>(a) + static_cast<float>(b));
}

template <typename T>
__device__ __forceinline__ void rotate_pair(T &x0, T &x1, T c, T s, bool inverse) {
  const T sn = inverse ? static_cast<T>(-static_cast<float>(s)) : s;
  const T y0 = rope_add(rope_mul(x0, c), rope_mul(static_cast<T>(-static_cast<float>(x1)), sn));
  const T y1 = rope_add(rope_mul(x1, c), rope_mul(x0, sn));
  x0 = y0;
  x1 = y1;
}

// 16-bit T: one channel pair packed in a 32-bit word (low half = even
// channel), rotated in place.
template <typename T>
__device__ __forceinline__ unsigned rotate_word(unsigned w, T c, T s, bool inverse) {
  T x0 = __builtin_bit_cast(T, static_cast<uint16_t>(w & 0xFFFFu));
  T x1 = __builtin_bit_cast(T, static_cast<uint16_t>(w >> 16));
  rotate_pair(x0, x1, c, s, inverse);
  return static_cast<unsigned>(__builtin_bit_cast(uint16_t, x0)) |
         (static_cast<unsigned>(__builtin_bit_cast(uint16_t, x1)) << 16);
}

// Rotate the N pairs packed in words w[0 .. N) -- pair p0 + m in word m --
// by row `row` of the descriptor's [*, R / 2] tables; pairs at or past R / 2
// pass through (and read no table entry).
template <typename T, int N, typename W>
__device__ __forceinline__ void rotate_words(W &w, const RopeDesc &r, int64_t row, int p0,
                                             bool inverse) {
  const T *cr = static_cast<const T *>(r.cos) + row * (r.R / 2);
  const T *sr = static_cast<const T *>(r.sin) + row * (r.R / 2);
#pragma unroll
  for (int m = 0; m < N; ++m)
    if (2 * (p0 + m) < r.R) w[m] = rotate_word<T>(w[m], cr[p0 + m], sr[p0 + m], inverse);
}

}  // namespace tsattn
