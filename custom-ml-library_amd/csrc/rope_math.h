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

#include "mfma_common.h"

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
// channel), rotated in place.  The same operations as rotate_pair, paired up so that each rounding step
// rounds two values with one packed conversion: (x0 c, x1 c), (x1 s, x0 s),
// then (y0, y1) -- the products of two 16-bit values are exact in fp32, and
// rnd(-x1 s) = -rnd(x1 s), so the results are rotate_pair's bit for bit.
template <typename T>
__device__ __forceinline__ unsigned rotate_word(unsigned w, T c, T s, bool inverse) {
#pragma clang fp contract(off)
  typedef float f2v __attribute__((ext_vector_type(2)));
  typedef T t2v __attribute__((ext_vector_type(2)));
  const float fc = static_cast<float>(c);
  const float fs = inverse ? -static_cast<float>(s) : static_cast<float>(s);
  const t2v xv = __builtin_bit_cast(t2v, w);
  const float x0 = static_cast<float>(xv[0]), x1 = static_cast<float>(xv[1]);
  const t2v pc = __builtin_convertvector(f2v{x0 * fc, x1 * fc}, t2v);
  const t2v ps = __builtin_convertvector(f2v{x1 * fs, x0 * fs}, t2v);
  const f2v y{static_cast<float>(pc[0]) - static_cast<float>(ps[0]),
              static_cast<float>(pc[1]) + static_cast<float>(ps[1])};
  return __builtin_bit_cast(unsigned, __builtin_convertvector(y, t2v));
}

// Rotate one 16-byte chunk of a row -- 4 pairs packed in x, pairs p0 .. p0 + 3
// (p0 a multiple of 4) -- by row `row` of the descriptor's [*, R / 2] tables,
// R a multiple of 8 so that a chunk is wholly inside or outside the rotated
// channels.  The table loads are unconditional 8-byte loads (the pair index
// clamped into range, the result selected), so a run of chunks issues all
// its loads before the first use instead of one guarded load at a time.
template <typename T>
__device__ __forceinline__ void rotate_chunk(u32x4 &x, const RopeDesc &r, int64_t row, int p0,
                                             bool inverse) {
  const int half = r.R / 2;
  const int pc = p0 < half ? p0 : half - 4;
  const int64_t at = row * half + pc;
  const u32x2 cw = *reinterpret_cast<const u32x2 *>(static_cast<const T *>(r.cos) + at);
  const u32x2 sw = *reinterpret_cast<const u32x2 *>(static_cast<const T *>(r.sin) + at);
  u32x4 y;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const unsigned c2 = cw[m >> 1], s2 = sw[m >> 1];
    const int sh = (m & 1) * 16;
    const T c = __builtin_bit_cast(T, static_cast<uint16_t>(c2 >> sh));
    const T s = __builtin_bit_cast(T, static_cast<uint16_t>(s2 >> sh));
    y[m] = rotate_word<T>(x[m], c, s, inverse);
  }
  if (p0 < half) x = y;
}

// rotate_chunk over N chunks at once, in two steps, so that a caller can
// put other work (DMA issue) between the table loads and the rotation:
// rope_load_tables issues all 2 N table loads -- x[i] will hold pairs p0[i]
// .. p0[i] + 3 of table row row[i] -- and resolves them (the empty asm
// statements use every loaded value unconditionally: the compiler cannot
// sink a load into the conditional use below it, which would serialise one
// memory latency per chunk); rope_rotate_loaded then rotates from registers.
template <typename T, int N>
__device__ __forceinline__ void rope_load_tables(const RopeDesc &r, const int64_t (&row)[N],
                                                 const int (&p0)[N], u32x2 (&cw)[N], u32x2 (&sw)[N]) {
  const int half = r.R / 2;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int pc = p0[i] < half ? p0[i] : half - 4;
    const int64_t at = row[i] * half + pc;
    cw[i] = *reinterpret_cast<const u32x2 *>(static_cast<const T *>(r.cos) + at);
    sw[i] = *reinterpret_cast<const u32x2 *>(static_cast<const T *>(r.sin) + at);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(cw[i]), "+v"(sw[i]));
}

template <typename T, int N>
__device__ __forceinline__ void rope_rotate_loaded(u32x4 (&x)[N], const u32x2 (&cw)[N], const u32x2 (&sw)[N],
                                                   const int (&p0)[N], int half, bool inverse) {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    u32x4 y;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int sh = (m & 1) * 16;
      const T c = __builtin_bit_cast(T, static_cast<uint16_t>(cw[i][m >> 1] >> sh));
      const T s = __builtin_bit_cast(T, static_cast<uint16_t>(sw[i][m >> 1] >> sh));
      y[m] = rotate_word<T>(x[i][m], c, s, inverse);
    }
    if (p0[i] < half) x[i] = y;
  }
}

template <typename T, int N>
__device__ __forceinline__ void rotate_chunks(u32x4 (&x)[N], const RopeDesc &r, const int64_t (&row)[N],
                                              const int (&p0)[N], bool inverse) {
  u32x2 cw[N], sw[N];
  rope_load_tables<T, N>(r, row, p0, cw, sw);
  rope_rotate_loaded<T, N>(x, cw, sw, p0, r.R / 2, inverse);
}

}  // namespace tsattn
