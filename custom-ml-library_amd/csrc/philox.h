// Counter-based random numbers for attention dropout: Philox4x32-10 (Salmon,
// Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC'11;
// the round constants and known-answer vectors of its Random123 release).
// Word group n (16 dropout words of 16 bits) of a stream with key (K0, K1)
// and counter c is the two blocks Philox4x32-10(t, key K0) and
// Philox4x32-10(t + 1, key K0), t = 2 (c + n) mod 2^64, each of the 128-bit
// counter (lo32 t, hi32 t, lo32 K1, hi32 K1): the four 32-bit outputs of each
// block give 8 words, little-endian.  A round takes two 32 x 32 -> 64-bit
// products (one instruction each on CDNA), where Philox4x64 needs eight
// 32-bit multiplies for its two 64 x 64 -> 128-bit products.
#pragma once

#include "mfma_common.h"

namespace tsattn {

// a ^ b ^ k in one instruction (gfx950's three-input bitwise op, truth table
// 0x96); the compiler emits two two-input XORs for the plain expression.  k is
// the round key, uniform over the wave.
__device__ __forceinline__ uint32_t xor3_key(uint32_t a, uint32_t b, uint32_t k) {
  uint32_t r;
  asm("v_bitop3_b32 %0, %1, %2, %3 bitop3:0x96" : "=v"(r) : "v"(a), "v"(b), "s"(k));
  return r;
}

__device__ __forceinline__ void philox4x32(uint32_t (&c)[4], uint32_t k0, uint32_t k1) {
  constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
  constexpr uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += W0;
      k1 += W1;
    }
    const uint64_t p0 = static_cast<uint64_t>(M0) * c[0], p1 = static_cast<uint64_t>(M1) * c[2];
    const uint32_t n0 = xor3_key(static_cast<uint32_t>(p1 >> 32), c[1], k0);
    const uint32_t n2 = xor3_key(static_cast<uint32_t>(p0 >> 32), c[3], k1);
    c[0] = n0;
    c[1] = static_cast<uint32_t>(p1);
    c[2] = n2;
    c[3] = static_cast<uint32_t>(p0);
  }
}

// The 16 words of group n of the problem's dropout stream.
__device__ __forceinline__ void dropout_block(const DropDesc &d, uint64_t n, uint64_t (&out)[4]) {
  const uint64_t t = 2 * (d.c0 + n);
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    uint32_t c[4] = {static_cast<uint32_t>(t) | static_cast<uint32_t>(half), static_cast<uint32_t>(t >> 32),
                     static_cast<uint32_t>(d.k1), static_cast<uint32_t>(d.k1 >> 32)};
    philox4x32(c, static_cast<uint32_t>(d.k0), static_cast<uint32_t>(d.k0 >> 32));
    out[2 * half] = c[0] | (static_cast<uint64_t>(c[1]) << 32);
    out[2 * half + 1] = c[2] | (static_cast<uint64_t>(c[3]) << 32);
  }
}

// Block index of the 16 words starting at key j16 (a multiple of 16) of
// query row `row` = (b Hq + h) Sq + i: rows are Sk16 = Sk rounded up to 16
// words apart.
__device__ __forceinline__ uint64_t dropout_block_index(const Problem &p, int64_t row, int j16) {
  return static_cast<uint64_t>(row) * static_cast<uint64_t>((p.Sk + 15) / 16) +
         static_cast<uint64_t>(j16 / 16);
}

// The two blocks of a word group (dropout_block), advanced a few rounds at a
// time, so that a kernel can spread the rounds between instructions they do
// not depend on (the MFMA steps of a tile); the arithmetic of philox4x32,
// round r keyed (K0 lo + r W0, K0 hi + r W1) mod 2^32.
struct PhiloxPair {
  uint32_t c[2][4];
};

__device__ __forceinline__ PhiloxPair philox_pair_start(const DropDesc &d, uint64_t n) {
  const uint64_t t = 2 * (d.c0 + n);
  PhiloxPair s;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    s.c[half][0] = static_cast<uint32_t>(t) | static_cast<uint32_t>(half);
    s.c[half][1] = static_cast<uint32_t>(t >> 32);
    s.c[half][2] = static_cast<uint32_t>(d.k1);
    s.c[half][3] = static_cast<uint32_t>(d.k1 >> 32);
  }
  return s;
}

// Rounds r0 .. r1 - 1 (of 10) of both blocks.
__device__ __forceinline__ void philox_pair_rounds(PhiloxPair &s, const DropDesc &d, int r0, int r1) {
  constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
  constexpr uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int r = r0; r < r1; ++r) {
    const uint32_t k0 = static_cast<uint32_t>(d.k0) + static_cast<uint32_t>(r) * W0;
    const uint32_t k1 = static_cast<uint32_t>(d.k0 >> 32) + static_cast<uint32_t>(r) * W1;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      uint32_t(&c)[4] = s.c[half];
      const uint64_t p0 = static_cast<uint64_t>(M0) * c[0], p1 = static_cast<uint64_t>(M1) * c[2];
      const uint32_t n0 = xor3_key(static_cast<uint32_t>(p1 >> 32), c[1], k0);
      const uint32_t n2 = xor3_key(static_cast<uint32_t>(p0 >> 32), c[3], k1);
      c[0] = n0;
      c[1] = static_cast<uint32_t>(p1);
      c[2] = n2;
      c[3] = static_cast<uint32_t>(p0);
    }
  }
}

// The 16 dropout words of a lane holding query row `row` against keys
// kv0 + 8 g + 4 h + r (g, r = 0..3; the MFMA accumulator row pattern of the
// forward kernel), kv0 a multiple of 32, from the finished pair of group
// n = dropout_block_index(p, row, kv0 + 16 h) (lane half h computes the
// block of keys kv0 + 16 h .. + 15): word (g, r) is bits 16 r .. of out[g].
// The two halves exchange the quarters the other needs (v_permlane32_swap
// exchanges the upper half of its first register with the lower half of its
// second).
__device__ __forceinline__ void philox_pair_rows(const PhiloxPair &s, uint64_t (&out)[4]) {
  // Block quarter m = keys 4 m .. 4 m + 3 of the block (words 2m, 2m + 1 of
  // w, the block's four outputs in order).  Half 0 needs its own quarters 0,
  // 2 and half 1's 0, 2 (keys 16 ..); half 1 needs half 0's 1, 3 and its own
  // 1, 3.  One upper/lower swap per dword of the pairs (q0, q1) and (q2, q3)
  // leaves exactly that in both halves, with no selects.
  uint32_t w[8];
#pragma unroll
  for (int half = 0; half < 2; ++half)
#pragma unroll
    for (int i = 0; i < 4; ++i) w[4 * half + i] = s.c[half][i];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(w[e]), "+v"(w[2 + e]));
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(w[4 + e]), "+v"(w[6 + e]));
  }
  out[0] = w[0] | (static_cast<uint64_t>(w[1]) << 32);
  out[2] = w[2] | (static_cast<uint64_t>(w[3]) << 32);
  out[1] = w[4] | (static_cast<uint64_t>(w[5]) << 32);
  out[3] = w[6] | (static_cast<uint64_t>(w[7]) << 32);
}

// All of it at once: the lane's 16 words of group n (the caller keeps the
// row's part of n, loop-invariant).
__device__ __forceinline__ void dropout_words_rows(const DropDesc &d, uint64_t n,
                                                   uint64_t (&out)[4]) {
  PhiloxPair s = philox_pair_start(d, n);
  philox_pair_rounds(s, d, 0, 10);
  philox_pair_rows(s, out);
}

// Keep bit of element (row, key j) on its own (the generic kernels: each
// lane computes the block holding its word).
__device__ __forceinline__ bool dropout_keeps_one(const Problem &p, int64_t row, int j) {
  uint64_t blk[4];
  dropout_block(p.drop, dropout_block_index(p, row, j & ~15), blk);
  return (static_cast<uint32_t>(blk[(j & 15) >> 2] >> (16 * (j & 3))) & 0xFFFFu) >= p.drop.thr;
}

// Keep masks of two dropout words packed in u (one per 16-bit half): 0xFFFF in
// each half whose word is >= thr, else 0, in three packed 16-bit operations.
// thr2 = thr in both halves (thr <= 65535; a threshold of 65536 keeps nothing
// and is the caller's to handle).
__device__ __forceinline__ uint32_t keep_mask_pair(uint32_t u, uint32_t thr2) {
  uint32_t t, d, k;
  // thr - w, saturated at 0: 0 iff kept
  asm("v_pk_sub_u16 %0, %1, %2 clamp" : "=v"(t) : "s"(thr2), "v"(u));
  // 0 kept, 1 dropped
  asm("v_pk_min_u16 %0, %1, %2" : "=v"(d) : "v"(t), "s"(0x00010001u));
  // kept: 0 - 1 = 0xFFFF; dropped: 1 - 1 = 0
  asm("v_pk_sub_u16 %0, %1, %2" : "=v"(k) : "v"(d), "s"(0x00010001u));
  return k;
}

// Keep bits of the 16 words of an MFMA accumulator lane from its pair masks
// km[k] (keep_mask_pair of words 2k, 2k + 1): word i's bit at 8 (i / 4) +
// i % 4 (lane half 0's key positions; the other half shifts them by 4).
// Pair mask k's two halves land at bits 2k and 16 + 2k, the upper ones move
// down by 15 (word i at bit i), then nibble g (words 4g ..) spreads to bits
// 8g ..: two instructions per pair and five after.
__device__ __forceinline__ uint32_t keep_bits16(const uint32_t (&km)[8]) {
  uint32_t acc = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) acc |= (km[k] & 0x00010001u) << (2 * k);
  uint32_t x = (acc | (acc >> 15)) & 0xFFFFu;
  x = (x | (x << 8)) & 0x00FF00FFu;
  return (x | (x << 4)) & 0x0F0F0F0Fu;
}

__device__ __forceinline__ bool dropout_keeps(const DropDesc &d, const uint64_t (&w)[4], int i) {
  return (static_cast<uint32_t>(w[i >> 2] >> (16 * (i & 3))) & 0xFFFFu) >= d.thr;
}

}  // namespace tsattn
