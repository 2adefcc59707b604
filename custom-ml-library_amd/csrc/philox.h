// Counter-based random numbers for attention dropout: Philox4x64-10 (Salmon,
// Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC'11),
// the generator behind numpy.random.Philox, so that a mask can be checked bit
// for bit on the host.  Block n of a stream with key k and counter c is
// Philox4x64-10 of the 256-bit counter c + 1 + n (NumPy increments before
// each block); its four 64-bit outputs are 16 dropout words of 16 bits,
// little-endian.
#pragma once

#include "mfma_common.h"

namespace tsattn {

__device__ __forceinline__ void philox4x64(uint64_t (&c)[4], uint64_t k0, uint64_t k1) {
  constexpr uint64_t M0 = 0xD2E7470EE14C6C93ull, M1 = 0xCA5A826395121157ull;
  constexpr uint64_t W0 = 0x9E3779B97F4A7C15ull, W1 = 0xBB67AE8584CAA73Bull;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += W0;
      k1 += W1;
    }
    const uint64_t hi0 = __umul64hi(M0, c[0]), lo0 = M0 * c[0];
    const uint64_t hi1 = __umul64hi(M1, c[2]), lo1 = M1 * c[2];
    const uint64_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0;
    c[1] = lo1;
    c[2] = n2;
    c[3] = lo0;
  }
}

// The 16 words of block n of the problem's dropout stream.
__device__ __forceinline__ void dropout_block(const DropDesc &d, uint64_t n, uint64_t (&out)[4]) {
  const uint64_t c0 = d.c0 + n;
  out[0] = c0;
  out[1] = d.c1 + (c0 < n ? 1u : 0u);  // carry past 2^64
  out[2] = 0;
  out[3] = 0;
  philox4x64(out, d.k0, d.k1);
}

// Block index of the 16 words starting at key j16 (a multiple of 16) of
// query row `row` = (b Hq + h) Sq + i: rows are Sk16 = Sk rounded up to 16
// words apart.
__device__ __forceinline__ uint64_t dropout_block_index(const Problem &p, int64_t row, int j16) {
  return static_cast<uint64_t>(row) * static_cast<uint64_t>((p.Sk + 15) / 16) +
         static_cast<uint64_t>(j16 / 16);
}

// The 16 dropout words of a lane holding query row `row` against keys
// kv0 + 8 g + 4 h + r (g, r = 0..3; the MFMA accumulator row pattern of the
// forward and dQ kernels), kv0 a multiple of 32: word (g, r) is bits 16 r ..
// of out[g].  Lane half h computes the block of keys kv0 + 16 h .. + 15 and
// the two halves exchange the quarters the other needs.
__device__ __forceinline__ void dropout_words_rows(const Problem &p, int64_t row, int kv0, int h,
                                                   uint64_t (&out)[4]) {
  uint64_t blk[4];
  dropout_block(p.drop, dropout_block_index(p, row, kv0 + 16 * h), blk);
  // block quarter m = keys 4 m .. 4 m + 3 of the block; this lane needs
  // quarters h and 2 + h of both blocks
  const uint64_t keep0 = h ? blk[1] : blk[0], keep1 = h ? blk[3] : blk[2];
  const uint64_t recv0 = partner64(h ? blk[0] : blk[1], h);
  const uint64_t recv1 = partner64(h ? blk[2] : blk[3], h);
  out[0] = h ? recv0 : keep0;
  out[1] = h ? recv1 : keep1;
  out[2] = h ? keep0 : recv0;
  out[3] = h ? keep1 : recv1;
}

// Keep bit of element (row, key j) on its own (the generic kernels: each
// lane computes the block holding its word).
__device__ __forceinline__ bool dropout_keeps_one(const Problem &p, int64_t row, int j) {
  uint64_t blk[4];
  dropout_block(p.drop, dropout_block_index(p, row, j & ~15), blk);
  return (static_cast<uint32_t>(blk[(j & 15) >> 2] >> (16 * (j & 3))) & 0xFFFFu) >= p.drop.thr;
}

__device__ __forceinline__ bool dropout_keeps(const DropDesc &d, const uint64_t (&w)[4], int i) {
  return (static_cast<uint32_t>(w[i >> 2] >> (16 * (i & 3))) & 0xFFFFu) >= d.thr;
}

}  // namespace tsattn
