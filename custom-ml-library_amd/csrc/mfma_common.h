// MFMA helpers for gfx950 (CDNA4): 32x32x16 f16/bf16 contractions with fp32
// accumulation, operand packing and wave-level row reductions.
//
// Lane layout of v_mfma_f32_32x32x16_{bf16,f16}, lane l = 32*h + c:
//   A (32 x 16, M x K): lane holds A[c][8h + j],            j = 0..7
//   B (16 x 32, K x N): lane holds B[8h + j][c],            j = 0..7
//   C (32 x 32):        lane holds C[8(i>>2) + 4h + (i&3)][c], i = 0..15
// Only the pairing of A and B elements along K matters for a contraction, so
// any K permutation shared by both operands is valid; the kernels use that to
// feed a C tile straight back in as the next contraction's B operand.
#pragma once

#include "tsattn_internal.h"

namespace tsattn {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

template <typename T>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c);

template <>
__device__ __forceinline__ f32x16 mfma32<bf16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16 mfma32<f16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Two floats -> one dword of two 16-bit values (first in the low half), RNE.
template <typename T>
__device__ __forceinline__ unsigned pack2(float lo, float hi);
template <>
__device__ __forceinline__ unsigned pack2<bf16>(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(unsigned, __builtin_convertvector(v, bf16x2));
}
template <>
__device__ __forceinline__ unsigned pack2<f16>(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(unsigned, __builtin_convertvector(v, f16x2));
}

// Row index of accumulator element i for lane half h.
__device__ __forceinline__ constexpr int crow(int i, int h) { return ((i >> 2) << 3) + (h << 2) + (i & 3); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float xor32_max(float x) {
  float y = __shfl_xor(x, 32, 64);
  return fmaxf(x, y);
}
__device__ __forceinline__ float xor32_sum(float x) { return x + __shfl_xor(x, 32, 64); }

__device__ __forceinline__ u32x4 ld16(const void *p) { return *static_cast<const u32x4 *>(p); }
__device__ __forceinline__ u32x2 ld8(const void *p) { return *static_cast<const u32x2 *>(p); }

// Low / high 16-bit halves of two dwords interleaved: (a.lo, b.lo) and (a.hi, b.hi).
__device__ __forceinline__ unsigned pack_lo(unsigned a, unsigned b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ unsigned pack_hi(unsigned a, unsigned b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// A [ROWS x D] tile of 16-bit elements staged global -> registers -> LDS by
// 256 threads.  Thread t owns 16-byte column chunk dc = t % (D/8) of RU
// consecutive rows starting at g*RU, g = t / (D/8): sixteen (or eight)
// neighbouring lanes read one contiguous row, and the RU rows let the thread
// also write the tile transposed ([D][ROWS]) from registers.
template <typename T, int D, int ROWS>
struct TileRegs {
  static constexpr int DC = D / 8;
  static constexpr int RU = ROWS * DC / 256;
  static_assert(RU == 2 || RU == 4, "tile must give each thread 2 or 4 rows");
  u32x4 r[RU];

  __device__ __forceinline__ void load(const T *base, int64_t stride, int row0, int valid,
                                       int tid) {
    const int dc = tid % DC, g = tid / DC;
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const int row = row0 + g * RU + u;
      r[u] = row < valid ? ld16(base + static_cast<int64_t>(row) * stride + dc * 8)
                         : u32x4{0, 0, 0, 0};
    }
  }
  // lds[row * rstride + d]
  __device__ __forceinline__ void store_rows(T *lds, int rstride, int tid) const {
    const int dc = tid % DC, g = tid / DC;
#pragma unroll
    for (int u = 0; u < RU; ++u)
      *reinterpret_cast<u32x4 *>(lds + (g * RU + u) * rstride + dc * 8) = r[u];
  }
  // lds[d * tstride + row]
  __device__ __forceinline__ void store_cols(T *lds, int tstride, int tid) const {
    const int dc = tid % DC, g = tid / DC;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = dc * 8 + 2 * e;
      if constexpr (RU == 4) {
        u32x2 even = {pack_lo(r[0][e], r[1][e]), pack_lo(r[2][e], r[3][e])};
        u32x2 odd = {pack_hi(r[0][e], r[1][e]), pack_hi(r[2][e], r[3][e])};
        *reinterpret_cast<u32x2 *>(lds + d * tstride + g * 4) = even;
        *reinterpret_cast<u32x2 *>(lds + (d + 1) * tstride + g * 4) = odd;
      } else {
        *reinterpret_cast<unsigned *>(lds + d * tstride + g * 2) = pack_lo(r[0][e], r[1][e]);
        *reinterpret_cast<unsigned *>(lds + (d + 1) * tstride + g * 2) = pack_hi(r[0][e], r[1][e]);
      }
    }
  }
};

inline bool aligned16(View v) {
  return (reinterpret_cast<uintptr_t>(v.data) % 16 == 0) && v.s0 % 8 == 0 && v.s1 % 8 == 0 &&
         v.s2 % 8 == 0;
}

// Dispatch order on MI355X sends consecutive workgroup ids round-robin over
// the 8 XCDs (each with its own L2).  Give each XCD a contiguous range of
// logical ids so workgroups sharing K/V land on the same L2.
__device__ __forceinline__ int xcd_remap(int pid, int total) {
  const int full = (total / 8) * 8;
  if (pid >= full) return pid;
  return (pid & 7) * (full >> 3) + (pid >> 3);
}

}  // namespace tsattn
