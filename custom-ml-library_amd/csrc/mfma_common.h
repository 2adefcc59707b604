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

// A general mask over the 16 scores of a lane's accumulator (MK = 1 boolean,
// 2 additive f32, 3 additive f16 / bf16).  Score i sits at mask byte offset
// off0 + kc(i) * step with kc(i) = 8 (i / 4) + i % 4 (the accumulator row
// pattern, the lane half folded into off0).
//
// The 16 elements are fetched by buffer loads issued as assembly at the start
// of a tile's MFMA block, so their latency hides under it: the compiler does
// not see these loads and adds no wait for them (its waits would also wait for
// the DMA loads issued after them).  The kernel waits with wait_vm(n), n = the
// loads it issued since, then resolve()s the registers.  The load width is a
// compile-time constant: no branch separates a load from its wait.  Offsets past the
// buffer range read as zero; elements the kernel does not allow are not used.
struct MaskFetch {
  uint32_t v[16];

  template <int BYTES>
  __device__ __forceinline__ void issue(u32x4 desc, uint32_t off0, uint32_t step) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t off = off0 + static_cast<uint32_t>(8 * (i >> 2) + (i & 3)) * step;
      if constexpr (BYTES == 1)
        asm volatile("buffer_load_ubyte %0, %1, %2, 0 offen" : "=v"(v[i]) : "v"(off), "s"(desc) : "memory");
      else if constexpr (BYTES == 2)
        asm volatile("buffer_load_ushort %0, %1, %2, 0 offen" : "=v"(v[i]) : "v"(off), "s"(desc) : "memory");
      else
        asm volatile("buffer_load_dword %0, %1, %2, 0 offen" : "=v"(v[i]) : "v"(off), "s"(desc) : "memory");
    }
  }
  __device__ __forceinline__ void resolve() {
#pragma unroll
    for (int i = 0; i < 16; ++i) asm volatile("" : "+v"(v[i]));
  }

  // Key-contiguous masks with 16-byte aligned rows: lane half h loads keys
  // 16 h .. 16 h + 15 of the lane's row within the 32-key tile (NQ 16-byte
  // loads: bool 1, 16-bit 2, f32 4) into v[0 .. 4 NQ), resolve(), then
  // unpack<ES>(h) trades quarters with the partner lane (keys 4 m .. 4 m + 3
  // of a half, m = 0..3): the lane keeps quarters h and 2 + h of its own half
  // and receives the same quarters of the other half, which gives exactly its
  // keys 8 g + 4 h + r -- and spreads them to v[4 g + r] as the scalar fetch
  // would.
  // The raw pieces stay in vv, untouched until resolve_vec() has run after
  // the wait (a copy before that would read registers still being loaded).
  u32x4 vv[4];
  template <int NQ>
  __device__ __forceinline__ void issue_vec(u32x4 desc, uint32_t off) {
#pragma unroll
    for (int q = 0; q < NQ; ++q)
      asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=v"(vv[q]) : "v"(off + 16u * q), "s"(desc) : "memory");
  }
  template <int NQ>
  __device__ __forceinline__ void resolve_vec() {
#pragma unroll
    for (int q = 0; q < NQ; ++q) asm volatile("" : "+v"(vv[q]));
  }
  template <int ES>  // bytes per element: QD = ES dwords per quarter
  __device__ __forceinline__ void unpack(int h);
};

// The value x of the partner lane l ^ 32 (v_permlane32_swap exchanges the
// upper half of one register with the lower half of another; with both
// holding x, lanes 0..31 find the partner's value in the second, lanes
// 32..63 in the first).  Assembly: the builtin returns the same register for
// both halves when its operands are equal.
__device__ __forceinline__ unsigned partner32(unsigned x, int h) {
  unsigned a = x, b = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return h ? a : b;
}

template <int ES>
__device__ __forceinline__ void MaskFetch::unpack(int h) {
  constexpr int QD = ES;  // dwords per quarter (4 elements)
  unsigned d[4 * QD];
#pragma unroll
  for (int i = 0; i < 4 * QD; ++i) d[i] = vv[i >> 2][i & 3];
  unsigned g[4][QD];
#pragma unroll
  for (int t = 0; t < QD; ++t) {
    const unsigned k0 = h ? d[QD + t] : d[t], k1 = h ? d[3 * QD + t] : d[2 * QD + t];
    const unsigned s0 = h ? d[t] : d[QD + t], s1 = h ? d[2 * QD + t] : d[3 * QD + t];
    const unsigned r0 = partner32(s0, h), r1 = partner32(s1, h);
    g[0][t] = h ? r0 : k0;
    g[1][t] = h ? r1 : k1;
    g[2][t] = h ? k0 : r0;
    g[3][t] = h ? k1 : r1;
  }
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if constexpr (ES == 1) v[4 * q + r] = (g[q][0] >> (8 * r)) & 0xFFu;
      else if constexpr (ES == 2) v[4 * q + r] = (g[q][r >> 1] >> (16 * (r & 1))) & 0xFFFFu;
      else v[4 * q + r] = g[q][r];
    }
}

// Mask modes MK: 1 boolean, 2 additive f32, 3 additive f16 / bf16, read
// element by element; 4, 5, 6 the same kinds read as 16-byte row pieces
// (key-contiguous, 16-byte aligned rows; the forward and dQ kernels).
constexpr int mask_kind(int MK) { return MK > 3 ? MK - 3 : MK; }
constexpr bool mask_vec(int MK) { return MK > 3; }
// Bytes per mask element.
template <int MK>
constexpr int mask_bytes() { return mask_kind(MK) == 1 ? 1 : (mask_kind(MK) == 2 ? 4 : 2); }

// Apply fetched mask elements: score i is allowed iff lo <= kc(i) < hi and
// the mask allows it; disallowed scores become -inf.  With an additive mask
// the allowed ones become x sl + mask log2(e), i.e. (scores * scale + mask)
// in log2 units, already scaled.
template <int MK>
__device__ __forceinline__ void mask_scores(float (&x)[16], const MaskFetch &mf, int mdtype,
                                            int lo, int hi, float sl) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int kc = 8 * (i >> 2) + (i & 3);
    const bool in = (kc >= lo) & (kc < hi);
    if constexpr (mask_kind(MK) == 1) {
      x[i] = in && mf.v[i] != 0u ? x[i] : -INFINITY;
    } else {
      float mv;
      if constexpr (mask_kind(MK) == 2) mv = __builtin_bit_cast(float, mf.v[i]);
      else if (mdtype == TSATTN_BF16) mv = __builtin_bit_cast(float, mf.v[i] << 16);
      else mv = static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(mf.v[i])));
      x[i] = in ? fmaf(x[i], sl, mv * kLog2e) : -INFINITY;
    }
  }
}

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

// ---------------------------------------------------------------------------
// Buffer resources: loads whose byte offset falls past `bytes` return zeros,
// so ragged tiles need no branches.  Offsets are 32-bit: the host routes to
// these kernels only views whose per-head slice stays below 2^31 bytes
// (mfma_view_ok in api.hip).
// ---------------------------------------------------------------------------
using rsrc_t = __amdgpu_buffer_rsrc_t;
constexpr int kRsrcFlags = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family)

__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, static_cast<int>(bytes),
                                           kRsrcFlags);
}
__device__ __forceinline__ u32x4 buf_load16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 0);
}
__device__ __forceinline__ float buf_load_f32(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(off), 0, 0));
}
// Lane l's 16 bytes land at lds_wave + 16*l (lds_wave is wave-uniform).
__device__ __forceinline__ void buf_load16_lds(rsrc_t r, void *lds_wave, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, (__attribute__((address_space(3))) void *)(lds_wave), 16,
      static_cast<int>(off), 0, 0, 0);
}
__device__ __forceinline__ void buf_load4_lds(rsrc_t r, void *lds_wave, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, (__attribute__((address_space(3))) void *)(lds_wave), 4,
      static_cast<int>(off), 0, 0, 0);
}
// Wait for this wave's outstanding vector-memory loads (incl. LDS-direct ones):
// s_waitcnt vmcnt(0) with expcnt / lgkmcnt left at their maxima (gfx9 encoding).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// ---------------------------------------------------------------------------
// Swizzled LDS tiles: [rows][D] 16-bit elements, row-major, no padding; the
// 16-byte chunk c of row r sits at chunk position c ^ swz<D>(r).  gfx950's
// LDS has 64 four-byte banks and serves 16 lanes of a 16-byte read (or 32
// lanes of an 8-byte read) per cycle.  The swizzle makes both access shapes
// conflict-free:
//  * row reads: 16 lanes read one chunk column of 16 consecutive rows;
//  * transpose reads: 32 lanes read 4 consecutive chunks of 4 consecutive
//    rows (4 rows x 64 bytes).
// D = 128 (a row covers all 64 banks): swz = 4*(r&3) + ((r>>2)&3), a bijection
// on 16 aligned rows whose high two bits differ across 4 aligned rows.
// D = 64 (two rows per bank line): swz = 4*((r>>1)&1) + ((r>>2)&3), a
// bijection on each row parity of 16 aligned rows that moves rows r and r+2
// to different 4-chunk groups.
// ---------------------------------------------------------------------------
template <int D>
__device__ __forceinline__ constexpr int swz(int r) {
  return D == 128 ? (((r & 3) << 2) | ((r >> 2) & 3)) : ((((r >> 1) & 1) << 2) | ((r >> 2) & 3));
}

template <int D>
__device__ __forceinline__ constexpr int toff(int r, int col) {
  return r * D + ((((col >> 3) ^ swz<D>(r))) << 3) + (col & 7);
}

// Direct global -> LDS copy of ROWS rows (from row0) of one head into a
// swizzled tile, split over NW waves; rows at or past the resource bound
// arrive as zeros.  `stride_b` is the row stride in bytes.
template <int D, int ROWS, int NW>
__device__ __forceinline__ void tile_to_lds(rsrc_t r, uint32_t stride_b, int row0, void *tile,
                                            int wave, int lane) {
  constexpr int LOADS = ROWS * D * 2 / 1024;
#pragma unroll
  for (int n = wave; n < LOADS; n += NW) {
    const int off = n * 1024 + lane * 16;
    const int row = off / (D * 2);
    const int chunk = ((off % (D * 2)) >> 4) ^ swz<D>(row);
    buf_load16_lds(r, static_cast<unsigned char *>(tile) + n * 1024,
                   static_cast<uint32_t>(row0 + row) * stride_b + chunk * 16);
  }
}

// Zero `bytes` of LDS (multiple of 16) with all NT threads.  Run once before
// the first tile load: whatever a range-checked load leaves in padded rows is
// then either zero or a finite value from an earlier tile, so masked rows
// (probability 0) never multiply a stale NaN.
template <int NT>
__device__ __forceinline__ void zero_lds(void *p, int bytes, int tid) {
  u32x4 *q = static_cast<u32x4 *>(p);
  for (int i = tid; i < bytes / 16; i += NT) q[i] = u32x4{0, 0, 0, 0};
}

typedef short s16x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ u32x2 ds_read_tr(const T *p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4 *)(const_cast<T *>(p)));
  return __builtin_bit_cast(u32x2, v);
}

// A operand (M = 32 columns from mbase, K = 16 rows from kbase) of a swizzled
// row-major tile, i.e. the transpose of the stored rows.  Element j of lane
// (c, h) is tile[kbase + 8(j>>2) + 4h + (j&3)][mbase + c]: the K order that a
// C tile hands over as a B operand (see crow()).
template <typename T, int D>
__device__ __forceinline__ u32x4 tr_frag(const T *tile, int kbase, int mbase, int lane) {
  const int i = lane & 15, g = lane >> 4, h = lane >> 5;
  const int col = mbase + 16 * (g & 1) + 4 * (i & 3);
  const int r0 = kbase + 4 * h + (i >> 2);
  const u32x2 a = ds_read_tr(tile + toff<D>(r0, col));
  const u32x2 b = ds_read_tr(tile + toff<D>(r0 + 8, col));
  return u32x4{a[0], a[1], b[0], b[1]};
}

// A operand (M = 32 rows from rbase, K = 16 columns from kbase) of a
// swizzled tile: lane (c, h) reads row rbase + c, columns kbase + 8h .. +7.
template <typename T, int D>
__device__ __forceinline__ u32x4 row_frag(const T *tile, int rbase, int kbase, int lane) {
  return ld16(tile + toff<D>(rbase + (lane & 31), kbase + 8 * (lane >> 5)));
}

inline bool aligned16(View v) {
  return (reinterpret_cast<uintptr_t>(v.data) % 16 == 0) && v.s0 % 8 == 0 && v.s1 % 8 == 0 &&
         v.s2 % 8 == 0;
}

// ---------------------------------------------------------------------------
// Streaming machinery shared by the forward and backward kernels: DMA tile
// loads that the compiler does not order against LDS reads, explicit waits,
// a fence-free barrier and the blocked K/V tile layout.
// ---------------------------------------------------------------------------
// gfx9 s_waitcnt immediates: vmcnt(n) with n in [0, 63] (low 4 bits in
// [3:0], high 2 bits in [15:14]), expcnt and lgkmcnt at their maxima; or
// lgkmcnt(0) alone.  n is wave-uniform; counts above 20 are clamped to 20,
// which waits for more loads than asked (always safe).
template <int N>
__device__ __forceinline__ void wait_vm_n() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ __forceinline__ void wait_vm(int n) {
  switch (n) {
    case 0: wait_vm_n<0>(); break;
    case 1: wait_vm_n<1>(); break;
    case 2: wait_vm_n<2>(); break;
    case 3: wait_vm_n<3>(); break;
    case 4: wait_vm_n<4>(); break;
    case 5: wait_vm_n<5>(); break;
    case 6: wait_vm_n<6>(); break;
    case 7: wait_vm_n<7>(); break;
    case 8: wait_vm_n<8>(); break;
    case 9: wait_vm_n<9>(); break;
    case 10: wait_vm_n<10>(); break;
    case 11: wait_vm_n<11>(); break;
    case 12: wait_vm_n<12>(); break;
    case 13: wait_vm_n<13>(); break;
    case 14: wait_vm_n<14>(); break;
    case 15: wait_vm_n<15>(); break;
    case 16: wait_vm_n<16>(); break;
    case 17: wait_vm_n<17>(); break;
    case 18: wait_vm_n<18>(); break;
    case 19: wait_vm_n<19>(); break;
    case 20: wait_vm_n<20>(); break;
    default: wait_vm_n<20>(); break;
  }
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Workgroup barrier without a memory fence: outstanding global -> LDS loads
// of later tiles stay in flight.  The scheduler may not move code across it.
__device__ __forceinline__ void phase_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// Buffer descriptor (raw, 32-bit records) as four SGPRs for inline assembly.
__device__ __forceinline__ u32x4 make_desc(const void *base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return u32x4{static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32) & 0xFFFFu, bytes,
               static_cast<uint32_t>(kRsrcFlags)};
}

// 16-byte global -> LDS load: lane l's bytes land at LDS address m0 + 16 l.
// Issued as assembly so that the compiler does not treat later LDS reads as
// depending on it (it would wait for every such load before each read); the
// kernel orders these loads itself with s_waitcnt vmcnt + s_barrier.
// The byte offset is voff (per lane) + soff (wave-uniform).
__device__ __forceinline__ void dma16(u32x4 desc, uint32_t lds_addr, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voff), "s"(desc),
                 "s"(__builtin_amdgcn_readfirstlane(soff))
               : "memory", "m0");
}

// The same for data read once (streaming: nontemporal cache policy).
__device__ __forceinline__ void dma16_nt(u32x4 desc, uint32_t lds_addr, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen nt lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voff), "s"(desc),
                 "s"(__builtin_amdgcn_readfirstlane(soff))
               : "memory", "m0");
}

// max(x, x of lane l ^ 32) without an LDS round trip: v_permlane32_swap
// exchanges the upper half of `a` with the lower half of `b`, so afterwards
// {a, b} holds {own, partner} in every lane.  (Assembly: the compiler builtin
// returns the same register for both halves when its operands are equal.)
__device__ __forceinline__ float half_swap_max(float x) {
  unsigned a = __builtin_bit_cast(unsigned, x), b = a;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}

// max(a, b, c) in one v_max3_f32, without the NaN canonicalisation the
// compiler adds around fmaxf (scores are never NaN unless an input is).
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// half_swap_max with the final max in one instruction (no canonicalisation).
__device__ __forceinline__ float half_swap_max3(float x) {
  unsigned a = __builtin_bit_cast(unsigned, x), b = a;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return max3f(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b), __builtin_bit_cast(float, b));
}

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void *)(p)));
}

// K / V tile layout in LDS: [BN x D] 16-bit elements cut into blocks of 16
// rows x 4 sixteen-byte chunks (1 KiB), block (r / 16, k / 4) at
// 1 KiB * ((r / 16) * D/32 + k / 4).  Inside a block, chunk k of row r sits at
// slot 4 (r % 16) + ((k % 4) ^ ((r / 4) % 4)).  One DMA instruction fills one
// block (four lanes per 64-byte row segment); K row fragments and V transpose
// fragments are conflict-free, and every fragment address is one of four
// per-lane bases plus a compile-time offset.
template <typename T, int D>
struct TileReader {
  static constexpr int QG = D / 32;
  uint32_t k_even, k_odd, v_lo, v_hi;  // byte offsets within a tile

  __device__ __forceinline__ explicit TileReader(int lane) {
    const int c = lane & 31, h = lane >> 5, i16 = lane & 15, g = lane >> 4;
    const int kb = (c >> 4) * QG * 1024 + (c & 15) * 64;
    k_even = kb + ((h ^ ((c >> 2) & 3)) << 4);
    k_odd = kb + (((2 + h) ^ ((c >> 2) & 3)) << 4);
    const int sel = 2 * (g & 1) + ((i16 & 3) >> 1);
    v_lo = (((4 * h + (i16 >> 2)) * 4 + (sel ^ h)) << 4) + (i16 & 1) * 8;
    v_hi = (((8 + 4 * h + (i16 >> 2)) * 4 + (sel ^ (h + 2))) << 4) + (i16 & 1) * 8;
  }
  // Row fragment (A operand of e.g. S^T = K Q^T): lane (c, h) holds tile
  // row 32 t + c, columns 16 i + 8 h .. +7.
  __device__ __forceinline__ u32x4 rows(const char *tile, int t, int i) const {
    return ld16(tile + ((i & 1) ? k_odd : k_even) + (2 * t * QG + (i >> 1)) * 1024);
  }
  // Column fragment (A operand of e.g. O^T += V^T P^T): lane (c, h) holds
  // tile column 32 dt + c at the 8 rows of k-step ks (rows 16 ks + ...) in
  // the order a C tile hands over as a B operand (see crow()).
  __device__ __forceinline__ u32x4 cols(const char *tile, int ks, int dt) const {
    const char *blk = tile + (ks * QG + dt) * 1024;
    const u32x2 a = ds_read_tr<T>(reinterpret_cast<const T *>(blk + v_lo));
    const u32x2 b = ds_read_tr<T>(reinterpret_cast<const T *>(blk + v_hi));
    return u32x4{a[0], a[1], b[0], b[1]};
  }
};

// Dispatch order on MI355X sends consecutive workgroup ids round-robin over
// the 8 XCDs (each with its own L2).  Give each XCD a contiguous range of
// logical ids so workgroups sharing K/V land on the same L2.
__device__ __forceinline__ int xcd_remap(int pid, int total) {
  const int full = (total / 8) * 8;
  if (pid >= full) return pid;
  return (pid & 7) * (full >> 3) + (pid >> 3);
}

// Logical id -> (head slice, work rank).  Heads are taken in groups of G;
// inside a group the ids walk the ranks from the heaviest (rank 0: the most
// causal work) down, cycling over the group's heads.  The tail of the grid
// then holds only light blocks, so greedy dispatch stays near the ideal
// makespan.  G is the number of heads whose blocks fill one XCD's resident
// slots (`xcd_slots` = workgroups resident per XCD), so short sequences mix a
// few heads while long ones keep one head per XCD and its K/V stream in L2.
__device__ __forceinline__ void heavy_first(int logical, int n_blk, int n_bh, int xcd_slots,
                                            int &bh, int &rank) {
  const int G = max(1, xcd_slots / n_blk);
  const int grp = logical / (G * n_blk);
  const int in = logical - grp * G * n_blk;
  const int heads = min(G, n_bh - grp * G);
  rank = in / heads;
  bh = grp * G + (in - rank * heads);
}

}  // namespace tsattn
