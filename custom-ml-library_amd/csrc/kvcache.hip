// KV-cache append into the reference's int8 format (src/tensorsmith/nn/
// cache.py:54-86, quantiser at :73-77): for every appended row x = src[b, h,
// t, 0:D] (already in the cache dtype), in fp32,
//   s = max(max_d |x_d| / 127, 1e-8),   q_d = round_half_even(x_d / s),
// stored as int8 at dst[b, h, pos + t, d] with s at scale[b, h, pos + t].
// One kernel does the reduction, the division, the rounding and both writes,
// so an append is one pass over the new rows.  Division is IEEE (correctly
// rounded) and rint rounds half to even, as NumPy's round does: the stored
// bytes and scales are bit-identical to the reference's.
#include "mfma_common.h"

namespace tsattn {
namespace {

constexpr int NT = 256;

template <typename T>
__global__ __launch_bounds__(NT) void kv_append_int8_kernel(int B, int H, int T_, int D, View src,
                                                            View dst, View scale, int64_t pos) {
  // one wave per row (b, h, t); lane handles elements lane, lane + 64, ...
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (NT / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= static_cast<int64_t>(B) * H * T_) return;
  const int t = static_cast<int>(row % T_);
  const int64_t bh = row / T_;
  const int h = static_cast<int>(bh % H), b = static_cast<int>(bh / H);
  const T *x = static_cast<const T *>(src.data) + b * src.s0 + h * src.s1 + static_cast<int64_t>(t) * src.s2;
  int8_t *q = static_cast<int8_t *>(const_cast<void *>(dst.data)) + b * dst.s0 + h * dst.s1 +
              (pos + t) * dst.s2;
  constexpr int PER = 8;  // D <= 512
  float v[PER];
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int d = lane + 64 * j;
    v[j] = d < D ? static_cast<float>(x[d]) : 0.f;
    m = fmaxf(m, fabsf(v[j]));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  const float s = fmaxf(m / 127.f, 1e-8f);
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int d = lane + 64 * j;
    if (d < D) q[d] = static_cast<int8_t>(rintf(v[j] / s));
  }
  if (lane == 0)
    static_cast<float *>(const_cast<void *>(scale.data))[b * scale.s0 + h * scale.s1 + (pos + t) * scale.s2] = s;
}

// n / d for 0 <= n < 2^31 as (mulhi(n, m) + n) >> l with l = ceil(log2 d)
// and m = floor(2^32 (2^l - d) / d) + 1 (Granlund and Montgomery, "Division
// by invariant integers using multiplication", PLDI 1994).
struct FastDiv {
  uint32_t m, l;
};

FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while ((uint64_t(1) << l) < d) ++l;
  return FastDiv{static_cast<uint32_t>((uint64_t(1) << 32) * ((uint64_t(1) << l) - d) / d + 1), l};
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, FastDiv f) { return (__umulhi(n, f.m) + n) >> f.l; }

// max over each aligned group of G lanes (G = 8, 16, 32) of a non-negative
// float, on its bit pattern: DPP quad swaps, the half-row and row mirrors,
// then a swizzle across the two rows of a 32-lane half.
template <int G>
__device__ __forceinline__ float group_max(float x) {
  uint32_t m = __float_as_uint(x);
  m = max(m, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(m), 0xB1, 0xF, 0xF, false)));
  m = max(m, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(m), 0x4E, 0xF, 0xF, false)));
  m = max(m, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(m), 0x141, 0xF, 0xF, false)));
  if constexpr (G >= 16)
    m = max(m, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(m), 0x140, 0xF, 0xF, false)));
  if constexpr (G >= 32) m = max(m, static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(m), 0x401F)));
  return __uint_as_float(m);
}

// max(m / 127, 1e-8) correctly rounded, without a division: q0 = m * r with
// r = RN(1 / 127), the exact remainder m - 127 q0 by one fma, and one fma
// correction.  For m an fp16 or bf16 magnitude the result equals the IEEE
// quotient (checked on every finite value of both formats; below 1.2e-6 the
// 1e-8 floor applies either way).
__device__ __forceinline__ float row_scale(float m) {
#pragma clang fp contract(off)
  constexpr float r = 1.f / 127.f;
  const float q0 = m * r;
  const float rem = __builtin_fmaf(-q0, 127.f, m);
  return fmaxf(__builtin_fmaf(rem, r, q0), 1e-8f);
}

// low bytes of a, b, c, d as one little-endian word
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0c0c0400u), cd = __builtin_amdgcn_perm(d, c, 0x0c0c0400u);
  return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

// Rows of D = 8 G 16-bit elements.  A wave takes RPW = RB * 64 / G
// consecutive rows t0 .. t0 + RPW - 1 of one (b, h) (wave -> (b, h, chunk)
// in scalar registers); lane (r, g) loads elements 8 g .. 8 g + 7 of rows
// r, r + 64 / G, ... in one 16-byte load each, all loads issued before any
// math, and stores their 8 codes with one 8-byte store.  Past the last row
// of (b, h) the loads repeat that row and nothing is stored.
//
// round_half_even(x / s) as NumPy computes it (the correctly rounded fp32
// quotient, then rint) comes from q = x * rcp(s): |q - x / s| <= 127 *
// (2^-23 + 2^-24) < 2.3e-5 (v_rcp_f32 is within one ulp) and the quotient's
// own rounding adds at most 2^-18, so the two round alike unless q lies
// within 5e-5 of a half-integer; a row with any such element is redone with
// the IEEE division.  Rounding to an integer adds 1.5 * 2^23 (the sum rounds
// half to even, |q| < 2^22), whose low byte is then the two's-complement code.
template <typename T, int G, int RB>
__global__ __launch_bounds__(NT) void kv_append_int8_vec_kernel(int H, int T_, uint32_t chunks, FastDiv fc,
                                                                FastDiv fh, uint32_t waves, View src,
                                                                View dst, View scale, int64_t pos) {
#pragma clang fp contract(off)
  constexpr int RPI = 64 / G, RPW = RPI * RB;
  constexpr float kMagic = 12582912.f;
  const int lane = threadIdx.x & 63, g = lane % G, rl = lane / G;
  const uint32_t w = __builtin_amdgcn_readfirstlane(blockIdx.x * (NT / 64) + (threadIdx.x >> 6));
  if (w >= waves) return;
  const uint32_t bh = fdiv(w, fc), chunk = w - bh * chunks;
  const uint32_t b = fdiv(bh, fh), h = bh - b * H;
  const int t0 = static_cast<int>(chunk) * RPW, last = T_ - 1 - t0;
  const T *sp = static_cast<const T *>(src.data) + b * src.s0 + h * src.s1 + t0 * src.s2 + 8 * g;
  int8_t *dp = static_cast<int8_t *>(const_cast<void *>(dst.data)) + b * dst.s0 + h * dst.s1 +
               (pos + t0) * dst.s2 + 8 * g;
  float *cp = static_cast<float *>(const_cast<void *>(scale.data)) + b * scale.s0 + h * scale.s1 +
              (pos + t0) * scale.s2;
  u32x4 raw[RB];
#pragma unroll
  for (int i = 0; i < RB; ++i)
    raw[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(sp + min(i * RPI + rl, last) * src.s2));
#pragma unroll
  for (int i = 0; i < RB; ++i) {
    const T *e = reinterpret_cast<const T *>(&raw[i]);
    float v[8];
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[j] = static_cast<float>(e[j]);
      m = fmaxf(m, fabsf(v[j]));
    }
    const float sc = row_scale(group_max<G>(m));
    const float rc = __builtin_amdgcn_rcpf(sc);
    uint32_t c[8];
    float worst = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float q = v[j] * rc;
      const float t = q + kMagic;
      worst = fmaxf(worst, fabsf(q - (t - kMagic)));
      c[j] = __float_as_uint(t);
    }
    if (worst > 0.5f - 5e-5f) {
#pragma unroll
      for (int j = 0; j < 8; ++j) c[j] = __float_as_uint(v[j] / sc + kMagic);
    }
    const int k = i * RPI + rl;
    if (k <= last) {
      __builtin_nontemporal_store(u32x2{pack_low_bytes(c[0], c[1], c[2], c[3]), pack_low_bytes(c[4], c[5], c[6], c[7])},
                                  reinterpret_cast<u32x2 *>(dp + k * dst.s2));
      if (g == 0) __builtin_nontemporal_store(sc, cp + k * scale.s2);
    }
  }
}

}  // namespace

hipError_t launch_kv_append_int8(int dtype, int B, int H, int T_, int D, View src, View dst,
                                 View scale, int64_t pos, hipStream_t st) {
  const int64_t rows = static_cast<int64_t>(B) * H * T_;
  Probe pr_("kv_append_int8", st);
  // 16-bit rows of 64, 128 or 256 elements with 16-byte aligned source chunks
  // and 8-byte aligned code rows: the vectorised kernel.
  const bool vec = dtype != TSATTN_F32 && (D == 64 || D == 128 || D == 256) &&
                   static_cast<int64_t>(B) * H * ((T_ + 7) / 8) < (int64_t(1) << 31) &&
                   reinterpret_cast<uintptr_t>(src.data) % 16 == 0 && src.s0 % 8 == 0 &&
                   src.s1 % 8 == 0 && src.s2 % 8 == 0 &&
                   reinterpret_cast<uintptr_t>(dst.data) % 8 == 0 && dst.s0 % 8 == 0 &&
                   dst.s1 % 8 == 0 && dst.s2 % 8 == 0;
  if (vec) {
    constexpr int RB = 2;  // rows per lane: 1 and 4 measured slower (5.5 TB/s against 6.2 at the C3 cache shape)
    const int G = D / 8, rpw = (64 / G) * RB;
    const uint32_t chunks = static_cast<uint32_t>((T_ + rpw - 1) / rpw);
    const uint32_t waves = chunks * static_cast<uint32_t>(B * H);
    const FastDiv fc = make_fastdiv(chunks), fh = make_fastdiv(H);
    const dim3 grid((waves + NT / 64 - 1) / (NT / 64)), block(NT);
#define TSATTN_APPEND(TY, GG) \
  kv_append_int8_vec_kernel<TY, GG, RB><<<grid, block, 0, st>>>(H, T_, chunks, fc, fh, waves, src, dst, scale, pos)
    if (dtype == TSATTN_F16) {
      if (G == 8) TSATTN_APPEND(f16, 8);
      else if (G == 16) TSATTN_APPEND(f16, 16);
      else TSATTN_APPEND(f16, 32);
    } else {
      if (G == 8) TSATTN_APPEND(bf16, 8);
      else if (G == 16) TSATTN_APPEND(bf16, 16);
      else TSATTN_APPEND(bf16, 32);
    }
#undef TSATTN_APPEND
    return hipGetLastError();
  }
  const dim3 grid(static_cast<unsigned>((rows + NT / 64 - 1) / (NT / 64))), block(NT);
  if (dtype == TSATTN_F32) kv_append_int8_kernel<float><<<grid, block, 0, st>>>(B, H, T_, D, src, dst, scale, pos);
  else if (dtype == TSATTN_F16) kv_append_int8_kernel<f16><<<grid, block, 0, st>>>(B, H, T_, D, src, dst, scale, pos);
  else kv_append_int8_kernel<bf16><<<grid, block, 0, st>>>(B, H, T_, D, src, dst, scale, pos);
  return hipGetLastError();
}

}  // namespace tsattn
