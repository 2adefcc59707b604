// Interleaved-pair rotary position embedding (the reference's
// rotary_embedding, src/tensorsmith/nn/attention.py:255-296) as one kernel,
// and the same rotation fused with the KV-cache append (cache.py:54-86).
//
// For channel pair (2i, 2i+1) of row t: c = cos[p, i], s = sin[p, i] with
// p = pos0 + t, taken from tables the host builds exactly as the reference
// does (fp32 angles p * base^(-2i/dim), cos / sin, cast to the tensor
// dtype); the rotation rounds as the reference's array arithmetic
// (rope_math.h), so results are bit-identical.  `inverse` rotates by -angle
// (the VJP, :289-294).  Channels at or past rotary_dim pass through.
#include "mfma_common.h"
#include "rope_math.h"

namespace tsattn {
namespace {

constexpr int NT = 256;

struct RopeArgs {
  int B, H, T, D, R;  // R = rotary dim (even, <= D)
  View x, out;        // [B, H, T, D]
  const void *cos, *sin;  // [*, R / 2] rows in the tensor dtype
  int64_t pos0;
  int inverse;
};

template <typename T>
__global__ __launch_bounds__(NT) void rope_kernel(RopeArgs a) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (NT / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= static_cast<int64_t>(a.B) * a.H * a.T) return;
  const int t = static_cast<int>(row % a.T);
  const int64_t bh = row / a.T;
  const int h = static_cast<int>(bh % a.H), b = static_cast<int>(bh / a.H);
  const T *x = static_cast<const T *>(a.x.data) + b * a.x.s0 + h * a.x.s1 + static_cast<int64_t>(t) * a.x.s2;
  T *y = static_cast<T *>(const_cast<void *>(a.out.data)) + b * a.out.s0 + h * a.out.s1 +
         static_cast<int64_t>(t) * a.out.s2;
  const T *cr = static_cast<const T *>(a.cos) + (a.pos0 + t) * (a.R / 2);
  const T *sr = static_cast<const T *>(a.sin) + (a.pos0 + t) * (a.R / 2);
  for (int p = lane; 2 * p < a.D; p += 64) {
    T x0 = x[2 * p], x1 = x[2 * p + 1];
    if (2 * p < a.R) rotate_pair(x0, x1, cr[p], sr[p], a.inverse != 0);
    y[2 * p] = x0;
    y[2 * p + 1] = x1;
  }
}

// The same with 16-byte chunks of rows (8 16-bit or 4 f32 values, NP = 4 or
// 2 pairs): a workgroup takes NT * RU consecutive chunks of one (b, h) --
// block `blk` of the nblk blocks of that head, so the head's coordinates come
// from the workgroup index alone -- and a thread RU of them, NT apart (each
// load instruction of a wave covers 1 KiB of consecutive chunks), all its
// loads issued before any rotation; one 8-byte load from each table per
// chunk.  Needs 16-byte aligned rows, D * size(T) a multiple of 16, R a
// multiple of 2 NP (a chunk is wholly inside or outside the rotated
// channels), 8-byte aligned tables and T * D * size(T) / 16 < 2^31.
constexpr int RU = 4;

template <typename T>
__global__ __launch_bounds__(NT) void rope_vec_kernel(RopeArgs a, int nblk) {
  constexpr int CH = 16 / static_cast<int>(sizeof(T)), NP = CH / 2;
  const int cpr = a.D / CH;
  const int bh = blockIdx.x / nblk, blk = blockIdx.x - bh * nblk;
  const int h = bh % a.H, b = bh / a.H;
  const int n = a.T * cpr;  // chunks of this head
  const T *xb = static_cast<const T *>(a.x.data) + b * a.x.s0 + h * a.x.s1;
  T *yb = static_cast<T *>(const_cast<void *>(a.out.data)) + b * a.out.s0 + h * a.out.s1;
  u32x4 v[RU];
  int tq[RU][2];
#pragma unroll
  for (int u = 0; u < RU; ++u) {
    int idx = (blk * RU + u) * NT + static_cast<int>(threadIdx.x);
    idx = idx < n ? idx : n - 1;  // past the head: reload its last chunk, store nothing
    const int t = idx / cpr;
    tq[u][0] = t;
    tq[u][1] = idx - t * cpr;
    v[u] = *reinterpret_cast<const u32x4 *>(xb + static_cast<int64_t>(t) * a.x.s2 + tq[u][1] * CH);
  }
#pragma unroll
  for (int u = 0; u < RU; ++u) {
    const int t = tq[u][0], q = tq[u][1], p0 = q * NP;
    if (2 * p0 < a.R) {
      const int64_t at = (a.pos0 + t) * (a.R / 2) + p0;
      const u32x2 cw = *reinterpret_cast<const u32x2 *>(static_cast<const T *>(a.cos) + at);
      const u32x2 sw = *reinterpret_cast<const u32x2 *>(static_cast<const T *>(a.sin) + at);
      if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int m = 0; m < NP; ++m) {
          // vector elements go through scalars: a bit cast of `v[u][i]`
          // itself reads element 0
          const unsigned w0 = v[u][2 * m], w1 = v[u][2 * m + 1], cb = cw[m], sb = sw[m];
          T x0 = __builtin_bit_cast(T, w0), x1 = __builtin_bit_cast(T, w1);
          rotate_pair(x0, x1, __builtin_bit_cast(T, cb), __builtin_bit_cast(T, sb), a.inverse != 0);
          v[u][2 * m] = __builtin_bit_cast(unsigned, x0);
          v[u][2 * m + 1] = __builtin_bit_cast(unsigned, x1);
        }
      } else {
#pragma unroll
        for (int m = 0; m < NP; ++m) {
          const int sh = (m & 1) * 16;
          const T c = __builtin_bit_cast(T, static_cast<uint16_t>(cw[m >> 1] >> sh));
          const T sn = __builtin_bit_cast(T, static_cast<uint16_t>(sw[m >> 1] >> sh));
          v[u][m] = rotate_word<T>(v[u][m], c, sn, a.inverse != 0);
        }
      }
    }
    if ((blk * RU + u) * NT + static_cast<int>(threadIdx.x) < n)
      *reinterpret_cast<u32x4 *>(yb + static_cast<int64_t>(t) * a.out.s2 + q * CH) = v[u];
  }
}

bool rope_vec_ok(const RopeArgs &a, int esize) {
  const int ch = 16 / esize;
  auto al = [](const void *p, int n) { return reinterpret_cast<uintptr_t>(p) % n == 0; };
  auto st = [&](const View &v) { return (v.s0 * esize) % 16 == 0 && (v.s1 * esize) % 16 == 0 && (v.s2 * esize) % 16 == 0; };
  return (a.D * esize) % 16 == 0 && a.R % ch == 0 && al(a.x.data, 16) && al(a.out.data, 16) &&
         st(a.x) && st(a.out) && al(a.cos, 8) && al(a.sin, 8) &&
         static_cast<int64_t>(a.T) * (a.D * esize / 16) + NT * RU < (int64_t(1) << 31);
}

struct AppendArgs {
  int B, H, T, D, R;      // R = 0: no rotation
  View k, v;              // new rows [B, H, T, D]
  View kc, vc, ks, vs;    // cache storage; ks / vs set for int8 caches
  const void *cos, *sin;  // [*, R / 2]
  int64_t pos;
};

// Quantise one wave-held row (PER values per lane, channels 2p, 2p + 1 for
// p = lane + 64 j) into int8 codes + scale, as the reference (cache.py:73-77).
template <typename T, int PER>
__device__ __forceinline__ void store_int8_row(const T (&x)[PER][2], int D, int lane, int8_t *q,
                                               float *scale) {
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j)
    if (2 * (lane + 64 * j) < D)
      m = fmaxf(m, fmaxf(fabsf(static_cast<float>(x[j][0])), fabsf(static_cast<float>(x[j][1]))));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  const float s = fmaxf(m / 127.f, 1e-8f);
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int p = lane + 64 * j;
    if (2 * p < D) {
      q[2 * p] = static_cast<int8_t>(rintf(static_cast<float>(x[j][0]) / s));
      q[2 * p + 1] = static_cast<int8_t>(rintf(static_cast<float>(x[j][1]) / s));
    }
  }
  if (lane == 0) *scale = s;
}

template <typename T, bool Q8>
__global__ __launch_bounds__(NT) void rope_append_kernel(AppendArgs a) {
  constexpr int PER = 4;  // pairs per lane: D <= 512
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (NT / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= static_cast<int64_t>(a.B) * a.H * a.T) return;
  const int t = static_cast<int>(row % a.T);
  const int64_t bh = row / a.T;
  const int h = static_cast<int>(bh % a.H), b = static_cast<int>(bh / a.H);
  const int64_t tp = a.pos + t;
  const T *kx = static_cast<const T *>(a.k.data) + b * a.k.s0 + h * a.k.s1 + static_cast<int64_t>(t) * a.k.s2;
  const T *vx = static_cast<const T *>(a.v.data) + b * a.v.s0 + h * a.v.s1 + static_cast<int64_t>(t) * a.v.s2;
  const T *cr = static_cast<const T *>(a.cos) + tp * (a.R / 2);
  const T *sr = static_cast<const T *>(a.sin) + tp * (a.R / 2);
  T kr[PER][2], vr[PER][2];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int p = lane + 64 * j;
    kr[j][0] = kr[j][1] = vr[j][0] = vr[j][1] = static_cast<T>(0.f);
    if (2 * p < a.D) {
      kr[j][0] = kx[2 * p];
      kr[j][1] = kx[2 * p + 1];
      vr[j][0] = vx[2 * p];
      vr[j][1] = vx[2 * p + 1];
      if (2 * p < a.R) rotate_pair(kr[j][0], kr[j][1], cr[p], sr[p], false);
    }
  }
  if constexpr (Q8) {
    int8_t *kq = static_cast<int8_t *>(const_cast<void *>(a.kc.data)) + b * a.kc.s0 + h * a.kc.s1 + tp * a.kc.s2;
    int8_t *vq = static_cast<int8_t *>(const_cast<void *>(a.vc.data)) + b * a.vc.s0 + h * a.vc.s1 + tp * a.vc.s2;
    float *ksp = static_cast<float *>(const_cast<void *>(a.ks.data)) + b * a.ks.s0 + h * a.ks.s1 + tp * a.ks.s2;
    float *vsp = static_cast<float *>(const_cast<void *>(a.vs.data)) + b * a.vs.s0 + h * a.vs.s1 + tp * a.vs.s2;
    store_int8_row<T, PER>(kr, a.D, lane, kq, ksp);
    store_int8_row<T, PER>(vr, a.D, lane, vq, vsp);
  } else {
    T *kc = static_cast<T *>(const_cast<void *>(a.kc.data)) + b * a.kc.s0 + h * a.kc.s1 + tp * a.kc.s2;
    T *vc = static_cast<T *>(const_cast<void *>(a.vc.data)) + b * a.vc.s0 + h * a.vc.s1 + tp * a.vc.s2;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int p = lane + 64 * j;
      if (2 * p < a.D) {
        kc[2 * p] = kr[j][0];
        kc[2 * p + 1] = kr[j][1];
        vc[2 * p] = vr[j][0];
        vc[2 * p + 1] = vr[j][1];
      }
    }
  }
}

dim3 row_grid(int B, int H, int T) {
  const int64_t rows = static_cast<int64_t>(B) * H * T;
  return dim3(static_cast<unsigned>((rows + NT / 64 - 1) / (NT / 64)));
}

}  // namespace

hipError_t launch_rope(int dtype, int B, int H, int T, int D, int R, View x, View out,
                       const void *cos, const void *sin, int64_t pos0, int inverse, hipStream_t st) {
  RopeArgs a{B, H, T, D, R, x, out, cos, sin, pos0, inverse};
  Probe pr_("rope", st);
  const int esize = dtype == TSATTN_F32 ? 4 : 2;
  if (rope_vec_ok(a, esize)) {
    const int64_t chunks = static_cast<int64_t>(T) * (D * esize / 16);  // per head
    const int nblk = static_cast<int>((chunks + NT * RU - 1) / (NT * RU));
    const int64_t blocks = static_cast<int64_t>(B) * H * nblk;
    if (blocks >= (int64_t(1) << 31)) return hipErrorInvalidConfiguration;
    const dim3 g(static_cast<unsigned>(blocks));
    if (dtype == TSATTN_F32) rope_vec_kernel<float><<<g, NT, 0, st>>>(a, nblk);
    else if (dtype == TSATTN_F16) rope_vec_kernel<f16><<<g, NT, 0, st>>>(a, nblk);
    else rope_vec_kernel<bf16><<<g, NT, 0, st>>>(a, nblk);
  } else if (dtype == TSATTN_F32) {
    rope_kernel<float><<<row_grid(B, H, T), NT, 0, st>>>(a);
  } else if (dtype == TSATTN_F16) {
    rope_kernel<f16><<<row_grid(B, H, T), NT, 0, st>>>(a);
  } else {
    rope_kernel<bf16><<<row_grid(B, H, T), NT, 0, st>>>(a);
  }
  return hipGetLastError();
}

hipError_t launch_rope_append(int dtype, int B, int H, int T, int D, int R, View k, View v, View kc,
                              View vc, const View *ks, const View *vs, const void *cos,
                              const void *sin, int64_t pos, hipStream_t st) {
  AppendArgs a{B, H, T, D, R, k, v, kc, vc, ks ? *ks : View{}, vs ? *vs : View{}, cos, sin, pos};
  const bool q8 = ks != nullptr;
  Probe pr_(q8 ? "rope_append_int8" : "rope_append", st);
  const dim3 g = row_grid(B, H, T);
  if (dtype == TSATTN_F32) {
    if (q8) rope_append_kernel<float, true><<<g, NT, 0, st>>>(a);
    else rope_append_kernel<float, false><<<g, NT, 0, st>>>(a);
  } else if (dtype == TSATTN_F16) {
    if (q8) rope_append_kernel<f16, true><<<g, NT, 0, st>>>(a);
    else rope_append_kernel<f16, false><<<g, NT, 0, st>>>(a);
  } else {
    if (q8) rope_append_kernel<bf16, true><<<g, NT, 0, st>>>(a);
    else rope_append_kernel<bf16, false><<<g, NT, 0, st>>>(a);
  }
  return hipGetLastError();
}

}  // namespace tsattn
