// The cached MultiHeadAttention step before the attention, in one kernel:
// the three input projections (src/tensorsmith/nn/transformer.py:124-138,
// q = x Wq^T (+ bq), k = x Wk^T (+ bk), v = x Wv^T (+ bv), Linear.weight
// [out, in]), RoPE of q and k at positions pos .. pos + len - 1 (:139-141,
// rotary_embedding, attention.py:255-296) and the append of k and v to the
// cache (:142 -> KVCache.append, cache.py:54-86, int8 rows with fp32 row
// scales when the cache is quantised).
//
// One workgroup = one head of q, k or v for 32 rows (b, t) of x; its eight
// waves split the embedding (k-steps of 16 in turn) and run
// out^T[n][r] += W[n][e] x[r][e] on MFMA 32x32x16 -- W rows and x rows are
// both row fragments, read straight from memory, two k-steps of loads in
// flight ahead of the MFMAs -- then sum their partial tiles through LDS.
// (For decode the weights dominate: (Hq + 2 Hkv) D E 2 bytes streamed by a
// few hundred waves, so the loads have to be deep.)  Wave 0 finishes: bias,
// rounding to the dtype (as the
// reference's Linear output), the rotation (lane (c, h) holds channels
// 8 g + 4 h .. + 3 of row c, so every channel pair is lane-local), then the
// row stores: q to its output, k and v into the cache (quantised per row
// with the reference's division for an int8 cache).
#include "mfma_common.h"
#include "rope_math.h"

namespace tsattn {
namespace {

constexpr int NT = 512;
constexpr int NW = NT / 64;
constexpr int KU = 2;  // k-steps per wave and load batch

struct QkvArgs {
  int rows, len, E, Hq, Hkv, rope;
  const void *x;
  int64_t xs_b, xs_t;  // element strides of x between batch rows and between positions
  const void *w[3], *bias[3];  // q, k, v
  View q, kc, vc, ks, vs;      // ks.data == nullptr: 16-bit caches
  const void *cos, *sin;
  int64_t pos;
};

// The same pointer in scalar registers (the compiler cannot prove a value
// selected by a block-uniform index uniform, and a buffer resource in vector
// registers turns every load into a loop over the lanes' values).
__device__ __forceinline__ const void *uniform_ptr(const void *p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const void *>((static_cast<uint64_t>(hi) << 32) | lo);
}

// CT: 32-channel tiles of the head per workgroup -- D / 32 (the whole head,
// which the int8 quantiser's row maximum needs), or fewer for 16-bit caches,
// so that more workgroups share the weight stream.
template <typename T, int D, int CT>
__global__ __launch_bounds__(NT, 1) void qkv_rope_append_kernel(QkvArgs a) {
  constexpr int TILES = CT, NCB = D / 32 / CT;
  static_assert(NCB * CT * 32 == D, "column blocks split the head");
  __shared__ float part[NW][TILES][16][64];

  const int lane = threadIdx.x & 63, c = lane & 31, h = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nslot = a.Hq + 2 * a.Hkv;
  const int slot = blockIdx.x % nslot, rest = blockIdx.x / nslot;
  const int cb = rest % NCB, rb = rest / NCB;
  const int c0 = 32 * CT * cb;  // first channel of this workgroup's columns
  const int kind = slot < a.Hq ? 0 : (slot < a.Hq + a.Hkv ? 1 : 2);
  const int head = kind == 0 ? slot : (kind == 1 ? slot - a.Hq : slot - a.Hq - a.Hkv);
  const void *wk = kind == 0 ? a.w[0] : (kind == 1 ? a.w[1] : a.w[2]);
  const T *W = static_cast<const T *>(
      uniform_ptr(static_cast<const T *>(wk) + (static_cast<int64_t>(head) * D + c0) * a.E));
  const int r0 = rb * 32;

  // row r = r0 + c of x is (b, t) = (r / len, r % len); rows past the last
  // read as zeros (offsets past the buffer range) and are not stored
  const int r = r0 + c;
  const bool live = r < a.rows;
  const int rr = live ? r : a.rows - 1;
  const int b = rr / a.len, tt = rr - b * a.len;
  const int64_t xext = (static_cast<int64_t>(a.rows / a.len) - 1) * a.xs_b +
                       (static_cast<int64_t>(a.len) - 1) * a.xs_t + a.E;
  const rsrc_t xr = make_rsrc(uniform_ptr(a.x), static_cast<uint32_t>(xext * 2));
  const rsrc_t wr = make_rsrc(W, static_cast<uint32_t>(32 * CT) * a.E * 2);
  const uint32_t xo = (static_cast<uint32_t>(b * a.xs_b + tt * a.xs_t + 8 * h) * 2) |
                      (live ? 0u : 0x80000000u);
  const uint32_t wo = (static_cast<uint32_t>(c) * a.E + 8 * h) * 2;
  const uint32_t wt = 32u * a.E * 2;  // bytes between 32-row tiles of W
  f32x16 acc[TILES];
#pragma unroll
  for (int t = 0; t < TILES; ++t) acc[t] = f32x16{};
  // k-steps w, w + NW, ...: batches of KU k-steps in two register sets, a
  // batch's loads issued a batch ahead of its MFMAs; k-steps past the
  // embedding read zeros (offsets past the buffer ranges), so every wave runs
  // the same even number of batches without branches
  const int nks = a.E / 16;
  const int nb = (nks + 2 * NW * KU - 1) / (2 * NW * KU) * 2;
  u32x4 xb[2][KU], wb[2][KU][TILES];
  auto load = [&](int bi, int buf) {
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int ks = (bi * KU + u) * NW + w;
      const bool in = ks < nks;
      const uint32_t ko = static_cast<uint32_t>(ks) * 32;
      xb[buf][u] = buf_load16(xr, in ? xo + ko : 0x80000000u);
#pragma unroll
      for (int t = 0; t < TILES; ++t) wb[buf][u][t] = buf_load16(wr, in ? wo + t * wt + ko : 0x80000000u);
    }
  };
  auto compute = [&](int buf) {
#pragma unroll
    for (int u = 0; u < KU; ++u)
#pragma unroll
      for (int t = 0; t < TILES; ++t) acc[t] = mfma32<T>(wb[buf][u][t], xb[buf][u], acc[t]);
  };
  load(0, 0);
  for (int bi = 0; bi < nb; bi += 2) {
    load(bi + 1, 1);
    compute(0);
    load(bi + 2, 0);  // (past the last batch: zeros, never used)
    compute(1);
  }
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) part[w][t][e][lane] = acc[t][e];
  __syncthreads();
  if (w != 0) return;

  const int64_t prow = a.pos + tt;
  const T *bias = static_cast<const T *>(a.bias[kind]);
  // y[t][e]: channel n = c0 + 32 t + 8 (e / 4) + 4 h + e % 4 of the head
  T y[TILES][16];
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      float s = 0.f;
#pragma unroll
      for (int v = 0; v < NW; ++v) s += part[v][t][e][lane];
      if (bias) s += static_cast<float>(bias[head * D + c0 + 32 * t + 8 * (e >> 2) + 4 * h + (e & 3)]);
      y[t][e] = static_cast<T>(s);
    }
  if (kind < 2 && a.rope) {
    const T *cs = static_cast<const T *>(a.cos) + prow * (D / 2);
    const T *sn = static_cast<const T *>(a.sin) + prow * (D / 2);
#pragma unroll
    for (int t = 0; t < TILES; ++t)
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        const int pair = (c0 + 32 * t + 8 * (e >> 2) + 4 * h + (e & 3)) / 2;
        rotate_pair(y[t][e], y[t][e + 1], cs[pair], sn[pair], false);
      }
  }
  auto pack4 = [&](int t, int g) {
    return u32x2{static_cast<uint32_t>(__builtin_bit_cast(uint16_t, y[t][4 * g])) |
                     (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, y[t][4 * g + 1])) << 16),
                 static_cast<uint32_t>(__builtin_bit_cast(uint16_t, y[t][4 * g + 2])) |
                     (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, y[t][4 * g + 3])) << 16)};
  };
  if (kind == 0) {
    T *q = static_cast<T *>(const_cast<void *>(a.q.data)) + b * a.q.s0 + head * a.q.s1 +
           static_cast<int64_t>(tt) * a.q.s2 + c0;
    if (live)
#pragma unroll
      for (int t = 0; t < TILES; ++t)
#pragma unroll
        for (int g = 0; g < 4; ++g) *reinterpret_cast<u32x2 *>(q + 32 * t + 8 * g + 4 * h) = pack4(t, g);
    return;
  }
  const View &cv = kind == 1 ? a.kc : a.vc;
  const int64_t crow = b * cv.s0 + head * cv.s1 + prow * cv.s2 + c0;
  if (NCB > 1 || !a.ks.data) {  // 16-bit caches (the host splits only those)
    T *dst = static_cast<T *>(const_cast<void *>(cv.data)) + crow;
    if (live)
#pragma unroll
      for (int t = 0; t < TILES; ++t)
#pragma unroll
        for (int g = 0; g < 4; ++g) *reinterpret_cast<u32x2 *>(dst + 32 * t + 8 * g + 4 * h) = pack4(t, g);
    return;
  }
  if constexpr (NCB == 1) {
  // int8 cache (cache.py:73-77): s = max(max |x| / 127, 1e-8), q = rint(x / s),
  // fp32 arithmetic on the row in the cache dtype; lanes c and c + 32 hold
  // the two halves of row c.
  float m = 0.f;
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) m = fmaxf(m, fabsf(static_cast<float>(y[t][e])));
  m = fmaxf(m, __shfl_xor(m, 32, 64));
  const float sc = fmaxf(m / 127.f, 1e-8f);
  int8_t *dst = static_cast<int8_t *>(const_cast<void *>(cv.data)) + crow;
  if (live) {
#pragma unroll
    for (int t = 0; t < TILES; ++t)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        uint32_t word = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          word |= (static_cast<uint32_t>(static_cast<int32_t>(rintf(static_cast<float>(y[t][4 * g + j]) / sc))) &
                   0xFFu) << (8 * j);
        *reinterpret_cast<uint32_t *>(dst + 32 * t + 8 * g + 4 * h) = word;
      }
    const View &sv = kind == 1 ? a.ks : a.vs;
    if (h == 0)
      static_cast<float *>(const_cast<void *>(sv.data))[b * sv.s0 + head * sv.s1 + prow * sv.s2] = sc;
  }
  }
}

}  // namespace

hipError_t launch_qkv_rope_append(int dtype, int batch, int len, int embed, int heads_q, int heads_kv,
                                  int dim, View x, const void *const w[3], const void *const bias[3],
                                  View q, View kc, View vc, const View *ks, const View *vs, const void *cos,
                                  const void *sin, int64_t pos, hipStream_t st) {
  QkvArgs a{batch * len, len, embed, heads_q, heads_kv, cos != nullptr, x.data, x.s0, x.s2,
            {w[0], w[1], w[2]}, {bias[0], bias[1], bias[2]}, q, kc, vc,
            ks ? *ks : View{nullptr, 0, 0, 0}, vs ? *vs : View{nullptr, 0, 0, 0}, cos, sin, pos};
  const int rblocks = (a.rows + 31) / 32;
  // 16-bit caches: one 32-channel tile of a head per workgroup; int8 caches:
  // the whole head (its row maximum)
  const int ncb = ks ? 1 : dim / 32;
  const dim3 grid(static_cast<unsigned>((heads_q + 2 * heads_kv) * ncb * rblocks)), block(NT);
  Probe pr_(ks ? "qkv_rope_append_int8" : "qkv_rope_append", st);
  if (dtype == TSATTN_BF16) {
    if (dim == 128) {
      if (ks) qkv_rope_append_kernel<bf16, 128, 4><<<grid, block, 0, st>>>(a);
      else qkv_rope_append_kernel<bf16, 128, 1><<<grid, block, 0, st>>>(a);
    } else {
      if (ks) qkv_rope_append_kernel<bf16, 64, 2><<<grid, block, 0, st>>>(a);
      else qkv_rope_append_kernel<bf16, 64, 1><<<grid, block, 0, st>>>(a);
    }
  } else {
    if (dim == 128) {
      if (ks) qkv_rope_append_kernel<f16, 128, 4><<<grid, block, 0, st>>>(a);
      else qkv_rope_append_kernel<f16, 128, 1><<<grid, block, 0, st>>>(a);
    } else {
      if (ks) qkv_rope_append_kernel<f16, 64, 2><<<grid, block, 0, st>>>(a);
      else qkv_rope_append_kernel<f16, 64, 1><<<grid, block, 0, st>>>(a);
    }
  }
  return hipGetLastError();
}

}  // namespace tsattn
