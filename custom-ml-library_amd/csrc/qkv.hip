// The cached MultiHeadAttention step before the attention, in one kernel:
// the three input projections (src/tensorsmith/nn/transformer.py:124-138,
// q = x Wq^T (+ bq), k = x Wk^T (+ bk), v = x Wv^T (+ bv), Linear.weight
// [out, in]), RoPE of q and k at positions pos .. pos + len - 1 (:139-141,
// rotary_embedding, attention.py:255-296) and the append of k and v to the
// cache (:142 -> KVCache.append, cache.py:54-86, int8 rows with fp32 row
// scales when the cache is quantised).
//
// One workgroup = one 32-channel tile of a head of q, k or v (16-bit
// caches; the whole head for int8 caches, whose quantiser needs the row
// maximum) for 32 rows (b, t) of x.  The embedding splits into 64-column
// chunks over eight accumulators (chunks v, v + 8, ... into accumulator v)
// that run out^T[n][r] += W[n][e] x[r][e] on MFMA 32x32x16 with W rows and
// x rows as row fragments, then sum in order 0..7 through LDS.  One-tile
// workgroups stage the fragments through per-wave LDS rings by DMA (whole
// cache lines per load instruction, three chunks ahead) and run two waves of
// four accumulators each, two workgroups per CU; whole-head workgroups load
// them directly and run eight waves of one accumulator.  Either way every accumulator sees the
// same chunks in the same order, so the projections are bit-identical
// across cache types.  The row blocks of one weight tile are consecutive in
// the XCD-local dispatch order, so they read the tile from HBM about once
// (the second read meets the first in that XCD's L2).  (For decode the weights dominate: (Hq + 2 Hkv) D E 2
// bytes.)  Wave 0 finishes: bias, rounding to the dtype (as the
// reference's Linear output), the rotation (lane (c, h) holds channels
// 8 g + 4 h .. + 3 of row c, so every channel pair is lane-local), then the
// row stores: q to its output, k and v into the cache (quantised per row
// with the reference's division for an int8 cache).
#include "mfma_common.h"
#include "rope_math.h"

namespace tsattn {
namespace {

constexpr int NACC = 8;  // chunk accumulators (summed in order)
#ifndef QKV_STAGES
#define QKV_STAGES 4
#endif
constexpr int QKV_NS = QKV_STAGES;  // ring stages per wave of the staged workgroups

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
// Threads per workgroup: two waves (four accumulators each) for staged
// one-tile workgroups, eight (one each) for whole heads.
template <int CT>
constexpr int qkv_threads() { return CT == 1 ? 128 : 512; }

// (Staged workgroups run two per CU, bounded by their LDS: one wave per SIMD.)
template <typename T, int D, int CT>
__global__ __launch_bounds__(qkv_threads<CT>(), 1) void qkv_rope_append_kernel(QkvArgs a) {
  constexpr int TILES = CT, NCB = D / 32 / CT;
  constexpr int NW = qkv_threads<CT>() / 64, APW = NACC / NW;  // waves, accumulators per wave
  static_assert(NCB * CT * 32 == D, "column blocks split the head");
  static_assert(APW * NW == NACC && (CT == 1 || APW == 1), "accumulators split over the waves");
  // CT == 1: per-wave staging rings (QKV_NS 8 KiB stages: 32 W rows and 32
  // x rows of 64 columns) during the loop, the partial tiles after it
  constexpr int RING = QKV_NS * 8192;
  constexpr int PART = NACC * TILES * 16 * 64 * 4;
  __shared__ __attribute__((aligned(1024))) char smem[CT == 1 ? (NW * RING > PART ? NW * RING : PART) : PART];
  auto part = reinterpret_cast<float (*)[TILES][16][64]>(smem);

  const int lane = threadIdx.x & 63, c = lane & 31, h = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // logical id = ((cb nslot) + slot) rblocks + rb: the row blocks of a
  // weight tile are consecutive, and consecutive logical ids share an XCD
  const int nslot = a.Hq + 2 * a.Hkv, rblocks = (a.rows + 31) / 32;
  const int logical = xcd_remap(blockIdx.x, static_cast<int>(gridDim.x));
  const int rb = logical % rblocks, rest = logical / rblocks;
  const int slot = rest % nslot, cb = rest / nslot;
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
  f32x16 acc[APW][TILES];
#pragma unroll
  for (int v = 0; v < APW; ++v)
#pragma unroll
    for (int t = 0; t < TILES; ++t) acc[v][t] = f32x16{};
  if constexpr (CT == 1) {
    // Staged through LDS: a wave takes the 64-column chunks w, w + NW, ...
    // of the embedding (chunk ch into accumulator ch % 8: its accumulator
    // k % APW for its k-th chunk) and DMAs each chunk's 32 W rows and 32 x
    // rows into its own QKV_NS-stage ring, QKV_NS - 1 chunks ahead of the
    // one it multiplies, eight rows of 128 bytes (whole cache lines) per load
    // instruction -- direct fragment loads touch 32 lines each, and the
    // address unit, not HBM, bounded them.  (At E 4096, 48 heads of 128 and
    // 64 rows: four waves one chunk ahead 17.0 us; two waves three ahead, 1.5x
    // the bytes in flight per CU, 16.2 us; four ahead 16.5 us.)  In the ring,
    // 16-byte unit u of row r holds unit u ^ (r % 8) of the chunk
    // (conflict-free fragment reads); columns past the embedding, and rows
    // past the last, read zeros; the loads past the wave's last chunk land in
    // the stage of a chunk already multiplied, which nothing reads again.  The
    // loop needs no barrier: no wave reads another's ring.
    const uint32_t sbase = lds_addr(smem) + w * RING;
    const int nch = (a.E + 63) / 64;
    const int mine = nch > w ? (nch - 1 - w) / NW + 1 : 0;  // this wave's chunks
    const int lr = lane >> 3, gu = (lane & 7) ^ lr;  // row within 8, global unit
    const u32x4 wdesc = make_desc(W, static_cast<uint32_t>(32) * a.E * 2);
    const u32x4 xdesc = make_desc(uniform_ptr(a.x), static_cast<uint32_t>(xext * 2));
    uint32_t wv[4], xv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 8 * i + lr;  // W row (channel) and x row of this lane's DMA piece
      wv[i] = (static_cast<uint32_t>(row) * a.E + 8 * gu) * 2;
      const int xr_ = r0 + row;
      const int xrr = xr_ < a.rows ? xr_ : a.rows - 1;
      const int xb_ = xrr / a.len, xt_ = xrr - xb_ * a.len;
      xv[i] = (static_cast<uint32_t>(xb_ * a.xs_b + xt_ * a.xs_t + 8 * gu) * 2) |
              (xr_ < a.rows ? 0u : 0x80000000u);
    }
    // chunk k of this wave (k-th of `mine`; past them: zeros) into the stage at st
    auto issue = [&](int k, uint32_t st) {
      const int ch = w + NW * k;
      const bool real = k < mine;
      const uint32_t col = static_cast<uint32_t>(ch) * 64 + 8 * gu;  // first column of the lane's unit
      const uint32_t far = (real && col < static_cast<uint32_t>(a.E)) ? 0u : 0x80000000u;
      const uint32_t soff = real ? static_cast<uint32_t>(ch) * 128 : 0u;
#pragma unroll
      for (int i = 0; i < 4; ++i) dma16(wdesc, st + i * 1024, wv[i] | far, soff);
#pragma unroll
      for (int i = 0; i < 4; ++i) dma16(xdesc, st + 4096 + i * 1024, xv[i] | far, soff);
    };
    // fragment of k-step s (0..3) of a staged 32 x 64 tile: row c, unit 2 s + h
    const uint32_t fo = static_cast<uint32_t>(c) * 128;
    const uint32_t last = sbase + (QKV_NS - 1) * 8192;
    uint32_t ist = sbase;  // stage of the next chunk issued
    int rd = 0;            // ring offset of the stage of the chunk multiplied
    auto step = [&](int k, f32x16 &ac) {
      issue(k + QKV_NS - 1, ist);
      ist = ist == last ? sbase : ist + 8192;
      wait_vm_n<8 * (QKV_NS - 1)>();  // chunk k has landed; the next chunks' loads stay in flight
      const char *stg = smem + w * RING + rd;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint32_t u = static_cast<uint32_t>((2 * s + h) ^ (c & 7)) * 16;
        const u32x4 wf = *reinterpret_cast<const u32x4 *>(stg + fo + u);
        const u32x4 xf = *reinterpret_cast<const u32x4 *>(stg + 4096 + fo + u);
        ac = mfma32<T>(wf, xf, ac);
      }
      wait_lgkm0();  // reads of this stage done before chunk k + QKV_NS overwrites it
      rd = rd == (QKV_NS - 1) * 8192 ? 0 : rd + 8192;
    };
    static_assert(8 * (QKV_NS - 1) <= 63 && QKV_NS >= 2, "the ring's loads fit the vector memory counter");
#pragma unroll
    for (int k = 0; k < QKV_NS - 1; ++k) {
      issue(k, ist);
      ist = ist == last ? sbase : ist + 8192;
    }
    for (int k = 0; k < mine; k += APW) {
#pragma unroll
      for (int v = 0; v < APW; ++v)
        if (k + v < mine) step(k + v, acc[v][0]);
    }
    wait_vm_n<0>();
    __syncthreads();  // every ring read before the partial tiles reuse the LDS
  } else {
    // Direct fragment loads (whole-head workgroups, whose fragments would not
    // fit the rings): the same chunks per wave and the same MFMA order as the
    // staged path, so the projections are bit-identical across cache types;
    // chunk loads double-buffered, columns past the embedding read zeros.
    const int nks = a.E / 16;
    const int nch = (a.E + 63) / 64;
    const int mine = nch > w ? (nch - 1 - w) / NW + 1 : 0;
    u32x4 xb[2][4], wb[2][4][TILES];
    auto load = [&](int k, int buf) {
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const int ks = 4 * (w + NW * k) + s4;
        const bool in = k < mine && ks < nks;
        const uint32_t ko = static_cast<uint32_t>(ks) * 32;
        xb[buf][s4] = buf_load16(xr, in ? xo + ko : 0x80000000u);
#pragma unroll
        for (int t = 0; t < TILES; ++t) wb[buf][s4][t] = buf_load16(wr, in ? wo + t * wt + ko : 0x80000000u);
      }
    };
    auto compute = [&](int buf) {
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
        for (int t = 0; t < TILES; ++t) acc[0][t] = mfma32<T>(wb[buf][s4][t], xb[buf][s4], acc[0][t]);
    };
    load(0, 0);
    for (int k = 0; k < mine; k += 2) {
      load(k + 1, 1);  // (past this wave's chunks: zeros, not used)
      compute(0);
      if (k + 1 < mine) {
        load(k + 2, 0);
        compute(1);
      }
    }
  }
#pragma unroll
  for (int v = 0; v < APW; ++v)
#pragma unroll
    for (int t = 0; t < TILES; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) part[w + NW * v][t][e][lane] = acc[v][t][e];
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
      for (int v = 0; v < NACC; ++v) s += part[v][t][e][lane];
      // the product in the dtype, then + bias in the dtype (functional.py:75-77)
      T yv = static_cast<T>(s);
      if (bias)
        yv = static_cast<T>(static_cast<float>(yv) +
                            static_cast<float>(bias[head * D + c0 + 32 * t + 8 * (e >> 2) + 4 * h + (e & 3)]));
      y[t][e] = yv;
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
  const dim3 grid(static_cast<unsigned>((heads_q + 2 * heads_kv) * ncb * rblocks));
  const dim3 block(ks ? qkv_threads<4>() : qkv_threads<1>());
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
