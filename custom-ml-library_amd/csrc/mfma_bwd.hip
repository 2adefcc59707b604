// Attention backward for gfx950 with MFMA 32x32x16 (f16/bf16 in, fp32
// accumulate).  Follows the reference's streaming VJP (src/tensorsmith/nn/
// attention.py:220-247):
//   delta_i = sum_d dO_id O_id                     (row_delta_kernel)
//   P_ij = exp(S_ij - LSE_i), dS_ij = P_ij (dP_ij - delta_i), dP = dO V^T
//   dV = P^T dO, dK = scale dS^T Q                 (dkdv_kernel)
//   dQ = scale dS K                                (dq_kernel)
// dK/dV and dQ are produced by two kernels that each own their output tile,
// so every gradient element is written exactly once: no atomics, bitwise
// deterministic results (checkpoint recompute reproduces them exactly).
// The dK/dV kernel sums the query heads of a GQA group itself (:245-247).
#include "mfma_common.h"

namespace tsattn {
namespace {

constexpr int NT = 256;

struct BwdArgs {
  Problem p;
  View q, k, v, o, dout, dq, dk, dv;
  const float *lse;
  float *delta;
  float sl;     // scale * log2(e)
  float scale;  // final gradient scale
};

template <typename T>
__device__ __forceinline__ T *mut(View v) {
  return static_cast<T *>(const_cast<void *>(v.data));
}

// ---------------------------------------------------------------------------
// delta = rowsum(dO * O) in fp32; D/8 threads per row.
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(NT) void row_delta_kernel(BwdArgs a) {
  constexpr int TPR = D / 8;
  constexpr int RPB = NT / TPR;
  const Problem &p = a.p;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / TPR;
  const int part = threadIdx.x % TPR;
  const int64_t rows = static_cast<int64_t>(p.B) * p.Hq * p.Sq;
  float s = 0.f;
  if (row < rows) {
    const int i = static_cast<int>(row % p.Sq);
    const int64_t bh = row / p.Sq;
    const int hq = static_cast<int>(bh % p.Hq), b = static_cast<int>(bh / p.Hq);
    const T *op = static_cast<const T *>(a.o.data) + b * a.o.s0 + hq * a.o.s1 +
                  static_cast<int64_t>(i) * a.o.s2 + part * 8;
    const T *gp = static_cast<const T *>(a.dout.data) + b * a.dout.s0 + hq * a.dout.s1 +
                  static_cast<int64_t>(i) * a.dout.s2 + part * 8;
    const u32x4 ov = ld16(op), gv = ld16(gp);
    const T *oe = reinterpret_cast<const T *>(&ov);
    const T *ge = reinterpret_cast<const T *>(&gv);
#pragma unroll
    for (int e = 0; e < 8; ++e) s += static_cast<float>(oe[e]) * static_cast<float>(ge[e]);
  }
#pragma unroll
  for (int m = TPR / 2; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
  if (row < rows && part == 0) a.delta[row] = s;
}

// ---------------------------------------------------------------------------
// dK / dV: one workgroup = 128 keys of one (b, kv head); wave w owns keys
// kw..kw+31.  Query tiles of 64 rows (all query heads of the group) stream
// through LDS twice: row-major (A operand of S = Q K^T and dP = dO V^T) and
// transposed (A operand of dV^T = dO^T P and dK^T = Q^T dS).
// ---------------------------------------------------------------------------
constexpr int KB = 128;  // keys per workgroup
constexpr int QT = 64;   // query rows per tile

template <typename T, int D>
struct KVLayout {
  static constexpr int RSTR = D + 8;   // row-major stride (elements)
  static constexpr int TSTR = QT + 4;  // transposed stride (elements)
  static constexpr int R_BYTES = QT * RSTR * 2;
  static constexpr int T_BYTES = D * TSTR * 2;
  // stage: Q | dO | Q^T | dO^T | lse2[QT] | delta[QT]
  static constexpr int OFF_G = R_BYTES;
  static constexpr int OFF_QT = 2 * R_BYTES;
  static constexpr int OFF_GT = 2 * R_BYTES + T_BYTES;
  static constexpr int OFF_L = 2 * R_BYTES + 2 * T_BYTES;
  static constexpr int OFF_D = OFF_L + QT * 4;
  static constexpr int STAGE = OFF_D + QT * 4;
  static constexpr int BYTES = 2 * STAGE;
};

template <typename T, int D>
__global__ __launch_bounds__(NT, 1) void dkdv_kernel(BwdArgs a) {
  using L = KVLayout<T, D>;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const Problem &p = a.p;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, c = lane & 31, h = lane >> 5;
  const int n_kb = (p.Sk + KB - 1) / KB;
  const int total = n_kb * p.Hkv * p.B;
  const int logical = xcd_remap(blockIdx.x, total);
  const int bh = logical / n_kb;
  const int kb = logical - bh * n_kb;  // early key blocks see the most queries: run them first
  const int b = bh / p.Hkv, hk = bh - b * p.Hkv;
  const int k0 = kb * KB, kw = k0 + 32 * w, key = kw + c;
  const int kv_end = kv_end_for(p, b);
  const bool keymask = p.mask.kind == TSATTN_MASK_BOOL && !(p.kv_prefix && p.kv_prefix[b]);
  const bool key_live = key < kv_end &&
                        (!keymask || static_cast<const uint8_t *>(p.mask.data)
                                         [b * p.mask.s0 + static_cast<int64_t>(key) * p.mask.s3]);

  // K and V rows of this lane's key as B operands (K^T / V^T with N = key).
  u32x4 kf[D / 16], vf[D / 16];
  {
    const T *kp = static_cast<const T *>(a.k.data) + b * a.k.s0 + hk * a.k.s1 +
                  static_cast<int64_t>(key) * a.k.s2;
    const T *vp = static_cast<const T *>(a.v.data) + b * a.v.s0 + hk * a.v.s1 +
                  static_cast<int64_t>(key) * a.v.s2;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      kf[ks] = key < kv_end ? ld16(kp + ks * 16 + h * 8) : u32x4{0, 0, 0, 0};
      vf[ks] = key < kv_end ? ld16(vp + ks * 16 + h * 8) : u32x4{0, 0, 0, 0};
    }
  }

  // Query tiles: only rows that can see a key of this block (causal).
  int q_start = 0;
  if (p.causal) {
    int64_t s = static_cast<int64_t>(k0) - p.offset;
    q_start = s <= 0 ? 0 : static_cast<int>(s < p.Sq ? s : p.Sq);
    q_start = (q_start / QT) * QT;
  }
  const int n_qt = k0 < kv_end ? (p.Sq - q_start + QT - 1) / QT : 0;
  const int n_iter = n_qt * p.rep;

  TileRegs<T, D, QT> qreg, greg;
  float lreg = 0.f;  // thread < QT: lse2 of row; QT <= thread < 2*QT: delta
  auto load_iter = [&](int itn) {
    const int r = itn / n_qt, q0 = q_start + (itn - r * n_qt) * QT;
    const int hq = hk * p.rep + r;
    qreg.load(static_cast<const T *>(a.q.data) + b * a.q.s0 + hq * a.q.s1, a.q.s2, q0, p.Sq, tid);
    greg.load(static_cast<const T *>(a.dout.data) + b * a.dout.s0 + hq * a.dout.s1, a.dout.s2, q0,
              p.Sq, tid);
    if (tid < 2 * QT) {
      const int row = q0 + (tid & (QT - 1));
      const int64_t idx = (static_cast<int64_t>(b) * p.Hq + hq) * p.Sq + row;
      if (row >= p.Sq) {
        lreg = 0.f;
      } else if (tid < QT) {
        const float v = a.lse[idx];
        lreg = isfinite(v) ? v * kLog2e : 0.f;  // safe_lse (attention.py:231)
      } else {
        lreg = a.delta[idx];
      }
    }
  };
  auto store_iter = [&](int stage) {
    unsigned char *s = smem + stage * L::STAGE;
    qreg.store_rows(reinterpret_cast<T *>(s), L::RSTR, tid);
    greg.store_rows(reinterpret_cast<T *>(s + L::OFF_G), L::RSTR, tid);
    qreg.store_cols(reinterpret_cast<T *>(s + L::OFF_QT), L::TSTR, tid);
    greg.store_cols(reinterpret_cast<T *>(s + L::OFF_GT), L::TSTR, tid);
    if (tid < 2 * QT) reinterpret_cast<float *>(s + L::OFF_L)[tid] = lreg;
  };

  f32x16 dk_acc[D / 32], dv_acc[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) dk_acc[dt] = dv_acc[dt] = f32x16{};
  const float sl = a.sl;

  if (n_iter > 0) {
    load_iter(0);
    store_iter(0);
  }
  __syncthreads();

  for (int itn = 0; itn < n_iter; ++itn) {
    const int stage = itn & 1;
    const int q0 = q_start + (itn % n_qt) * QT;
    if (itn + 1 < n_iter) load_iter(itn + 1);

    // Does any (query row of this tile, key of this wave) pair survive?
    const bool wave_live = kw < kv_end && (!p.causal || static_cast<int64_t>(q0) + QT - 1 + p.offset >= kw);
    if (wave_live) {
      const unsigned char *s = smem + stage * L::STAGE;
      const T *ql = reinterpret_cast<const T *>(s);
      const T *gl = reinterpret_cast<const T *>(s + L::OFF_G);
      const T *qtl = reinterpret_cast<const T *>(s + L::OFF_QT);
      const T *gtl = reinterpret_cast<const T *>(s + L::OFF_GT);
      const float *ll = reinterpret_cast<const float *>(s + L::OFF_L);
      const float *dl = reinterpret_cast<const float *>(s + L::OFF_D);
      const bool edge = (p.causal && static_cast<int64_t>(q0) + p.offset < kw + 31) ||
                        kw + 32 > kv_end || q0 + QT > p.Sq || keymask;

      unsigned pp[4][4], pd[4][4];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        f32x16 sacc = f32x16{}, dpacc = f32x16{};
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks) {
          const int off = (sub * 32 + c) * L::RSTR + ks * 16 + h * 8;
          sacc = mfma32<T>(ld16(ql + off), kf[ks], sacc);
          dpacc = mfma32<T>(ld16(gl + off), vf[ks], dpacc);
        }
        // sacc[i] = S[q0 + 32 sub + crow(i, h)][key]
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int rq = sub * 32 + g * 8 + h * 4;
          const float4 l4 = *reinterpret_cast<const float4 *>(ll + rq);
          const float4 d4 = *reinterpret_cast<const float4 *>(dl + rq);
          const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
          const float dv4[4] = {d4.x, d4.y, d4.z, d4.w};
          float pv[4], dsv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int i = g * 4 + e;
            bool ok = true;
            if (edge) {
              const int qrow = q0 + rq + e;
              ok = key_live && qrow < p.Sq &&
                   (!p.causal || static_cast<int64_t>(qrow) + p.offset >= key);
            }
            pv[e] = ok ? fast_exp2(fmaf(sacc[i], sl, -lv[e])) : 0.f;
            dsv[e] = pv[e] * (dpacc[i] - dv4[e]);
          }
          // element pair (i, i+1) -> kstep 2*sub + (i >> 3), dword (i & 7) >> 1
          const int ks = 2 * sub + (g >> 1), dw = (g & 1) * 2;
          pp[ks][dw] = pack2<T>(pv[0], pv[1]);
          pp[ks][dw + 1] = pack2<T>(pv[2], pv[3]);
          pd[ks][dw] = pack2<T>(dsv[0], dsv[1]);
          pd[ks][dw + 1] = pack2<T>(dsv[2], dsv[3]);
        }
      }
      // dV^T += dO^T P, dK^T += Q^T dS over the 64 query rows (4 ksteps of 16).
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const u32x4 bp = {pp[ks][0], pp[ks][1], pp[ks][2], pp[ks][3]};
        const u32x4 bd = {pd[ks][0], pd[ks][1], pd[ks][2], pd[ks][3]};
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
          const int off = (dt * 32 + c) * L::TSTR + ks * 16 + h * 4;
          const u32x2 glo = ld8(gtl + off), ghi = ld8(gtl + off + 8);
          const u32x2 qlo = ld8(qtl + off), qhi = ld8(qtl + off + 8);
          dv_acc[dt] = mfma32<T>(u32x4{glo[0], glo[1], ghi[0], ghi[1]}, bp, dv_acc[dt]);
          dk_acc[dt] = mfma32<T>(u32x4{qlo[0], qlo[1], qhi[0], qhi[1]}, bd, dk_acc[dt]);
        }
      }
    }

    if (itn + 1 < n_iter) store_iter(stage ^ 1);
    __syncthreads();
  }

  if (key >= p.Sk) return;
  // lane holds dK^T[d = 32 dt + crow(i, h)][key]
  T *dkp = mut<T>(a.dk) + b * a.dk.s0 + hk * a.dk.s1 + static_cast<int64_t>(key) * a.dk.s2;
  T *dvp = mut<T>(a.dv) + b * a.dv.s0 + hk * a.dv.s1 + static_cast<int64_t>(key) * a.dv.s2;
  const float sc = a.scale;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = dt * 32 + g * 8 + h * 4;
      *reinterpret_cast<u32x2 *>(dkp + d) =
          u32x2{pack2<T>(dk_acc[dt][g * 4] * sc, dk_acc[dt][g * 4 + 1] * sc),
                pack2<T>(dk_acc[dt][g * 4 + 2] * sc, dk_acc[dt][g * 4 + 3] * sc)};
      *reinterpret_cast<u32x2 *>(dvp + d) =
          u32x2{pack2<T>(dv_acc[dt][g * 4], dv_acc[dt][g * 4 + 1]),
                pack2<T>(dv_acc[dt][g * 4 + 2], dv_acc[dt][g * 4 + 3])};
    }
  }
}

// ---------------------------------------------------------------------------
// dQ: one workgroup = 128 query rows of one (b, q head); wave w owns 32 rows.
// Key tiles of 64 stream through LDS as K, V (A operands of S^T = K Q^T and
// dP^T = V dO^T) and K^T (A operand of dQ^T = K^T dS^T).
// ---------------------------------------------------------------------------
constexpr int QB = 128;  // query rows per workgroup
constexpr int KT = 64;   // keys per tile

template <typename T, int D>
struct QLayout {
  static constexpr int RSTR = D + 8;
  static constexpr int TSTR = KT + 4;
  static constexpr int R_ELEMS = KT * RSTR;
  static constexpr int T_ELEMS = D * TSTR;
  static constexpr int STAGE = 2 * R_ELEMS + T_ELEMS;  // K | V | K^T
  static constexpr int BYTES = 2 * STAGE * 2;
};

template <typename T, int D>
__global__ __launch_bounds__(NT, 1) void dq_kernel(BwdArgs a) {
  using L = QLayout<T, D>;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  T *lds = reinterpret_cast<T *>(smem);
  const Problem &p = a.p;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, c = lane & 31, h = lane >> 5;
  const int n_qb = (p.Sq + QB - 1) / QB;
  const int total = n_qb * p.Hq * p.B;
  const int logical = xcd_remap(blockIdx.x, total);
  const int bh = logical / n_qb;
  const int qb = n_qb - 1 - (logical - bh * n_qb);
  const int b = bh / p.Hq, hq = bh - b * p.Hq, hk = hq / p.rep;
  const int q0 = qb * QB, qw = q0 + 32 * w, qrow = qw + c;
  const int kv_end = kv_end_for(p, b);
  const bool keymask = p.mask.kind == TSATTN_MASK_BOOL && !(p.kv_prefix && p.kv_prefix[b]);

  int64_t lim = kv_end, wlim = kv_end;
  if (p.causal) {
    lim = min(lim, static_cast<int64_t>(min(q0 + QB, p.Sq) - 1) + p.offset + 1);
    wlim = min(wlim, static_cast<int64_t>(min(qw + 32, p.Sq) - 1) + p.offset + 1);
  }
  if (qw >= p.Sq) wlim = 0;
  const int n_tiles = lim > 0 ? static_cast<int>((lim + KT - 1) / KT) : 0;
  const int w_tiles = wlim > 0 ? static_cast<int>((wlim + KT - 1) / KT) : 0;

  u32x4 qf[D / 16], gf[D / 16];
  float lse2 = 0.f, delta = 0.f;
  {
    const T *qp = static_cast<const T *>(a.q.data) + b * a.q.s0 + hq * a.q.s1 +
                  static_cast<int64_t>(qrow) * a.q.s2;
    const T *gp = static_cast<const T *>(a.dout.data) + b * a.dout.s0 + hq * a.dout.s1 +
                  static_cast<int64_t>(qrow) * a.dout.s2;
    const bool ok = qrow < p.Sq;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      qf[ks] = ok ? ld16(qp + ks * 16 + h * 8) : u32x4{0, 0, 0, 0};
      gf[ks] = ok ? ld16(gp + ks * 16 + h * 8) : u32x4{0, 0, 0, 0};
    }
    if (ok) {
      const int64_t idx = (static_cast<int64_t>(b) * p.Hq + hq) * p.Sq + qrow;
      const float lv = a.lse[idx];
      lse2 = isfinite(lv) ? lv * kLog2e : 0.f;
      delta = a.delta[idx];
    }
  }

  const T *kbase = static_cast<const T *>(a.k.data) + b * a.k.s0 + hk * a.k.s1;
  const T *vbase = static_cast<const T *>(a.v.data) + b * a.v.s0 + hk * a.v.s1;
  TileRegs<T, D, KT> kreg, vreg;
  auto load_tile = [&](int kv0) {
    kreg.load(kbase, a.k.s2, kv0, kv_end, tid);
    vreg.load(vbase, a.v.s2, kv0, kv_end, tid);
  };
  auto store_tile = [&](int stage) {
    T *s = lds + stage * L::STAGE;
    kreg.store_rows(s, L::RSTR, tid);
    vreg.store_rows(s + L::R_ELEMS, L::RSTR, tid);
    kreg.store_cols(s + 2 * L::R_ELEMS, L::TSTR, tid);
  };

  f32x16 acc[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) acc[dt] = f32x16{};
  const float sl = a.sl;
  const uint8_t *kmask = static_cast<const uint8_t *>(p.mask.data);

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int it = 0; it < n_tiles; ++it) {
    const int stage = it & 1;
    const int kv0 = it * KT;
    if (it + 1 < n_tiles) load_tile(kv0 + KT);

    if (it < w_tiles) {
      const T *kl = lds + stage * L::STAGE;
      const T *vl = kl + L::R_ELEMS;
      const T *ktl = kl + 2 * L::R_ELEMS;
      f32x16 s[2] = {f32x16{}, f32x16{}}, dp[2] = {f32x16{}, f32x16{}};
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int off = (t * 32 + c) * L::RSTR + ks * 16 + h * 8;
          s[t] = mfma32<T>(ld16(kl + off), qf[ks], s[t]);
          dp[t] = mfma32<T>(ld16(vl + off), gf[ks], dp[t]);
        }
      }
      const bool edge = (kv0 + KT > kv_end) || keymask ||
                        (p.causal && static_cast<int64_t>(kv0 + KT - 1) > qw + p.offset);
      unsigned long long kbits = ~0ull;
      if (edge && keymask) {
        const int key = kv0 + lane;
        kbits = __ballot(key < p.Sk && kmask[b * p.mask.s0 + static_cast<int64_t>(key) * p.mask.s3]);
      }
      const int64_t qpos = static_cast<int64_t>(qrow) + p.offset;
      unsigned pd[4][4];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
          float ds[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            bool ok = true;
            if (edge) {
              const int kk = t * 32 + crow(i + e, h);
              const int key = kv0 + kk;
              ok = key < kv_end && (!p.causal || qpos >= key) && ((kbits >> kk) & 1ull);
            }
            const float pv = ok ? fast_exp2(fmaf(s[t][i + e], sl, -lse2)) : 0.f;
            ds[e] = pv * (dp[t][i + e] - delta);
          }
          pd[t * 2 + (i >> 3)][(i & 7) >> 1] = pack2<T>(ds[0], ds[1]);
        }
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const u32x4 bd = {pd[ks][0], pd[ks][1], pd[ks][2], pd[ks][3]};
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
          const T *kr = ktl + (dt * 32 + c) * L::TSTR + ks * 16 + h * 4;
          const u32x2 lo = ld8(kr), hi = ld8(kr + 8);
          acc[dt] = mfma32<T>(u32x4{lo[0], lo[1], hi[0], hi[1]}, bd, acc[dt]);
        }
      }
    }

    if (it + 1 < n_tiles) store_tile(stage ^ 1);
    __syncthreads();
  }

  if (qrow >= p.Sq) return;
  T *dqp = mut<T>(a.dq) + b * a.dq.s0 + hq * a.dq.s1 + static_cast<int64_t>(qrow) * a.dq.s2;
  const float sc = a.scale;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = dt * 32 + g * 8 + h * 4;
      *reinterpret_cast<u32x2 *>(dqp + d) =
          u32x2{pack2<T>(acc[dt][g * 4] * sc, acc[dt][g * 4 + 1] * sc),
                pack2<T>(acc[dt][g * 4 + 2] * sc, acc[dt][g * 4 + 3] * sc)};
    }
  }
}

template <typename T, int D>
hipError_t launch(const BwdArgs &a, hipStream_t st) {
  const Problem &p = a.p;
  const int64_t rows = static_cast<int64_t>(p.B) * p.Hq * p.Sq;
  constexpr int RPB = NT / (D / 8);
  row_delta_kernel<T, D><<<dim3((rows + RPB - 1) / RPB), dim3(NT), 0, st>>>(a);

  static bool attr_set = false;  // raise the dynamic-LDS limit once per instantiation
  if (!attr_set) {
    hipFuncSetAttribute(reinterpret_cast<const void *>(&dkdv_kernel<T, D>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, KVLayout<T, D>::BYTES);
    hipFuncSetAttribute(reinterpret_cast<const void *>(&dq_kernel<T, D>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, QLayout<T, D>::BYTES);
    attr_set = true;
  }
  const int n_kb = (p.Sk + KB - 1) / KB;
  dkdv_kernel<T, D><<<dim3(n_kb * p.Hkv * p.B), dim3(NT), KVLayout<T, D>::BYTES, st>>>(a);
  const int n_qb = (p.Sq + QB - 1) / QB;
  dq_kernel<T, D><<<dim3(n_qb * p.Hq * p.B), dim3(NT), QLayout<T, D>::BYTES, st>>>(a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_mfma_backward(const Problem &p, int dtype, View q, View k, View v, View o,
                                View dout, const float *lse, View dq, View dk, View dv,
                                float *delta, hipStream_t st) {
  BwdArgs a{p, q, k, v, o, dout, dq, dk, dv, lse, delta,
            static_cast<float>(p.scale) * kLog2e, static_cast<float>(p.scale)};
  if (dtype == TSATTN_BF16) return p.Dqk == 128 ? launch<bf16, 128>(a, st) : launch<bf16, 64>(a, st);
  return p.Dqk == 128 ? launch<f16, 128>(a, st) : launch<f16, 64>(a, st);
}

}  // namespace tsattn
