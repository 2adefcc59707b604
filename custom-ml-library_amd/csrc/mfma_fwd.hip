// Flash-style attention forward for gfx950: MFMA 32x32x16 (f16/bf16 in,
// fp32 accumulate), online softmax in the exp2 domain, row LSE saved.
//
// Algorithm: the reference's streaming forward (src/tensorsmith/nn/
// attention.py:175-198) -- running max m, denominator l and accumulator per
// query row, rescaled by exp(m - m') per key tile; O = acc / l; LSE = m +
// log l; fully masked rows give O = 0, LSE = -inf.
//
// Work split: one workgroup = 4 wavefronts = 128 query rows of one (b, h);
// each wave owns 32 rows.  Key and value tiles of 64 rows are copied global
// -> LDS by direct buffer loads (no staging registers), double buffered, into
// swizzled row-major tiles.  The wave computes S^T = K Q^T so that each lane
// owns one query column: the softmax statistics and the rescale of the
// accumulator O^T = V^T P^T stay lane-local, and P^T leaves the accumulator
// registers as the next contraction's B operand without data movement.  The
// V^T operand is read from the row-major V tile with LDS transpose reads.
#include "mfma_common.h"

namespace tsattn {
namespace {

constexpr int BM = 128;  // query rows per workgroup
constexpr int BN = 64;   // keys per tile
constexpr int NT = 256;  // threads
constexpr int NW = NT / 64;

struct FwdArgs {
  Problem p;
  View q, k, v, o;
  float *lse;
  float sl;  // scale * log2(e)
  int n_qblocks;
  int total;
};

template <typename T>
__device__ __forceinline__ const T *head_ptr(View v, int b, int h) {
  return static_cast<const T *>(v.data) + b * v.s0 + h * v.s1;
}

template <typename T, int D>
__global__ __launch_bounds__(NT, 2) void fwd_kernel(FwdArgs a) {
  constexpr int TILE = BN * D;  // elements per K (or V) tile
  __shared__ __attribute__((aligned(1024))) T lds[2 * 2 * TILE];  // [stage][K | V]

  const Problem &p = a.p;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, c = lane & 31, h = lane >> 5;
  const int logical = xcd_remap(blockIdx.x, a.total);
  const int bh = logical / a.n_qblocks;
  const int qb = a.n_qblocks - 1 - (logical - bh * a.n_qblocks);  // long causal rows first
  const int b = bh / p.Hq, hq = bh - b * p.Hq, hk = hq / p.rep;
  const int q0 = qb * BM, qw = q0 + w * 32, qrow = qw + c;

  const int kv_end = kv_end_for(p, b);
  const bool keymask = p.mask.kind == TSATTN_MASK_BOOL && !(p.kv_prefix && p.kv_prefix[b]);

  // Key range of the workgroup (all its rows) and of this wave.
  int64_t lim = kv_end, wlim = kv_end;
  const int last_q = min(q0 + BM, p.Sq) - 1;
  const int last_qw = min(qw + 32, p.Sq) - 1;
  if (p.causal) {
    lim = min(lim, static_cast<int64_t>(last_q) + p.offset + 1);
    wlim = min(wlim, static_cast<int64_t>(last_qw) + p.offset + 1);
  }
  if (qw >= p.Sq) wlim = 0;
  const int n_tiles = lim > 0 ? static_cast<int>((lim + BN - 1) / BN) : 0;
  const int w_tiles = wlim > 0 ? static_cast<int>((wlim + BN - 1) / BN) : 0;

  const uint32_t qs_b = static_cast<uint32_t>(a.q.s2) * 2;
  const uint32_t ks_b = static_cast<uint32_t>(a.k.s2) * 2;
  const uint32_t vs_b = static_cast<uint32_t>(a.v.s2) * 2;
  const rsrc_t qrs = make_rsrc(head_ptr<T>(a.q, b, hq), static_cast<uint32_t>(p.Sq) * qs_b);
  const rsrc_t krs = make_rsrc(head_ptr<T>(a.k, b, hk), static_cast<uint32_t>(kv_end) * ks_b);
  const rsrc_t vrs = make_rsrc(head_ptr<T>(a.v, b, hk), static_cast<uint32_t>(kv_end) * vs_b);

  // Q fragments (B operand of S^T = K Q^T): lane holds Q[qrow][16ks + 8h .. +7].
  u32x4 qf[D / 16];
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks)
    qf[ks] = buf_load16(qrs, static_cast<uint32_t>(qrow) * qs_b + (ks * 16 + h * 8) * 2);

  auto issue = [&](int kv0, int stage) {
    T *kt = lds + stage * 2 * TILE;
    tile_to_lds<D, BN, NW>(krs, ks_b, kv0, kt, w, lane);
    tile_to_lds<D, BN, NW>(vrs, vs_b, kv0, kt + TILE, w, lane);
  };

  f32x16 oacc[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) oacc[dt] = f32x16{};
  float m = -INFINITY, l = 0.f;
  const float sl = a.sl;
  const uint8_t *kmask = static_cast<const uint8_t *>(p.mask.data);

  zero_lds<NT>(lds, sizeof(lds), tid);
  __syncthreads();
  if (n_tiles > 0) issue(0, 0);
  wait_vmem();
  __syncthreads();

  for (int it = 0; it < n_tiles; ++it) {
    const int stage = it & 1;
    const int kv0 = it * BN;
    if (it + 1 < n_tiles) issue(kv0 + BN, stage ^ 1);

    if (it < w_tiles) {
      const T *kt = lds + stage * 2 * TILE;
      const T *vt = kt + TILE;
      f32x16 s[2] = {f32x16{}, f32x16{}};
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
          s[t] = mfma32<T>(row_frag<T, D>(kt, t * 32, ks * 16, lane), qf[ks], s[t]);
      }

      const bool edge = (kv0 + BN > kv_end) || keymask ||
                        (p.causal && static_cast<int64_t>(kv0 + BN - 1) > qw + p.offset);
      if (edge) {
        unsigned long long kbits = ~0ull;
        if (keymask) {
          const int key = kv0 + lane;
          const bool ok = key < p.Sk && kmask[b * p.mask.s0 + static_cast<int64_t>(key) * p.mask.s3];
          kbits = __ballot(ok);
        }
        const int64_t qpos = static_cast<int64_t>(qrow) + p.offset;
        const bool causal = p.causal != 0;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int kk = t * 32 + crow(i, h);
            const int key = kv0 + kk;
            const bool ok = (key < kv_end) & (!causal | (qpos >= key)) & (((kbits >> kk) & 1ull) != 0);
            s[t][i] = ok ? s[t][i] : -INFINITY;
          }
        }
      }

      float mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[t][i]);
      mx = xor32_max(mx);
      const float m_new = fmaxf(m, mx * sl);
      const float base = m_new == -INFINITY ? 0.f : m_new;
      const float corr = fast_exp2(m - base);
      m = m_new;
      l *= corr;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) oacc[dt] *= corr;

      unsigned pb[4][4];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
          const float p0 = fast_exp2(fmaf(s[t][i], sl, -base));
          const float p1 = fast_exp2(fmaf(s[t][i + 1], sl, -base));
          l += p0 + p1;
          pb[t * 2 + (i >> 3)][(i & 7) >> 1] = pack2<T>(p0, p1);
        }
      }

#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const u32x4 bf = {pb[ks][0], pb[ks][1], pb[ks][2], pb[ks][3]};
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
          oacc[dt] = mfma32<T>(tr_frag<T, D>(vt, ks * 16, dt * 32, lane), bf, oacc[dt]);
      }
    }

    wait_vmem();
    __syncthreads();
  }

  const float lt = xor32_sum(l);  // lanes c and c+32 share a query row
  if (qrow >= p.Sq) return;
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  T *op = static_cast<T *>(const_cast<void *>(a.o.data)) + b * a.o.s0 + hq * a.o.s1 +
          static_cast<int64_t>(qrow) * a.o.s2;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = dt * 32 + g * 8 + h * 4;
      u32x2 pk = {pack2<T>(oacc[dt][g * 4 + 0] * inv, oacc[dt][g * 4 + 1] * inv),
                  pack2<T>(oacc[dt][g * 4 + 2] * inv, oacc[dt][g * 4 + 3] * inv)};
      *reinterpret_cast<u32x2 *>(op + d) = pk;
    }
  }
  if (a.lse && h == 0)
    a.lse[(static_cast<int64_t>(b) * p.Hq + hq) * p.Sq + qrow] =
        lt > 0.f ? (m + log2f(lt)) * kLn2 : -INFINITY;
}

template <typename T, int D>
hipError_t launch(const FwdArgs &a, hipStream_t st) {
  { Probe pr_("fwd_mfma", st); fwd_kernel<T, D><<<dim3(a.total), dim3(NT), 0, st>>>(a); }
  return hipGetLastError();
}

}  // namespace

bool mfma_supported(const Problem &p, int dtype) {
  if (dtype != TSATTN_F16 && dtype != TSATTN_BF16) return false;
  if (p.Dqk != p.Dv || (p.Dqk != 64 && p.Dqk != 128)) return false;
  if (!(p.scale > 0.0)) return false;
  if (p.mask.kind == TSATTN_MASK_NONE) return true;
  // key masks [B,1,1,K] with their derived lengths
  return p.mask.kind == TSATTN_MASK_BOOL && p.mask.s1 == 0 && p.mask.s2 == 0 && p.kv_len != nullptr;
}

hipError_t launch_mfma_forward(const Problem &p, int dtype, View q, View k, View v, View o,
                               float *lse, hipStream_t st) {
  FwdArgs a{p, q, k, v, o, lse, static_cast<float>(p.scale) * kLog2e, (p.Sq + BM - 1) / BM, 0};
  a.total = a.n_qblocks * p.Hq * p.B;
  if (dtype == TSATTN_BF16) return p.Dqk == 128 ? launch<bf16, 128>(a, st) : launch<bf16, 64>(a, st);
  return p.Dqk == 128 ? launch<f16, 128>(a, st) : launch<f16, 64>(a, st);
}

}  // namespace tsattn
