// KV-cache decode attention for gfx950: a few query rows per KV head against
// a long cached prefix; bound by HBM bandwidth, not by math.  RoPE can be
// folded into the query load (Problem::rope; the cache holds rotated keys).
//
// Math: the reference's online softmax (src/tensorsmith/nn/attention.py:
// 185-193) applied twice.  Each workgroup reduces one split of the cache to a
// partial state (running max m, denominator l, accumulator acc) -- inside it
// every lane keeps its own state over the keys it streams, so no cross-lane
// traffic happens per key -- and decode_merge_kernel combines the splits with
// the same rescale-by-exp(m - M) rule.  Fully masked rows give 0.
//
// Memory layout: each key row is read by D/8 neighbouring lanes, 8 elements
// each -- 16-byte loads for 16-bit caches (one wave instruction covers 64*16 B
// of consecutive keys), two for fp32 caches -- and kU such row pieces for K
// and kU for V are issued before any is consumed, so every wave keeps 2*kU
// KiB (fp32: 4*kU KiB) in flight.
//
// int8 caches (the reference's quantised KVCache, src/tensorsmith/nn/
// cache.py:73-77 and :91-98): K and V rows are int8 with one fp32 scale per
// (b, h, key).  The same lanes read 8-byte int8 chunks and the row scales;
// the scale of K is applied to the lane group's dot product and the scale of
// V is folded into the probability, so dequantisation costs one multiply per
// key instead of a pass over the cache.  The dequantised values enter the
// math in fp32 (the reference rounds them to the cache dtype first: at most
// half an ulp of that dtype per element).
#include <mutex>
#include <type_traits>

#include "mfma_common.h"
#include "rope_math.h"

namespace tsattn {
namespace {

constexpr int NT = 256;
constexpr int kU = 4;  // key instructions in flight per batch (per operand, 16-byte loads)
constexpr int kMaxRows = 8;

struct DecArgs {
  Problem p;
  View q, k, v, o;
  View ks, vs;  // int8 caches: fp32 row scales [B, Hkv, capacity, 1]
  float *ws;
  int split_len, max_splits, rows;  // rows = rep * Sq query rows per KV head
  float sl;                         // scale * log2(e)
};

// Keys any row may attend to: [0, eff_end).
__device__ __forceinline__ int eff_end(const Problem &p, int b) {
  int e = kv_end_for(p, b);
  if (p.causal) {
    const int64_t lim = static_cast<int64_t>(p.Sq) - 1 + p.offset + 1;
    if (lim < e) e = static_cast<int>(lim < 0 ? 0 : lim);
  }
  return e;
}

__device__ __forceinline__ void merge_state(float &m, float &l, float *acc, float m2, float l2,
                                            const float *acc2) {
  const float mx = fmaxf(m, m2);
  const float base = mx == -INFINITY ? 0.f : mx;
  const float c1 = fast_exp2(m - base), c2 = fast_exp2(m2 - base);
  l = l * c1 + l2 * c2;
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = acc[e] * c1 + acc2[e] * c2;
  m = mx;
}

template <typename T>
__device__ __forceinline__ void unpack8(u32x4 x, float *out) {
  const T *e = reinterpret_cast<const T *>(&x);
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = static_cast<float>(e[i]);
}

__device__ __forceinline__ void unpack8_i8(u32x2 x, float *out) {
  const int8_t *e = reinterpret_cast<const int8_t *>(&x);
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = static_cast<float>(e[i]);
}


// Cache rows as loaded: 8 values of the cache type -- int8 (8 B), 16-bit
// (16 B) or fp32 (32 B, two 16-byte loads).
struct F32x8 {
  u32x4 lo, hi;
};
template <typename KT>
using KvChunk = std::conditional_t<std::is_same_v<KT, int8_t>, u32x2,
                                   std::conditional_t<std::is_same_v<KT, float>, F32x8, u32x4>>;

template <typename KT>
__device__ __forceinline__ KvChunk<KT> load_chunk(const KT *p) {
  if constexpr (std::is_same_v<KT, float>) {
    const u32x4 *q = reinterpret_cast<const u32x4 *>(p);
    return F32x8{__builtin_nontemporal_load(q), __builtin_nontemporal_load(q + 1)};
  } else {
    return __builtin_nontemporal_load(reinterpret_cast<const KvChunk<KT> *>(p));
  }
}

// 8 query (T) values of a row: 16 bytes, or 32 for fp32.
template <typename T>
__device__ __forceinline__ void load_q8(const T *p, float *out) {
  if constexpr (std::is_same_v<T, float>) {
    const float4 a = *reinterpret_cast<const float4 *>(p), b = *reinterpret_cast<const float4 *>(p + 4);
    out[0] = a.x, out[1] = a.y, out[2] = a.z, out[3] = a.w;
    out[4] = b.x, out[5] = b.y, out[6] = b.z, out[7] = b.w;
  } else {
    const u32x4 raw = ld16(p);
    const T *e = reinterpret_cast<const T *>(&raw);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = static_cast<float>(e[i]);
  }
}

// A loaded row piece as 8 floats.
template <typename KT>
__device__ __forceinline__ void unpack_kv(const KvChunk<KT> &x, float *out) {
  if constexpr (std::is_same_v<KT, int8_t>) {
    unpack8_i8(x, out);
  } else if constexpr (std::is_same_v<KT, float>) {
    const float4 a = __builtin_bit_cast(float4, x.lo), b = __builtin_bit_cast(float4, x.hi);
    out[0] = a.x, out[1] = a.y, out[2] = a.z, out[3] = a.w;
    out[4] = b.x, out[5] = b.y, out[6] = b.z, out[7] = b.w;
  } else {
    unpack8<KT>(x, out);
  }
}

// Sum over each aligned group of LPK lanes (the lanes holding one key row).
// For LPK = 16 (D = 128) a DPP butterfly inside each 16-lane row: quad_perm
// swaps within quads, then rotations by 4 and 8 lanes; no LDS traffic.
template <int LPK>
__device__ __forceinline__ float group_sum(float d) {
  if constexpr (LPK == 16) {
    auto dpp = [](float x, int ctrl_sel) {
      const int v = __builtin_bit_cast(int, x);
      int r;
      switch (ctrl_sel) {
        case 0: r = __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false); break;   // quad_perm [1,0,3,2]
        case 1: r = __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false); break;   // quad_perm [2,3,0,1]
        case 2: r = __builtin_amdgcn_update_dpp(0, v, 0x124, 0xF, 0xF, false); break;  // row_ror:4
        default: r = __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false); break; // row_ror:8
      }
      return __builtin_bit_cast(float, r);
    };
    d += dpp(d, 0);
    d += dpp(d, 1);
    d += dpp(d, 2);
    d += dpp(d, 3);
    return d;
  } else {
#pragma unroll
    for (int x = LPK / 2; x >= 1; x >>= 1) d += __shfl_xor(d, x, 64);
    return d;
  }
}

template <typename T, int D, int R, bool Q8>
__global__ __launch_bounds__(NT) void decode_split_kernel(DecArgs a) {
  using KT = std::conditional_t<Q8, int8_t, T>;  // cache element type
  constexpr int U = kU;
  constexpr int LPK = D / 8;      // lanes per key row
  constexpr int KPI = 64 / LPK;   // keys per wave instruction
  constexpr int BATCH = KPI * U;  // keys per wave per batch
  __shared__ float red[4][R][10 * LPK];

  const Problem &p = a.p;
  const int split = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int dc = lane % LPK, kg = lane / LPK;
  const int end = eff_end(p, b);
  const int k_begin = split * a.split_len;
  if (k_begin >= end) return;  // this split holds no keys for row b
  const int k_stop = min(k_begin + a.split_len, end);
  // A key mask that is exactly the prefix [0, kv_len[b]) is already applied by k_stop.
  const bool masked = p.mask.kind != TSATTN_MASK_NONE &&
                      !(p.kv_prefix && p.kv_prefix[b] && p.mask.s1 == 0 && p.mask.s2 == 0);

  // Query rows r = rr * Sq + i (query head hk*rep + rr, position i), pre-scaled
  // so that s = q.k is already in log2 units.  With RoPE folded in (the keys
  // in the cache are stored rotated), row i is rotated to position q_pos0 + i
  // here, rounded to T as the RoPE kernel rounds it.
  float qv[R][8];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r < a.rows) {
      const int hq = hk * p.rep + r / p.Sq, i = r % p.Sq;
      const T *qp = static_cast<const T *>(a.q.data) + b * a.q.s0 + hq * a.q.s1 +
                    static_cast<int64_t>(i) * a.q.s2 + dc * 8;
      if constexpr (std::is_same_v<T, float>) {
        load_q8<T>(qp, qv[r]);  // (fp32: no folded rotation; the host refuses it)
      } else {
        u32x4 raw = ld16(qp);
        if (p.rope.R > 0) rotate_chunk<T>(raw, p.rope, p.rope.qpos0 + i, 4 * dc, false);
        unpack8<T>(raw, qv[r]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) qv[r][e] *= a.sl;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qv[r][e] = 0.f;
    }
  }
  float m[R], l[R], acc[R][8];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[r][e] = 0.f;
  }

  const KT *kbase = static_cast<const KT *>(a.k.data) + b * a.k.s0 + hk * a.k.s1 + dc * 8;
  const KT *vbase = static_cast<const KT *>(a.v.data) + b * a.v.s0 + hk * a.v.s1 + dc * 8;
  const float *ksb = Q8 ? static_cast<const float *>(a.ks.data) + b * a.ks.s0 + hk * a.ks.s1 : nullptr;
  const float *vsb = Q8 ? static_cast<const float *>(a.vs.data) + b * a.vs.s0 + hk * a.vs.s1 : nullptr;
  const float log2e = kLog2e;
  // Keys past k_stop are read from row k_stop - 1 (in bounds, finite) and
  // masked, so every load is unconditional.  K/V are streamed once: loads
  // are non-temporal.
  auto body = [&](auto masked_tag) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    for (int kb = k_begin + w * BATCH; kb < k_stop; kb += 4 * BATCH) {
      KvChunk<KT> kr[U], vr[U];
      float ksc[U], vsc[U];
      float kslot = 0.f, vslot = 0.f;
      if constexpr (Q8) {
        // one scale load per operand for the batch's BATCH keys: lane l takes
        // key kb + l % BATCH; each lane then shuffles in its own keys' scales
        const int key = min(kb + (lane % BATCH), k_stop - 1);
        kslot = ksb[static_cast<int64_t>(key) * a.ks.s2];
        vslot = vsb[static_cast<int64_t>(key) * a.vs.s2];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int key = min(kb + u * KPI + kg, k_stop - 1);
        kr[u] = load_chunk<KT>(kbase + static_cast<int64_t>(key) * a.k.s2);
        vr[u] = load_chunk<KT>(vbase + static_cast<int64_t>(key) * a.v.s2);
      }
      if constexpr (Q8) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          ksc[u] = __shfl(kslot, u * KPI + kg, 64);
          vsc[u] = __shfl(vslot, u * KPI + kg, 64);
        }
      }
      float s[U][R];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float kf[8];
        unpack_kv<KT>(kr[u], kf);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float d = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) d = fmaf(qv[r][e], kf[e], d);
          s[u][r] = group_sum<LPK>(d);
          if constexpr (Q8) s[u][r] *= ksc[u];
        }
      }
      // masks: keys past the split, causal, user mask (bool or additive, any broadcast)
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int key = kb + u * KPI + kg;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int i = r % p.Sq;
          bool ok = key < k_stop && r < a.rows &&
                    (!p.causal || static_cast<int64_t>(i) + p.offset >= key);
          if constexpr (MASKED) {
            if (ok) {
              const int hq = hk * p.rep + r / p.Sq;
              const int64_t mi = b * p.mask.s0 + hq * p.mask.s1 + static_cast<int64_t>(i) * p.mask.s2 +
                                 static_cast<int64_t>(key) * p.mask.s3;
              if (p.mask.kind == TSATTN_MASK_BOOL)
                ok = static_cast<const uint8_t *>(p.mask.data)[mi] != 0;
              else
                s[u][r] += load_additive<float>(p.mask.data, mi, p.mask.dtype) * log2e;
            }
          }
          if (!ok) s[u][r] = -INFINITY;
        }
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float mb = m[r];
#pragma unroll
        for (int u = 0; u < U; ++u) mb = fmaxf(mb, s[u][r]);
        const float base = mb == -INFINITY ? 0.f : mb;
        const float corr = fast_exp2(m[r] - base);
        l[r] *= corr;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r][e] *= corr;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float pv = fast_exp2(s[u][r] - base);
          l[r] += pv;
          float vf[8];
          unpack_kv<KT>(vr[u], vf);
          const float pw = Q8 ? pv * vsc[u] : pv;  // int8: V's row scale folded into P
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[r][e] = fmaf(pw, vf[e], acc[r][e]);
        }
        m[r] = mb;
      }
    }
  };
  if (masked) body(std::true_type{});
  else body(std::false_type{});

  // Merge the key groups of the wave (lanes dc, dc+LPK, ...), then the waves.
#pragma unroll
  for (int x = LPK; x < 64; x <<= 1) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float a2[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) a2[e] = __shfl_xor(acc[r][e], x, 64);
      const float m2 = __shfl_xor(m[r], x, 64), l2 = __shfl_xor(l[r], x, 64);
      merge_state(m[r], l[r], acc[r], m2, l2, a2);
    }
  }
  if (kg == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float *slot = &red[w][r][dc * 10];
#pragma unroll
      for (int e = 0; e < 8; ++e) slot[e] = acc[r][e];
      slot[8] = m[r];
      slot[9] = l[r];
    }
  }
  __syncthreads();
  if (w != 0 || kg != 0) return;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r >= a.rows) break;
#pragma unroll
    for (int ww = 1; ww < 4; ++ww) {
      const float *slot = &red[ww][r][dc * 10];
      merge_state(m[r], l[r], acc[r], slot[8], slot[9], slot);
    }
    float *out = a.ws + ((static_cast<int64_t>(b * p.Hkv + hk) * a.max_splits + split) * a.rows + r) *
                            static_cast<int64_t>(D + 2);
#pragma unroll
    for (int e = 0; e < 8; ++e) out[dc * 8 + e] = acc[r][e];
    if (dc == 0) {
      out[D] = m[r];
      out[D + 1] = l[r];
    }
  }
}

// One wave per output row (b, hq, i): combine the splits' partial states.
// Lane s reads split s's (m, l) so the maxima and the weights exp2(m_s - M)
// come from one round of loads; the accumulators are then summed over the
// splits with lane d owning value columns d, d + 64, ...
template <typename T, int D>
__global__ __launch_bounds__(64) void decode_merge_kernel(DecArgs a) {
  const Problem &p = a.p;
  const int b = blockIdx.y, row = blockIdx.x;  // row = hq * Sq + i
  const int hq = row / p.Sq, i = row - hq * p.Sq;
  const int hk = hq / p.rep, r = (hq - hk * p.rep) * p.Sq + i;
  const int lane = threadIdx.x;
  const int end = eff_end(p, b);
  const int n = end > 0 ? (end + a.split_len - 1) / a.split_len : 0;
  const float *base = a.ws + (static_cast<int64_t>(b * p.Hkv + hk) * a.max_splits * a.rows + r) *
                                 static_cast<int64_t>(D + 2);
  const int64_t stride = static_cast<int64_t>(a.rows) * (D + 2);
  constexpr int PER = (D + 63) / 64;
  float acc[PER] = {};
  float M = -INFINITY, L = 0.f;
  // passes of up to SB splits; each issues every load of its splits (the
  // partial rows and their (m, l), indices clamped to the last split, which
  // then weighs 0) before any use, so a pass costs one memory latency
  constexpr int SB = 16;
  for (int s0 = 0; s0 < n; s0 += SB) {
    float pv[SB][PER];
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const float *part = base + min(s0 + u, n - 1) * stride;
#pragma unroll
      for (int t = 0; t < PER; ++t) {
        const int d = lane + 64 * t;
        pv[u][t] = part[d < D ? d : D - 1];
      }
    }
    const int s = s0 + lane;
    const bool live = lane < SB && s < n;
    const float ms = live ? base[s * stride + D] : -INFINITY;
    const float ls = live ? base[s * stride + D + 1] : 0.f;
    float mx = ms;
#pragma unroll
    for (int x = 32; x >= 1; x >>= 1) mx = fmaxf(mx, __shfl_xor(mx, x, 64));
    const float M2 = fmaxf(M, mx);
    const float mb = M2 == -INFINITY ? 0.f : M2;
    const float cold = fast_exp2(M - mb);  // rescale what earlier passes summed
    const float cs = live ? fast_exp2(ms - mb) : 0.f;
    float lsum = ls * cs;
#pragma unroll
    for (int x = 32; x >= 1; x >>= 1) lsum += __shfl_xor(lsum, x, 64);
    L = L * cold + lsum;
#pragma unroll
    for (int t = 0; t < PER; ++t) acc[t] *= cold;
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const float c = __shfl(cs, u, 64);  // 0 past the last split
#pragma unroll
      for (int t = 0; t < PER; ++t) acc[t] = fmaf(pv[u][t], c, acc[t]);
    }
    M = M2;
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  T *op = static_cast<T *>(const_cast<void *>(a.o.data)) + b * a.o.s0 + hq * a.o.s1 +
          static_cast<int64_t>(i) * a.o.s2;
#pragma unroll
  for (int t = 0; t < PER; ++t) {
    const int d = lane + 64 * t;
    if (d < D) op[d] = static_cast<T>(acc[t] * inv);
  }
}

template <typename T, int D, int R, bool Q8>
hipError_t launch_rows(const DecArgs &a, hipStream_t st) {
  const Problem &p = a.p;
  {
    Probe pr_(Q8 ? "decode_split_int8" : "decode_split", st);
    decode_split_kernel<T, D, R, Q8><<<dim3(a.max_splits, p.Hkv, p.B), dim3(NT), 0, st>>>(a);
  }
  { Probe pr_("decode_merge", st); decode_merge_kernel<T, D><<<dim3(p.Hq * p.Sq, p.B), dim3(64), 0, st>>>(a); }
  return hipGetLastError();
}

template <typename T, int D, bool Q8>
hipError_t launch_dim(const DecArgs &a, hipStream_t st) {
  if (a.rows <= 1) return launch_rows<T, D, 1, Q8>(a, st);
  if (a.rows <= 2) return launch_rows<T, D, 2, Q8>(a, st);
  if (a.rows <= 4) return launch_rows<T, D, 4, Q8>(a, st);
  return launch_rows<T, D, 8, Q8>(a, st);
}

template <bool Q8>
hipError_t launch_any(const DecArgs &a, int dtype, hipStream_t st) {
  const int d = a.p.Dqk;
  if constexpr (!Q8) {
    if (dtype == TSATTN_F32) {
      if (d == 64) return launch_dim<float, 64, false>(a, st);
      if (d == 128) return launch_dim<float, 128, false>(a, st);
      return launch_dim<float, 256, false>(a, st);
    }
  }
  if (dtype == TSATTN_BF16) {
    if (d == 64) return launch_dim<bf16, 64, Q8>(a, st);
    if (d == 128) return launch_dim<bf16, 128, Q8>(a, st);
    return launch_dim<bf16, 256, Q8>(a, st);
  }
  if (d == 64) return launch_dim<f16, 64, Q8>(a, st);
  if (d == 128) return launch_dim<f16, 128, Q8>(a, st);
  return launch_dim<f16, 256, Q8>(a, st);
}

// Keys per split.  Never a power of two: with 2^k keys every split of every
// cache row starts at the same offset modulo a large power of two (rows are
// themselves power-of-two sized), so the workgroups running together hit the
// same HBM channels -- 512-key splits measured 64% of peak bandwidth at
// B64 H32 D128, 640-key splits 82%.  Halved (640, 320, 160, 80) until the
// grid has 4096 workgroups.
int choose_split(const Problem &p, int split_len) {
  if (split_len > 0) return split_len;
  int s = 640;
  while (s > 80 && static_cast<int64_t>(p.B) * p.Hkv * ((p.Sk + s - 1) / s) < 4096) s >>= 1;
  return s;
}

}  // namespace

bool decode_supported(const Problem &p, int dtype) {
  if (dtype != TSATTN_F16 && dtype != TSATTN_BF16 && dtype != TSATTN_F32) return false;
  if (dtype == TSATTN_F32 && p.rope.R > 0) return false;  // (the folded rotation is 16-bit)
  if (p.Dqk != p.Dv || (p.Dqk != 64 && p.Dqk != 128 && p.Dqk != 256)) return false;
  return p.rep * p.Sq <= kMaxRows;
}

size_t decode_workspace_bytes(const Problem &p, int split_len) {
  const int s = choose_split(p, split_len);
  const int64_t splits = (p.Sk + s - 1) / s;
  return static_cast<size_t>(p.B) * p.Hkv * splits * p.rep * p.Sq * (p.Dv + 2) * sizeof(float);
}

// ---------------------------------------------------------------------------
// Library-owned scratch for tsattn_decode_forward_noalloc: the split kernel's
// partial (acc, m, l) states live in this array instead of a caller
// workspace.  Each GPU the library runs on holds its own copy (zero-filled
// .bss of the code object, kept until the process ends).  In host code
// `scratch` names a host-side stand-in, never the device array: kernels get
// the address hipGetSymbolAddress reports for the current device.  Every
// call on one GPU shares that GPU's copy; the split kernel writes every slot
// the merge reads before the merge runs, so nothing needs clearing, but
// calls that overlap on one GPU (different streams) race.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[TSATTN_DECODE_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};
}  // namespace

hipError_t decode_scratch(void **ptr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *addr = nullptr;
    e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!addr) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = addr;
  }
  *ptr = g_scratch_ptr[dev];
  return hipSuccess;
}

hipError_t launch_decode(const Problem &p, int dtype, View q, View k, View v, View o,
                         int split_len, void *workspace, hipStream_t st) {
  DecArgs a{p, q, k, v, o, View{}, View{}, static_cast<float *>(workspace), 0, 0, p.rep * p.Sq,
            static_cast<float>(p.scale) * kLog2e};
  a.split_len = choose_split(p, split_len);
  a.max_splits = (p.Sk + a.split_len - 1) / a.split_len;
  return launch_any<false>(a, dtype, st);
}

hipError_t launch_decode_int8(const Problem &p, int dtype, View q, View k, View v, View ks,
                              View vs, View o, int split_len, void *workspace, hipStream_t st) {
  DecArgs a{p, q, k, v, o, ks, vs, static_cast<float *>(workspace), 0, 0, p.rep * p.Sq,
            static_cast<float>(p.scale) * kLog2e};
  a.split_len = choose_split(p, split_len);
  a.max_splits = (p.Sk + a.split_len - 1) / a.split_len;
  return launch_any<true>(a, dtype, st);
}

}  // namespace tsattn
