// Generic attention kernels: one wavefront per query (or key) row, VALU math
// in the accumulator type (float for f32/f16/bf16, double for f64).
//
// The dK/dV kernel's four waves (four keys) share each 64-row chunk of Q and
// dO, which every lane walks along its own row: with ST the chunk is staged
// through LDS once per workgroup by whole-row loads and each lane reads its
// row there (rows padded by one element, so the 64 lanes' walks hit 64
// banks), instead of 64 rows per load instruction from memory.  Same
// arithmetic in the same order either way; problems whose chunk does not fit
// in LDS run without it.  (The same staging of K / V in the forward and dQ
// kernels measured slower: four rows per workgroup do not repay it at the
// lower occupancy the staged chunk leaves.)
//
// These carry every case the reference allows that the MFMA kernels do not
// specialise: fp32 / fp64 inputs, any head dims (Dv != Dqk included,
// reference tests/test_transformer.py:44-46), boolean or additive masks of any
// broadcast shape, any scale sign.  Same recurrence as the reference's
// streaming backend (src/tensorsmith/nn/attention.py:175-198) and its VJP
// (:220-244): running max / sum / accumulator per row over 64-key chunks, and
// P recomputed from the saved LSE in the backward.  Dropout as the dense
// backend (:140-144, :210-217): P V takes P * mask, dS = P (dP * mask -
// delta), the mask regenerated per element from the problem's Philox stream.
#include "philox.h"

namespace tsattn {
namespace {

constexpr int kWaves = 4;        // rows per workgroup
constexpr int kChunk = 64;       // keys (or queries) per chunk = one lane each
constexpr int kMaxDimSlots = 8;  // head dims up to 8 * 64 = 512

template <typename A>
__device__ __forceinline__ A neg_inf() {
  return -static_cast<A>(INFINITY);
}

__device__ __forceinline__ float exp_acc(float x) { return expf(x); }
__device__ __forceinline__ double exp_acc(double x) { return exp(x); }
__device__ __forceinline__ float log_acc(float x) { return logf(x); }
__device__ __forceinline__ double log_acc(double x) { return log(x); }

template <typename A>
__device__ __forceinline__ A wave_max(A x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    A y = __shfl_xor(x, m, 64);
    x = x > y ? x : y;
  }
  return x;
}

template <typename A>
__device__ __forceinline__ A wave_sum(A x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
  return x;
}

// Dropout mask value of element (row, j): 0, or the keep scale in the
// compute type (the reference's keep.astype(compute dtype) / (1 - p)).
template <typename A>
__device__ __forceinline__ A drop_factor(const Problem &p, int64_t row, int j) {
  if (!p.drop.on) return A(1);
  const A scale = sizeof(A) == 8 ? static_cast<A>(p.drop.scale64) : static_cast<A>(p.drop.scale);
  return dropout_keeps_one(p, row, j) ? scale : A(0);
}

template <typename T>
__device__ __forceinline__ const T *row_ptr(View v, int b, int h, int s) {
  return static_cast<const T *>(v.data) + b * v.s0 + h * v.s1 + static_cast<int64_t>(s) * v.s2;
}
template <typename T>
__device__ __forceinline__ T *row_ptr_mut(View v, int b, int h, int s) {
  return const_cast<T *>(row_ptr<T>(v, b, h, s));
}

// Row stride, in elements of `esz` bytes, of a staged chunk of D-element rows:
// a whole number of 16-byte units, and an odd one, so the 16-byte reads of
// the 16 lanes an LDS pass serves fall in 16 different bank groups.
__host__ __device__ inline int staged_ld(int D, int esz) {
  const int vw = 16 / esz;
  return (((D + vw - 1) / vw) | 1) * vw;
}

// Elements D rounded up to whole 16-byte units (keeps the next region aligned).
__host__ __device__ inline int round16(int D, int esz) {
  const int vw = 16 / esz;
  return (D + vw - 1) / vw * vw;
}

// sum_d x[d] y[d] in order d = 0, 1, ... over 16-byte aligned LDS rows, read
// 16 bytes at a time.
template <typename A>
__device__ __forceinline__ A dot_lds(const A *x, const A *y, int D) {
  constexpr int VW = 16 / sizeof(A);
  typedef A V __attribute__((ext_vector_type(VW)));
  A acc = 0;
  int d = 0;
  for (; d + VW <= D; d += VW) {
    const V a = *reinterpret_cast<const V *>(x + d), c = *reinterpret_cast<const V *>(y + d);
#pragma unroll
    for (int e = 0; e < VW; ++e) acc += a[e] * c[e];
  }
  for (; d < D; ++d) acc += x[d] * y[d];
  return acc;
}

// Rows r0 .. r0 + 63 of operand x (batch b, head h), D elements each, into dst
// as A with row stride ld; rows from n_rows on are zero.  Wave w of the NW
// loads rows w, w + NW, ..., one coalesced row per step.  Every thread of the
// workgroup calls it; the caller synchronises.
template <typename T, typename A, int NW>
__device__ __forceinline__ void stage_chunk(A *dst, View x, int b, int h, int64_t r0, int n_rows,
                                            int D, int ld) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int r = w; r < kChunk; r += NW) {
    const int64_t row = r0 + r;
    A *out = dst + r * ld;
    if (row < n_rows) {
      const T *src = row_ptr<T>(x, b, h, static_cast<int>(row));
      for (int d = lane; d < D; d += 64) out[d] = to_acc<A>(src[d]);
    } else {
      for (int d = lane; d < D; d += 64) out[d] = A(0);
    }
  }
}

// Scores of query rows i0 .. i0 + R - 1 (held in qrows, row stride Dqk)
// against key j, each with the reference's order: scale, then mask (bool ->
// -inf, additive -> +), then causal (:102-113); rows from Sq on get -inf.
// Each element of the key row is loaded once for the R rows; with VK (rows
// 16-byte aligned) 16 bytes at a time, the sums in the same order.
template <typename T, typename A, int R, bool VK>
__device__ __forceinline__ void score_rows(const Problem &p, const A *qrows, const T *krow, int b,
                                           int hq, int i0, int j, int kv_end, A (&s)[R]) {
  if (j >= kv_end) {
#pragma unroll
    for (int r = 0; r < R; ++r) s[r] = neg_inf<A>();
    return;
  }
  A acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0;
  int d = 0;
  if constexpr (VK) {
    constexpr int VW = 16 / sizeof(T);
    typedef T V __attribute__((ext_vector_type(VW)));
    for (; d + VW <= p.Dqk; d += VW) {
      const V kk = *reinterpret_cast<const V *>(krow + d);
#pragma unroll
      for (int e = 0; e < VW; ++e) {
        const A kd = to_acc<A>(static_cast<T>(kk[e]));
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] += qrows[r * p.Dqk + d + e] * kd;
      }
    }
  }
  for (; d < p.Dqk; ++d) {
    const A kd = to_acc<A>(krow[d]);
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] += qrows[r * p.Dqk + d] * kd;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = i0 + r;
    if (i >= p.Sq || (p.causal && static_cast<int64_t>(i) + p.offset < static_cast<int64_t>(j))) {
      s[r] = neg_inf<A>();
      continue;
    }
    A x = acc[r] * static_cast<A>(p.scale);
    if (p.mask.kind != TSATTN_MASK_NONE) {
      const int64_t mi = b * p.mask.s0 + hq * p.mask.s1 + static_cast<int64_t>(i) * p.mask.s2 +
                         static_cast<int64_t>(j) * p.mask.s3;
      if (p.mask.kind == TSATTN_MASK_BOOL) {
        if (!static_cast<const uint8_t *>(p.mask.data)[mi]) x = neg_inf<A>();
      } else {
        x += load_additive<A>(p.mask.data, mi, p.mask.dtype);
      }
    }
    s[r] = x;
  }
}

// ---------------------------------------------------------------------------
// Forward: grid (ceil(Sq / (4 R)), Hq, B); wave w owns the R query rows from
// (blockIdx.x * 4 + w) R, lane l the key j0 + l of each 64-key chunk, so each
// K and V element a lane loads serves R rows.
// ---------------------------------------------------------------------------
template <typename T, typename A, int R, bool VK>
__global__ __launch_bounds__(256) void generic_forward_kernel(Problem p, View q, View k, View v,
                                                              View o, A *lse) {
  extern __shared__ unsigned char smem_raw[];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int b = blockIdx.z, hq = blockIdx.y, hk = hq / p.rep;
  const int i0 = (blockIdx.x * kWaves + w) * R;
  A *qrows = reinterpret_cast<A *>(smem_raw) + w * R * (p.Dqk + kChunk);
  A *pbuf = qrows + R * p.Dqk;  // [R][kChunk]
  const int kv_end = kv_end_for(p, b);

#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = i0 + r;
    if (i < p.Sq) {
      const T *qp = row_ptr<T>(q, b, hq, i);
      for (int d = lane; d < p.Dqk; d += 64) qrows[r * p.Dqk + d] = to_acc<A>(qp[d]);
    } else {
      for (int d = lane; d < p.Dqk; d += 64) qrows[r * p.Dqk + d] = A(0);
    }
  }
  // Uniform chunk count for the workgroup: the furthest key any of its rows sees.
  int64_t last_row = (static_cast<int64_t>(blockIdx.x) * kWaves + kWaves) * R - 1;
  if (last_row > p.Sq - 1) last_row = p.Sq - 1;
  int64_t stop = kv_end;
  if (p.causal && last_row + p.offset + 1 < stop) stop = last_row + p.offset + 1;
  if (stop < 0) stop = 0;
  __syncthreads();

  A m[R], l[R], acc[R][kMaxDimSlots];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    m[r] = neg_inf<A>();
    l[r] = 0;
#pragma unroll
    for (int t = 0; t < kMaxDimSlots; ++t) acc[r][t] = 0;
  }

  for (int j0 = 0; j0 < stop; j0 += kChunk) {
    const int j = j0 + lane;
    A s[R];
    score_rows<T, A, R, VK>(p, qrows, row_ptr<T>(k, b, hk, j < p.Sk ? j : 0), b, hq, i0, j, kv_end, s);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const A cmax = wave_max(s[r]);
      const A m_new = m[r] > cmax ? m[r] : cmax;
      const A base = isfinite(m_new) ? m_new : A(0);
      const A corr = exp_acc(m[r] - base);
      const A pj = exp_acc(s[r] - base);
      l[r] = l[r] * corr + wave_sum(pj);  // the denominator sums the undropped P
      m[r] = m_new;
#pragma unroll
      for (int t = 0; t < kMaxDimSlots; ++t) acc[r][t] *= corr;
      // (a zero P stays zero under any mask value)
      pbuf[r * kChunk + lane] =
          p.drop.on && pj != A(0)
              ? pj * drop_factor<A>(p, (static_cast<int64_t>(b) * p.Hq + hq) * p.Sq + i0 + r, j)
              : pj;
    }
    __syncthreads();
    const int n = (stop - j0) < kChunk ? static_cast<int>(stop - j0) : kChunk;
    for (int jj = 0; jj < n; ++jj) {
      A pv[R];
      bool any = false;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        pv[r] = pbuf[r * kChunk + jj];
        any |= pv[r] != A(0);
      }
      if (!any) continue;  // masked or underflowed key for every row: contributes nothing
      const T *vrow = row_ptr<T>(v, b, hk, j0 + jj);
#pragma unroll
      for (int t = 0; t < kMaxDimSlots; ++t) {
        const int d = lane + 64 * t;
        if (d < p.Dv) {
          const A vd = to_acc<A>(vrow[d]);
#pragma unroll
          for (int r = 0; r < R; ++r)
            if (pv[r] != A(0)) acc[r][t] += pv[r] * vd;
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = i0 + r;
    if (i >= p.Sq) continue;
    const A inv = l[r] > A(0) ? A(1) / l[r] : A(1);
    T *op = row_ptr_mut<T>(o, b, hq, i);
#pragma unroll
    for (int t = 0; t < kMaxDimSlots; ++t) {
      const int d = lane + 64 * t;
      if (d < p.Dv) op[d] = from_acc<T, A>(acc[r][t] * inv);
    }
    if (lse && lane == 0)
      lse[(static_cast<int64_t>(b) * p.Hq + hq) * p.Sq + i] =
          l[r] > A(0) ? m[r] + log_acc(l[r]) : neg_inf<A>();
  }
}

// ---------------------------------------------------------------------------
// Backward pass 1: delta_i = sum_d dout_i,d * out_i,d (attention.py:232).
// ---------------------------------------------------------------------------
template <typename T, typename A>
__global__ __launch_bounds__(256) void generic_delta_kernel(Problem p, View o, View dout, A *delta) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int b = blockIdx.z, hq = blockIdx.y, i = blockIdx.x * kWaves + w;
  if (i >= p.Sq) return;
  const T *op = row_ptr<T>(o, b, hq, i);
  const T *gp = row_ptr<T>(dout, b, hq, i);
  A s = 0;
  for (int d = lane; d < p.Dv; d += 64) s += to_acc<A>(op[d]) * to_acc<A>(gp[d]);
  s = wave_sum(s);
  if (lane == 0) delta[(static_cast<int64_t>(b) * p.Hq + hq) * p.Sq + i] = s;
}

// ---------------------------------------------------------------------------
// Backward pass 2: dq_i = scale * sum_j p_ij (dp_ij - delta_i) k_j (:237-239).
// Wave w owns the R query rows from (blockIdx.x * 4 + w) R, lane l the key
// j0 + l of each chunk (each K and V element a lane loads serves R rows).
// ---------------------------------------------------------------------------
template <typename T, typename A, int R, bool VK>
__global__ __launch_bounds__(256) void generic_dq_kernel(Problem p, View q, View k, View v,
                                                         View dout, const A *lse, const A *delta,
                                                         View dq) {
  extern __shared__ unsigned char smem_raw[];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int b = blockIdx.z, hq = blockIdx.y, hk = hq / p.rep;
  const int i0 = (blockIdx.x * kWaves + w) * R;
  A *qrows = reinterpret_cast<A *>(smem_raw) + w * R * (p.Dqk + p.Dv + kChunk);
  A *grows = qrows + R * p.Dqk;  // [R][Dv]
  A *dsbuf = grows + R * p.Dv;   // [R][kChunk]
  const int kv_end = kv_end_for(p, b);
  A row_lse[R], row_delta[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = i0 + r;
    row_lse[r] = 0;
    row_delta[r] = 0;
    if (i < p.Sq) {
      const T *qp = row_ptr<T>(q, b, hq, i);
      const T *gp = row_ptr<T>(dout, b, hq, i);
      for (int d = lane; d < p.Dqk; d += 64) qrows[r * p.Dqk + d] = to_acc<A>(qp[d]);
      for (int d = lane; d < p.Dv; d += 64) grows[r * p.Dv + d] = to_acc<A>(gp[d]);
      const int64_t rr = (static_cast<int64_t>(b) * p.Hq + hq) * p.Sq + i;
      row_lse[r] = lse[rr];
      if (!isfinite(row_lse[r])) row_lse[r] = 0;  // safe_lse (:231)
      row_delta[r] = delta[rr];
    } else {
      for (int d = lane; d < p.Dqk; d += 64) qrows[r * p.Dqk + d] = A(0);
      for (int d = lane; d < p.Dv; d += 64) grows[r * p.Dv + d] = A(0);
    }
  }
  int64_t last_row = (static_cast<int64_t>(blockIdx.x) * kWaves + kWaves) * R - 1;
  if (last_row > p.Sq - 1) last_row = p.Sq - 1;
  int64_t stop = kv_end;
  if (p.causal && last_row + p.offset + 1 < stop) stop = last_row + p.offset + 1;
  if (stop < 0) stop = 0;
  __syncthreads();

  A acc[R][kMaxDimSlots];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int t = 0; t < kMaxDimSlots; ++t) acc[r][t] = 0;
  const A scale = static_cast<A>(p.scale);
  for (int j0 = 0; j0 < stop; j0 += kChunk) {
    const int j = j0 + lane;
    A ds[R];
#pragma unroll
    for (int r = 0; r < R; ++r) ds[r] = 0;
    if (j < kv_end) {
      A s[R];
      score_rows<T, A, R, VK>(p, qrows, row_ptr<T>(k, b, hk, j), b, hq, i0, j, kv_end, s);
      A dp[R];
#pragma unroll
      for (int r = 0; r < R; ++r) dp[r] = 0;
      const T *vrow = row_ptr<T>(v, b, hk, j);
      int d = 0;
      if constexpr (VK) {
        constexpr int VW = 16 / sizeof(T);
        typedef T V __attribute__((ext_vector_type(VW)));
        for (; d + VW <= p.Dv; d += VW) {
          const V vv = *reinterpret_cast<const V *>(vrow + d);
#pragma unroll
          for (int e = 0; e < VW; ++e) {
            const A vd = to_acc<A>(static_cast<T>(vv[e]));
#pragma unroll
            for (int r = 0; r < R; ++r) dp[r] += grows[r * p.Dv + d + e] * vd;
          }
        }
      }
      for (; d < p.Dv; ++d) {
        const A vd = to_acc<A>(vrow[d]);
#pragma unroll
        for (int r = 0; r < R; ++r) dp[r] += grows[r * p.Dv + d] * vd;
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const A pij = exp_acc(s[r] - row_lse[r]);  // 0 for rows from Sq on
        if (pij != A(0)) {
          A dpr = dp[r];
          if (p.drop.on)
            dpr *= drop_factor<A>(p, (static_cast<int64_t>(b) * p.Hq + hq) * p.Sq + i0 + r, j);
          ds[r] = pij * (dpr - row_delta[r]) * scale;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) dsbuf[r * kChunk + lane] = ds[r];
    __syncthreads();
    const int n = (stop - j0) < kChunk ? static_cast<int>(stop - j0) : kChunk;
    for (int jj = 0; jj < n; ++jj) {
      A c[R];
      bool any = false;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        c[r] = dsbuf[r * kChunk + jj];
        any |= c[r] != A(0);
      }
      if (!any) continue;
      const T *krow = row_ptr<T>(k, b, hk, j0 + jj);
#pragma unroll
      for (int t = 0; t < kMaxDimSlots; ++t) {
        const int d = lane + 64 * t;
        if (d < p.Dqk) {
          const A kd = to_acc<A>(krow[d]);
#pragma unroll
          for (int r = 0; r < R; ++r)
            if (c[r] != A(0)) acc[r][t] += c[r] * kd;
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = i0 + r;
    if (i >= p.Sq) continue;
    T *out = row_ptr_mut<T>(dq, b, hq, i);
#pragma unroll
    for (int t = 0; t < kMaxDimSlots; ++t) {
      const int d = lane + 64 * t;
      if (d < p.Dqk) out[d] = from_acc<T, A>(acc[r][t]);
    }
  }
}

// ---------------------------------------------------------------------------
// Backward pass 3: per key row j of KV head hk, summed over the query heads
// of its group (:240-247): dv_j = sum_i p_ij dout_i, dk_j = sum_i ds_ij q_i.
// grid (ceil(Sk/NW), Hkv, B), NW waves = keys per workgroup: eight when the
// Q / dO chunk is staged (it serves twice the keys), else four.
// ---------------------------------------------------------------------------
template <bool ST>
constexpr int dkdv_waves() {
  return ST ? 8 : 4;
}

template <typename T, typename A, bool ST>
__global__ __launch_bounds__(64 * dkdv_waves<ST>()) void generic_dkdv_kernel(
    Problem p, View q, View k, View v, View dout, const A *lse, const A *delta, View dk, View dv) {
  constexpr int NW = dkdv_waves<ST>();
  extern __shared__ unsigned char smem_raw[];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int b = blockIdx.z, hk = blockIdx.y;
  const int j = blockIdx.x * NW + w;
  const int kv_end = kv_end_for(p, b);
  const bool key_ok = j < p.Sk;
  // per wave: K row, V row (each from a 16-byte boundary), P and dS chunks
  constexpr int esz = sizeof(A);
  const int dq16 = round16(p.Dqk, esz), kreg = dq16 + round16(p.Dv, esz) + 2 * kChunk;
  A *krow = reinterpret_cast<A *>(smem_raw) + w * kreg;
  A *vrow = krow + dq16;
  A *pbuf = vrow + round16(p.Dv, esz);
  A *dsbuf = pbuf + kChunk;
  // staged Q / dO chunk (ST)
  const int ldq = staged_ld(p.Dqk, esz), ldg = staged_ld(p.Dv, esz);
  A *qst = reinterpret_cast<A *>(smem_raw) + NW * kreg;
  A *gst = qst + kChunk * ldq;
  if (key_ok) {
    const T *kp = row_ptr<T>(k, b, hk, j);
    const T *vp = row_ptr<T>(v, b, hk, j);
    for (int d = lane; d < p.Dqk; d += 64) krow[d] = to_acc<A>(kp[d]);
    for (int d = lane; d < p.Dv; d += 64) vrow[d] = to_acc<A>(vp[d]);
  }
  // First query row that can see any key of this workgroup (causal).
  int64_t first_key = static_cast<int64_t>(blockIdx.x) * NW;
  int64_t start = 0;
  if (p.causal) {
    start = first_key - p.offset;
    if (start < 0) start = 0;
    start = (start / kChunk) * kChunk;
  }
  __syncthreads();

  A acc_k[kMaxDimSlots], acc_v[kMaxDimSlots];
#pragma unroll
  for (int t = 0; t < kMaxDimSlots; ++t) acc_k[t] = acc_v[t] = 0;
  const A scale = static_cast<A>(p.scale);
  for (int r = 0; r < p.rep; ++r) {
    const int hq = hk * p.rep + r;
    for (int64_t i0 = start; i0 < p.Sq; i0 += kChunk) {
      const int i = static_cast<int>(i0) + lane;
      if constexpr (ST) {
        stage_chunk<T, A, NW>(qst, q, b, hq, i0, p.Sq, p.Dqk, ldq);
        stage_chunk<T, A, NW>(gst, dout, b, hq, i0, p.Sq, p.Dv, ldg);
        __syncthreads();
      }
      A pij = 0, ds = 0;
      if (key_ok && j < kv_end && i < p.Sq) {
        A acc = 0;
        if constexpr (ST) {
          acc = dot_lds(qst + lane * ldq, krow, p.Dqk);
        } else {
          // q row i is read straight from memory (lane-private row)
          const T *qp = row_ptr<T>(q, b, hq, i);
          for (int d = 0; d < p.Dqk; ++d) acc += to_acc<A>(qp[d]) * krow[d];
        }
        A s = acc * scale;
        bool ok = !(p.causal && static_cast<int64_t>(i) + p.offset < static_cast<int64_t>(j));
        if (ok && p.mask.kind != TSATTN_MASK_NONE) {
          int64_t mi = b * p.mask.s0 + hq * p.mask.s1 + static_cast<int64_t>(i) * p.mask.s2 +
                       static_cast<int64_t>(j) * p.mask.s3;
          if (p.mask.kind == TSATTN_MASK_BOOL) {
            ok = static_cast<const uint8_t *>(p.mask.data)[mi] != 0;
          } else {
            s += load_additive<A>(p.mask.data, mi, p.mask.dtype);
          }
        }
        if (ok) {
          const int64_t rr = (static_cast<int64_t>(b) * p.Hq + hq) * p.Sq + i;
          A l = lse[rr];
          if (!isfinite(l)) l = 0;
          pij = exp_acc(s - l);
          if (pij != A(0)) {
            A dp = 0;
            if constexpr (ST) {
              dp = dot_lds(gst + lane * ldg, vrow, p.Dv);
            } else {
              const T *gp = row_ptr<T>(dout, b, hq, i);
              for (int d = 0; d < p.Dv; ++d) dp += to_acc<A>(gp[d]) * vrow[d];
            }
            const A f = drop_factor<A>(p, rr, j);  // rr = the query row's index
            ds = pij * (dp * f - delta[rr]) * scale;
            pij *= f;  // dV takes P * mask
          }
        }
      }
      pbuf[lane] = pij;
      dsbuf[lane] = ds;
      __syncthreads();
      const int n = (p.Sq - i0) < kChunk ? static_cast<int>(p.Sq - i0) : kChunk;
      for (int ii = 0; ii < n; ++ii) {
        const A pv = pbuf[ii], dsv = dsbuf[ii];
        if (pv == A(0) && dsv == A(0)) continue;
        if constexpr (ST) {
          const A *gr = gst + ii * ldg, *qr = qst + ii * ldq;
#pragma unroll
          for (int t = 0; t < kMaxDimSlots; ++t) {
            const int d = lane + 64 * t;
            if (d < p.Dv) acc_v[t] += pv * gr[d];
            if (d < p.Dqk) acc_k[t] += dsv * qr[d];
          }
        } else {
          const T *gp = row_ptr<T>(dout, b, hq, static_cast<int>(i0) + ii);
          const T *qp = row_ptr<T>(q, b, hq, static_cast<int>(i0) + ii);
#pragma unroll
          for (int t = 0; t < kMaxDimSlots; ++t) {
            const int d = lane + 64 * t;
            if (d < p.Dv) acc_v[t] += pv * to_acc<A>(gp[d]);
            if (d < p.Dqk) acc_k[t] += dsv * to_acc<A>(qp[d]);
          }
        }
      }
      __syncthreads();
    }
  }
  if (!key_ok) return;
  T *kout = row_ptr_mut<T>(dk, b, hk, j);
  T *vout = row_ptr_mut<T>(dv, b, hk, j);
#pragma unroll
  for (int t = 0; t < kMaxDimSlots; ++t) {
    const int d = lane + 64 * t;
    if (d < p.Dqk) kout[d] = from_acc<T, A>(acc_k[t]);
    if (d < p.Dv) vout[d] = from_acc<T, A>(acc_v[t]);
  }
}

// LDS of one staged 64-row chunk of each of two operands (row strides
// staged_ld).
template <typename A>
size_t staged_bytes(const Problem &p) {
  return static_cast<size_t>(kChunk) *
         (staged_ld(p.Dqk, sizeof(A)) + staged_ld(p.Dv, sizeof(A))) * sizeof(A);
}

// Whether `kernel` may take `smem` bytes of dynamic LDS: at most the 160 KiB a
// gfx950 workgroup can hold, and above 64 KiB only once the runtime accepts
// the kernel's raised limit (asked on every call: cheap, and per device).
inline bool lds_ok(const void *kernel, size_t smem) {
  if (smem > 160 * 1024) return false;
  if (smem <= 64 * 1024) return true;
  return hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                             static_cast<int>(smem)) == hipSuccess;
}

// Query rows per wave of the forward and dQ kernels: four, or one where the
// runtime refuses their LDS (up to 139 KiB for fp64 at head dims of 512).
constexpr int kRows = 4;

// Every row of the view starts on a 16-byte boundary (base and strides).
template <typename T>
bool rows16(const View &x) {
  const auto al = [](int64_t n) { return (n * static_cast<int64_t>(sizeof(T))) % 16 == 0; };
  return reinterpret_cast<uintptr_t>(x.data) % 16 == 0 && al(x.s0) && al(x.s1) && al(x.s2);
}

template <typename T, typename A>
hipError_t forward_impl(const Problem &p, View q, View k, View v, View o, void *lse,
                        hipStream_t st) {
  const size_t smem4 = static_cast<size_t>(kWaves) * kRows * (p.Dqk + kChunk) * sizeof(A);
  Probe pr_("generic_fwd", st);
  if (lds_ok(reinterpret_cast<const void *>(&generic_forward_kernel<T, A, kRows, false>), smem4) &&
      lds_ok(reinterpret_cast<const void *>(&generic_forward_kernel<T, A, kRows, true>), smem4)) {
    const dim3 grid((p.Sq + kWaves * kRows - 1) / (kWaves * kRows), p.Hq, p.B);
    if (rows16<T>(k))
      generic_forward_kernel<T, A, kRows, true><<<grid, dim3(256), smem4, st>>>(p, q, k, v, o, static_cast<A *>(lse));
    else
      generic_forward_kernel<T, A, kRows, false><<<grid, dim3(256), smem4, st>>>(p, q, k, v, o, static_cast<A *>(lse));
  } else {
    const dim3 grid((p.Sq + kWaves - 1) / kWaves, p.Hq, p.B);
    const size_t smem = static_cast<size_t>(kWaves) * (p.Dqk + kChunk) * sizeof(A);
    generic_forward_kernel<T, A, 1, false><<<grid, dim3(256), smem, st>>>(p, q, k, v, o, static_cast<A *>(lse));
  }
  return hipGetLastError();
}

template <typename T, typename A>
hipError_t backward_impl(const Problem &p, View q, View k, View v, View o, View dout,
                         const void *lse, View dq, View dk, View dv, void *delta,
                         hipStream_t st) {
  A *dl = static_cast<A *>(delta);
  const A *ls = static_cast<const A *>(lse);
  dim3 grid_q((p.Sq + kWaves - 1) / kWaves, p.Hq, p.B);
  { Probe pr_("generic_bwd_delta", st); generic_delta_kernel<T, A><<<grid_q, dim3(256), 0, st>>>(p, o, dout, dl); }
  {
    const size_t smem4 = static_cast<size_t>(kWaves) * kRows * (p.Dqk + p.Dv + kChunk) * sizeof(A);
    Probe pr_("generic_bwd_dq", st);
    if (lds_ok(reinterpret_cast<const void *>(&generic_dq_kernel<T, A, kRows, false>), smem4) &&
        lds_ok(reinterpret_cast<const void *>(&generic_dq_kernel<T, A, kRows, true>), smem4)) {
      const dim3 grid((p.Sq + kWaves * kRows - 1) / (kWaves * kRows), p.Hq, p.B);
      if (rows16<T>(k) && rows16<T>(v))
        generic_dq_kernel<T, A, kRows, true><<<grid, dim3(256), smem4, st>>>(p, q, k, v, dout, ls, dl, dq);
      else
        generic_dq_kernel<T, A, kRows, false><<<grid, dim3(256), smem4, st>>>(p, q, k, v, dout, ls, dl, dq);
    } else {
      const size_t smem_q = static_cast<size_t>(kWaves) * (p.Dqk + p.Dv + kChunk) * sizeof(A);
      generic_dq_kernel<T, A, 1, false><<<grid_q, dim3(256), smem_q, st>>>(p, q, k, v, dout, ls, dl, dq);
    }
  }
  constexpr int nws = dkdv_waves<true>(), nwd = dkdv_waves<false>();
  const size_t smem_ks = static_cast<size_t>(nws) *
                             (round16(p.Dqk, sizeof(A)) + round16(p.Dv, sizeof(A)) + 2 * kChunk) *
                             sizeof(A) +
                         staged_bytes<A>(p);
  {
    Probe pr_("generic_bwd_dkdv", st);
    if (lds_ok(reinterpret_cast<const void *>(&generic_dkdv_kernel<T, A, true>), smem_ks)) {
      const dim3 grid_k((p.Sk + nws - 1) / nws, p.Hkv, p.B);
      generic_dkdv_kernel<T, A, true><<<grid_k, dim3(64 * nws), smem_ks, st>>>(p, q, k, v, dout, ls, dl, dk, dv);
    } else {
      const dim3 grid_k((p.Sk + nwd - 1) / nwd, p.Hkv, p.B);
      const size_t smem_k = static_cast<size_t>(nwd) *
                            (round16(p.Dqk, sizeof(A)) + round16(p.Dv, sizeof(A)) + 2 * kChunk) *
                            sizeof(A);
      generic_dkdv_kernel<T, A, false><<<grid_k, dim3(64 * nwd), smem_k, st>>>(p, q, k, v, dout, ls, dl, dk, dv);
    }
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_generic_forward(const Problem &p, int dtype, View q, View k, View v, View o,
                                  void *lse, hipStream_t st) {
  switch (dtype) {
    case TSATTN_F32: return forward_impl<float, float>(p, q, k, v, o, lse, st);
    case TSATTN_F64: return forward_impl<double, double>(p, q, k, v, o, lse, st);
    case TSATTN_F16: return forward_impl<f16, float>(p, q, k, v, o, lse, st);
    case TSATTN_BF16: return forward_impl<bf16, float>(p, q, k, v, o, lse, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_generic_backward(const Problem &p, int dtype, View q, View k, View v, View o,
                                   View dout, const void *lse, View dq, View dk, View dv,
                                   void *delta, hipStream_t st) {
  switch (dtype) {
    case TSATTN_F32: return backward_impl<float, float>(p, q, k, v, o, dout, lse, dq, dk, dv, delta, st);
    case TSATTN_F64: return backward_impl<double, double>(p, q, k, v, o, dout, lse, dq, dk, dv, delta, st);
    case TSATTN_F16: return backward_impl<f16, float>(p, q, k, v, o, dout, lse, dq, dk, dv, delta, st);
    case TSATTN_BF16: return backward_impl<bf16, float>(p, q, k, v, o, dout, lse, dq, dk, dv, delta, st);
  }
  return hipErrorInvalidValue;
}

// Key-padding mask -> (kv_len, kv_prefix): one wave per batch row.
__global__ __launch_bounds__(256) void key_mask_lengths_kernel(const uint8_t *mask, int64_t sb,
                                                               int64_t sk, int K, int32_t *kv_len,
                                                               int32_t *kv_prefix) {
  typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
  __shared__ int red[2][4];
  const int b = blockIdx.x, t = threadIdx.x;
  const uint8_t *row = mask + b * sb;
  int last = -1, count = 0;
  int j0 = 0;
  if (sk == 1 && reinterpret_cast<uintptr_t>(row) % 16 == 0) {
    // 16 bytes per load; bit 7 of byte i of f is set iff byte i is nonzero.
    const int nv = K / 16;
    for (int v = t; v < nv; v += 256) {
      const u32x4_t x = *reinterpret_cast<const u32x4_t *>(row + 16 * static_cast<int64_t>(v));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const unsigned f = (((x[e] & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | x[e]) & 0x80808080u;
        count += __builtin_popcount(f);
        if (f) last = 16 * v + 4 * e + (31 - __builtin_clz(f)) / 8;
      }
    }
    j0 = nv * 16;
  }
  for (int j = j0 + t; j < K; j += 256) {
    if (row[static_cast<int64_t>(j) * sk]) {
      last = j;
      ++count;
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const int o = __shfl_xor(last, m, 64);
    last = last > o ? last : o;
    count += __shfl_xor(count, m, 64);
  }
  if ((t & 63) == 0) {
    red[0][t >> 6] = last;
    red[1][t >> 6] = count;
  }
  __syncthreads();
  if (t == 0) {
    last = max(max(red[0][0], red[0][1]), max(red[0][2], red[0][3]));
    count = red[1][0] + red[1][1] + red[1][2] + red[1][3];
    kv_len[b] = last + 1;
    if (kv_prefix) kv_prefix[b] = (count == last + 1) ? 1 : 0;
  }
}

hipError_t launch_key_mask_lengths(const uint8_t *mask, int64_t sb, int64_t sk, int B, int K,
                                   int32_t *kv_len, int32_t *kv_prefix, hipStream_t st) {
  { Probe pr_("key_mask_lengths", st); key_mask_lengths_kernel<<<dim3(B), dim3(256), 0, st>>>(mask, sb, sk, K, kv_len, kv_prefix); }
  return hipGetLastError();
}

}  // namespace tsattn
