// Attention backward for gfx950 with MFMA 32x32x16 (f16/bf16 in, fp32
// accumulate).  Follows the reference's streaming VJP (src/tensorsmith/nn/
// attention.py:220-247):
//   delta_i = sum_d dO_id O_id                     (row_prep_kernel)
//   P_ij = exp(S_ij - LSE_i), dS_ij = P_ij (dP_ij - delta_i), dP = dO V^T
//   dV = P^T dO, dK = scale dS^T Q                 (dkdv_kernel)
//   dQ = scale dS K                                (dq_kernel)
// dK/dV and dQ are produced by two kernels that each own their output tile,
// so every gradient element is written exactly once: no atomics, bitwise
// deterministic results (checkpoint recompute reproduces them exactly).
// The dK/dV kernel sums the query heads of a GQA group itself (:245-247).
//
// Tiles reach LDS by direct buffer loads into swizzled row-major layouts;
// transposed operands (Q^T, dO^T, K^T) come from LDS transpose reads.
#include <type_traits>

#include "mfma_common.h"

namespace tsattn {
namespace {

constexpr int NT = 256;
constexpr int NW = NT / 64;

struct BwdArgs {
  Problem p;
  View q, k, v, o, dout, dq, dk, dv;
  const float *lse;
  float *delta;  // [rows] delta, then [rows] lse2 = safe(lse) * log2(e)
  float sl;      // scale * log2(e)
  float scale;   // final gradient scale
};

template <typename T>
__device__ __forceinline__ T *mut(View v) {
  return static_cast<T *>(const_cast<void *>(v.data));
}
template <typename T>
__device__ __forceinline__ const T *head_ptr(View v, int b, int h) {
  return static_cast<const T *>(v.data) + b * v.s0 + h * v.s1;
}

// ---------------------------------------------------------------------------
// Row pre-pass: delta = rowsum(dO * O) and lse2 = (isfinite(lse) ? lse : 0) *
// log2(e) -- the reference's safe_lse (attention.py:231) in exp2 units.
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(NT) void row_prep_kernel(BwdArgs a) {
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
  if (row < rows && part == 0) {
    a.delta[row] = s;
    const float l = a.lse[row];
    a.delta[rows + row] = isfinite(l) ? l * kLog2e : 0.f;
  }
}

// ---------------------------------------------------------------------------
// dK / dV: one workgroup = 128 keys of one (b, kv head), 8 wavefronts.  The
// workgroup's K and V rows stay in LDS for its whole life (blocked layout,
// loaded once by DMA); query tiles of 64 rows -- Q, dO and their lse2 /
// delta values, for every query head of the GQA group -- stream through a
// 2-stage ring by DMA loads, one fence-free barrier per tile.  Wave w owns
// key group kg = w % 4 (32 keys) and query half qh = w / 4 (32 rows of each
// tile), so its persistent state is its dK^T / dV^T accumulators and two
// waves share each SIMD; the query halves' partial sums are added through
// LDS at the end.  Per tile a wave computes S = Q K^T and dP = dO V^T from
// row fragments (16 MFMAs), P and dS on the VALU, then dV^T += dO^T P and
// dK^T += Q^T dS from column fragments (16 MFMAs); fragments are prefetched
// two steps ahead.
// ---------------------------------------------------------------------------
constexpr int KB = 128;   // keys per workgroup
constexpr int QT = 64;    // query rows per tile
constexpr int NTK = 512;  // threads of the dK/dV kernel
constexpr int NWK = NTK / 64;
constexpr int KV_NS = 2;  // Q / dO ring stages

template <typename T, int D>
__global__ __launch_bounds__(NTK, 2) void dkdv_kernel(BwdArgs a) {
  constexpr int KV_B = KB * D * 2;           // bytes of the K (or V) block
  constexpr int TILE_B = QT * D * 2;         // bytes of a Q (or dO) tile
  constexpr int KBLK = KV_B / 1024, NBLK = TILE_B / 1024;
  constexpr int STAGE_B = 2 * TILE_B + 1024; // Q | dO | lse2 (256 B) delta (256 B), padded
  constexpr int LPT = 2 * NBLK / NWK;        // Q + dO DMA loads per wave per tile
  constexpr int SKS = D / 16, PDT = D / 32, QG = D / 32;
  // workgroups resident per CU: 160 KiB of LDS, at most two by the launch bounds
  constexpr int kLdsFit = 160 * 1024 / (2 * KV_B + KV_NS * STAGE_B);
  constexpr int kWgPerCu = kLdsFit < 2 ? kLdsFit : 2;
  static_assert(LPT >= 1 && LPT * NWK == 2 * NBLK, "tile loads must split evenly over the waves");
  static_assert(2 * KBLK % NWK == 0, "K/V loads must split evenly over the waves");
  static_assert(SKS == 2 * PDT, "one dV and one dK MFMA per step");
  __shared__ __attribute__((aligned(1024))) char kv_lds[2 * KV_B];            // K | V
  __shared__ __attribute__((aligned(1024))) char ring[KV_NS * STAGE_B];

  const Problem &p = a.p;
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 31, h = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kg = w & 3, qh = w >> 2;
  const int n_kb = (p.Sk + KB - 1) / KB;
  const int total = n_kb * p.Hkv * p.B;
  const int logical = xcd_remap(blockIdx.x, total);
  int bh, kb;  // early key blocks see the most queries: run them first
  heavy_first(logical, n_kb, p.Hkv * p.B, 32 * kWgPerCu, bh, kb);
  const int b = bh / p.Hkv, hk = bh - b * p.Hkv;
  const int k0 = kb * KB, kw = k0 + 32 * kg, key = kw + c;
  const int kv_end = kv_end_for(p, b);
  const bool keymask = p.mask.kind == TSATTN_MASK_BOOL && !(p.kv_prefix && p.kv_prefix[b]);
  const bool key_live = key < kv_end &&
                        (!keymask || static_cast<const uint8_t *>(p.mask.data)
                                         [b * p.mask.s0 + static_cast<int64_t>(key) * p.mask.s3]);
  const int64_t rows = static_cast<int64_t>(p.B) * p.Hq * p.Sq;
  const bool causal = p.causal != 0;

  // Query tiles: only rows that can see a key of this block (causal).
  int q_start = 0;
  if (causal) {
    const int64_t s0 = static_cast<int64_t>(k0) - p.offset;
    q_start = s0 <= 0 ? 0 : static_cast<int>(s0 < p.Sq ? s0 : p.Sq);
    q_start = (q_start / QT) * QT;
  }
  const int n_qt = k0 < kv_end ? (p.Sq - q_start + QT - 1) / QT : 0;
  const int n_iter = n_qt * p.rep;

  const uint32_t qs_b = static_cast<uint32_t>(a.q.s2) * 2, gs_b = static_cast<uint32_t>(a.dout.s2) * 2;
  const uint32_t ks_b = static_cast<uint32_t>(a.k.s2) * 2, vs_b = static_cast<uint32_t>(a.v.s2) * 2;
  const uint32_t kv0 = lds_addr(kv_lds), ring0 = lds_addr(ring);
  // Blocked layout: block n = (n / QG, n % QG); its lane l fetches row
  // 16 (n / QG) + l / 4, chunk 4 (n % QG) + ((l % 4) ^ ((l / 16) % 4)).  A
  // wave's blocks are w, w + 8, ..., all with n % QG = w % QG.
  const uint32_t lane_chunk = 4 * (w % QG) + ((lane & 3) ^ ((lane >> 4) & 3));
  const uint32_t lrow = lane >> 2;
  const int lpt_w = LPT + (w < 2 ? 1 : 0);  // waves 0 / 1 also load lse2 / delta
  auto tile_of = [&](int itn, int &hq, int &q0) {
    const int r = itn / n_qt;
    hq = hk * p.rep + r;
    q0 = q_start + (itn - r * n_qt) * QT;
  };
  auto issue = [&](int itn) {
    int hq, q0;
    tile_of(itn, hq, q0);
    const uint32_t st = ring0 + (itn % KV_NS) * STAGE_B;
    const u32x4 qdesc = make_desc(head_ptr<T>(a.q, b, hq), static_cast<uint32_t>(p.Sq) * qs_b);
    const u32x4 gdesc = make_desc(head_ptr<T>(a.dout, b, hq), static_cast<uint32_t>(p.Sq) * gs_b);
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int e = w + NWK * u;
      const int n = e < NBLK ? e : e - NBLK;
      const uint32_t row0 = static_cast<uint32_t>(q0 + 16 * (n / QG));
      if (e < NBLK) dma16(qdesc, st + n * 1024, lrow * qs_b + lane_chunk * 16, row0 * qs_b);
      else dma16(gdesc, st + TILE_B + n * 1024, lrow * gs_b + lane_chunk * 16, row0 * gs_b);
    }
    if (w < 2) {
      const int64_t base = (static_cast<int64_t>(b) * p.Hq + hq) * p.Sq + (w == 0 ? rows : 0);
      const u32x4 rdesc = make_desc(a.delta + base, static_cast<uint32_t>(p.Sq) * 4);
      if (lane < QT / 4) dma16(rdesc, st + 2 * TILE_B + w * QT * 4, lane * 16, static_cast<uint32_t>(q0) * 4);
    }
  };

  const TileReader<T, D> rd(lane);
  f32x16 dk_acc[PDT], dv_acc[PDT];
#pragma unroll
  for (int dt = 0; dt < PDT; ++dt) dk_acc[dt] = dv_acc[dt] = f32x16{};
  const float sl = a.sl;

  // No zeroing: every LDS byte the loop reads is written by a DMA load first
  // (lanes past a buffer's range write zeros).
  if (n_iter > 0) {
    const u32x4 kdesc = make_desc(head_ptr<T>(a.k, b, hk), static_cast<uint32_t>(kv_end) * ks_b);
    const u32x4 vdesc = make_desc(head_ptr<T>(a.v, b, hk), static_cast<uint32_t>(kv_end) * vs_b);
#pragma unroll
    for (int u = 0; u < 2 * KBLK / NWK; ++u) {
      const int e = w + NWK * u;
      const int n = e < KBLK ? e : e - KBLK;
      const uint32_t row0 = static_cast<uint32_t>(k0 + 16 * (n / QG));
      if (e < KBLK) dma16(kdesc, kv0 + n * 1024, lrow * ks_b + lane_chunk * 16, row0 * ks_b);
      else dma16(vdesc, kv0 + KV_B + n * 1024, lrow * vs_b + lane_chunk * 16, row0 * vs_b);
    }
    issue(0);
  }
  wait_vm(0);
  __syncthreads();

  const char *kt = kv_lds, *vt = kv_lds + KV_B;
  for (int itn = 0; itn < n_iter; ++itn) {
    if (itn + 1 < n_iter) issue(itn + 1);
    const char *qt = ring + (itn % KV_NS) * STAGE_B;
    const char *gt = qt + TILE_B;
    const float *rv = reinterpret_cast<const float *>(qt + 2 * TILE_B);
    int hq, q0;
    tile_of(itn, hq, q0);
    const int qs = q0 + 32 * qh;  // first query row of this wave's half

    constexpr int FD = 2;
    // S = Q K^T, dP = dO V^T over this wave's 32 rows x 32 keys:
    // sacc[e] = S[qs + crow(e, h)][key].  B operands are K / V row fragments.
    f32x16 sacc = f32x16{}, dpacc = f32x16{};
    {
      u32x4 qa[FD + 1], ga[FD + 1], kb_[FD + 1], vb[FD + 1];
      auto load = [&](int i) {
        qa[i % (FD + 1)] = rd.rows(qt, qh, i);
        ga[i % (FD + 1)] = rd.rows(gt, qh, i);
        kb_[i % (FD + 1)] = rd.rows(kt, kg, i);
        vb[i % (FD + 1)] = rd.rows(vt, kg, i);
      };
#pragma unroll
      for (int i = 0; i < FD; ++i) load(i);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < SKS; ++i) {
        sacc = mfma32<T>(qa[i % (FD + 1)], kb_[i % (FD + 1)], sacc);
        dpacc = mfma32<T>(ga[i % (FD + 1)], vb[i % (FD + 1)], dpacc);
        if (i + FD < SKS) load(i + FD);
        __builtin_amdgcn_sched_barrier(0);
      }
    }

    // P = exp2(S sl - lse2), dS = P (dP - delta); rows crow(e, h) = 8 g + 4 h + e % 4.
    const bool edge = keymask || kw + 32 > kv_end || qs + 32 > p.Sq ||
                      (causal && static_cast<int64_t>(qs) + p.offset < kw + 31);
    int lo = -64, hi = 64;
    if (edge) {
      hi = key_live ? p.Sq - qs - 4 * h : -64;
      if (causal) {
        const int64_t l0 = static_cast<int64_t>(key) - p.offset - qs - 4 * h;
        lo = l0 < -64 ? -64 : (l0 > 64 ? 64 : static_cast<int>(l0));
      }
    }
    u32x4 pp[2], pd[2];
    // Interior tiles skip the per-element bounds (three VALU ops each).
    auto grad = [&](auto masked) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 l4 = *reinterpret_cast<const float4 *>(rv + 32 * qh + 8 * g + 4 * h);
        const float4 d4 = *reinterpret_cast<const float4 *>(rv + QT + 32 * qh + 8 * g + 4 * h);
        const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
        const float dl[4] = {d4.x, d4.y, d4.z, d4.w};
        float pv[4], dsv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int e = 4 * g + r, kc = 8 * g + r;
          pv[r] = fast_exp2(fmaf(sacc[e], sl, -lv[r]));
          if (masked) pv[r] = (kc >= lo) & (kc < hi) ? pv[r] : 0.f;
          dsv[r] = pv[r] * (dpacc[e] - dl[r]);
        }
        pp[g >> 1][(g & 1) * 2] = pack2<T>(pv[0], pv[1]);
        pp[g >> 1][(g & 1) * 2 + 1] = pack2<T>(pv[2], pv[3]);
        pd[g >> 1][(g & 1) * 2] = pack2<T>(dsv[0], dsv[1]);
        pd[g >> 1][(g & 1) * 2 + 1] = pack2<T>(dsv[2], dsv[3]);
      }
    };
    if (edge) grad(std::true_type{});
    else grad(std::false_type{});

    // dV^T += dO^T P, dK^T += Q^T dS over this wave's 32 query rows; step i:
    // value block i % PDT, query k-step i / PDT (rows 32 qh + 16 (i / PDT) ..).
    {
      u32x4 gc[FD + 1], qc[FD + 1];
      auto load = [&](int i) {
        gc[i % (FD + 1)] = rd.cols(gt, 2 * qh + i / PDT, i % PDT);
        qc[i % (FD + 1)] = rd.cols(qt, 2 * qh + i / PDT, i % PDT);
      };
#pragma unroll
      for (int i = 0; i < FD; ++i) load(i);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < SKS; ++i) {
        dv_acc[i % PDT] = mfma32<T>(gc[i % (FD + 1)], pp[i / PDT], dv_acc[i % PDT]);
        dk_acc[i % PDT] = mfma32<T>(qc[i % (FD + 1)], pd[i / PDT], dk_acc[i % PDT]);
        if (i + FD < SKS) load(i + FD);
        __builtin_amdgcn_sched_barrier(0);
      }
    }

    wait_vm(0);  // the next tile (issued at the top of this iteration)
    wait_lgkm0();
    phase_barrier();
  }

  // Epilogue.  The loop ended on a barrier after every wave's last LDS read,
  // so both LDS areas are free.  Slice kg of each holds, per tensor, the
  // partial dK^T (ring) / dV^T (K/V area) of the qh = 1 wave with that kg as
  // [dt][g][lane] float4 runs.  The qh = 0 wave adds them to its own, scales,
  // rounds, and writes the block's rows back into the front of its slice:
  // key row r (0..31) at r * 2D bytes, 16-byte chunk q at q ^ (r % CPR), the
  // XOR keeping the row writes off one bank.  Then every thread stores whole
  // 16-byte chunks of rows, so the global writes are coalesced.
  constexpr int CPR = D / 8;                                   // 16-byte chunks per row
  constexpr int SLICE_B = PDT * 4 * 64 * 16;                   // per wave, per tensor
  static_assert(sizeof(ring) >= 4 * SLICE_B && sizeof(kv_lds) >= 4 * SLICE_B, "epilogue LDS");
  static_assert(32 * 2 * D <= SLICE_B, "rows fit in a slice");
  static_assert(KB * CPR % NTK == 0, "store chunks split evenly over the threads");
  char *slice_k = ring + kg * SLICE_B, *slice_v = kv_lds + kg * SLICE_B;
  if (qh == 1) {
#pragma unroll
    for (int dt = 0; dt < PDT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int off = ((dt * 4 + g) * 64 + lane) * 16;
        *reinterpret_cast<float4 *>(slice_k + off) =
            float4{dk_acc[dt][4 * g], dk_acc[dt][4 * g + 1], dk_acc[dt][4 * g + 2], dk_acc[dt][4 * g + 3]};
        *reinterpret_cast<float4 *>(slice_v + off) =
            float4{dv_acc[dt][4 * g], dv_acc[dt][4 * g + 1], dv_acc[dt][4 * g + 2], dv_acc[dt][4 * g + 3]};
      }
  }
  __syncthreads();
  if (qh == 0) {
#pragma unroll
    for (int dt = 0; dt < PDT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int off = ((dt * 4 + g) * 64 + lane) * 16;
        const float4 pk = *reinterpret_cast<const float4 *>(slice_k + off);
        const float4 pv = *reinterpret_cast<const float4 *>(slice_v + off);
        dk_acc[dt][4 * g] += pk.x, dk_acc[dt][4 * g + 1] += pk.y;
        dk_acc[dt][4 * g + 2] += pk.z, dk_acc[dt][4 * g + 3] += pk.w;
        dv_acc[dt][4 * g] += pv.x, dv_acc[dt][4 * g + 1] += pv.y;
        dv_acc[dt][4 * g + 2] += pv.z, dv_acc[dt][4 * g + 3] += pv.w;
      }
    // lane holds dK^T[d = 32 dt + 8 g + 4 h + r][key row c]: 4 consecutive d
    const float sc = a.scale;
#pragma unroll
    for (int dt = 0; dt < PDT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int off = c * 2 * D + (((4 * dt + g) ^ (c % CPR)) * 16) + 8 * h;
        *reinterpret_cast<u32x2 *>(slice_k + off) =
            u32x2{pack2<T>(dk_acc[dt][4 * g] * sc, dk_acc[dt][4 * g + 1] * sc),
                  pack2<T>(dk_acc[dt][4 * g + 2] * sc, dk_acc[dt][4 * g + 3] * sc)};
        *reinterpret_cast<u32x2 *>(slice_v + off) =
            u32x2{pack2<T>(dv_acc[dt][4 * g], dv_acc[dt][4 * g + 1]),
                  pack2<T>(dv_acc[dt][4 * g + 2], dv_acc[dt][4 * g + 3])};
      }
  }
  __syncthreads();
  T *dkb = mut<T>(a.dk) + b * a.dk.s0 + hk * a.dk.s1;
  T *dvb = mut<T>(a.dv) + b * a.dv.s0 + hk * a.dv.s1;
#pragma unroll
  for (int u = 0; u < KB * CPR / NTK; ++u) {
    const int idx = u * NTK + tid, row = idx / CPR, q = idx % CPR;
    const int key_r = k0 + row;
    if (key_r >= p.Sk) continue;
    const int rr = row % 32, src = (row / 32) * SLICE_B + rr * 2 * D + ((q ^ (rr % CPR)) * 16);
    const u32x4 vk = *reinterpret_cast<const u32x4 *>(ring + src);
    const u32x4 vv = *reinterpret_cast<const u32x4 *>(kv_lds + src);
    *reinterpret_cast<u32x4 *>(dkb + static_cast<int64_t>(key_r) * a.dk.s2 + q * 8) = vk;
    *reinterpret_cast<u32x4 *>(dvb + static_cast<int64_t>(key_r) * a.dv.s2 + q * 8) = vv;
  }
}

// ---------------------------------------------------------------------------
// dQ: one workgroup = 128 query rows of one (b, q head), 4 waves x 32 rows,
// two workgroups per CU; a wave keeps its Q and dO rows as B operands in
// registers.  Key tiles of 32 rows stream global -> LDS by DMA loads into a
// 4-stage ring (issued two tiles ahead, blocked layout), one fence-free
// barrier per tile.  Per tile j a wave runs one MFMA block -- S_j^T = K Q^T
// and dP_j^T = V dO^T from row fragments, fused with dQ^T += K_{j-1}^T
// dS_{j-1}^T from column fragments of the previous K tile -- then forms
// P = exp2(S sl - lse2) and dS = P (dP - delta) on the VALU.
// ---------------------------------------------------------------------------
constexpr int QB = 128;  // query rows per workgroup
constexpr int KT = 32;   // keys per tile
constexpr int DQ_PD = 2;              // tiles issued ahead
constexpr int DQ_NS = DQ_PD + 2;      // ring stages: tile j is read in iterations j and j + 1

template <typename T, int D>
__global__ __launch_bounds__(NT, 2) void dq_kernel(BwdArgs a) {
  constexpr int TILE_B = KT * D * 2;   // bytes per K (or V) tile
  constexpr int NBLK = TILE_B / 1024;  // 1 KiB blocks per tile
  constexpr int LPT = 2 * NBLK / NW;   // DMA loads per wave per K+V tile
  constexpr int SKS = D / 16, PDT = D / 32, QG = D / 32;
  static_assert(LPT >= 1 && LPT * NW == 2 * NBLK, "tile loads must split evenly over the waves");
  static_assert(SKS == 2 * PDT, "one dQ MFMA per step");
  __shared__ __attribute__((aligned(1024))) char lds[DQ_NS * 2 * TILE_B];  // [stage][K | V]

  const Problem &p = a.p;
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 31, h = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_qb = (p.Sq + QB - 1) / QB;
  const int total = n_qb * p.Hq * p.B;
  const int logical = xcd_remap(blockIdx.x, total);
  int bh, rank;
  heavy_first(logical, n_qb, p.Hq * p.B, 64, bh, rank);  // 2 WG per CU
  const int qb = n_qb - 1 - rank;  // long causal rows first
  const int b = bh / p.Hq, hq = bh - b * p.Hq, hk = hq / p.rep;
  const int q0 = qb * QB, qw = q0 + 32 * w, qrow = qw + c;
  const int kv_end = kv_end_for(p, b);
  const bool keymask = p.mask.kind == TSATTN_MASK_BOOL && !(p.kv_prefix && p.kv_prefix[b]);
  const bool causal = p.causal != 0;

  int64_t lim = kv_end, wlim = kv_end;
  if (causal) {
    lim = min(lim, static_cast<int64_t>(min(q0 + QB, p.Sq) - 1) + p.offset + 1);
    wlim = min(wlim, static_cast<int64_t>(min(qw + 32, p.Sq) - 1) + p.offset + 1);
  }
  if (qw >= p.Sq) wlim = 0;
  const int n_tiles = lim > 0 ? static_cast<int>((lim + KT - 1) / KT) : 0;
  const int w_tiles = wlim > 0 ? static_cast<int>((wlim + KT - 1) / KT) : 0;

  u32x4 qf[SKS], gf[SKS];
  float lse2, delta;
  {
    const uint32_t qs_b = static_cast<uint32_t>(a.q.s2) * 2, gs_b = static_cast<uint32_t>(a.dout.s2) * 2;
    const rsrc_t qrs = make_rsrc(head_ptr<T>(a.q, b, hq), static_cast<uint32_t>(p.Sq) * qs_b);
    const rsrc_t grs = make_rsrc(head_ptr<T>(a.dout, b, hq), static_cast<uint32_t>(p.Sq) * gs_b);
#pragma unroll
    for (int ks = 0; ks < SKS; ++ks) {
      qf[ks] = buf_load16(qrs, static_cast<uint32_t>(qrow) * qs_b + (ks * 16 + h * 8) * 2);
      gf[ks] = buf_load16(grs, static_cast<uint32_t>(qrow) * gs_b + (ks * 16 + h * 8) * 2);
    }
    const int64_t rows = static_cast<int64_t>(p.B) * p.Hq * p.Sq;
    const int64_t base = (static_cast<int64_t>(b) * p.Hq + hq) * p.Sq;
    const rsrc_t drs = make_rsrc(a.delta + base, static_cast<uint32_t>(p.Sq) * 4);
    const rsrc_t lrs = make_rsrc(a.delta + rows + base, static_cast<uint32_t>(p.Sq) * 4);
    delta = buf_load_f32(drs, static_cast<uint32_t>(qrow) * 4);
    lse2 = buf_load_f32(lrs, static_cast<uint32_t>(qrow) * 4);
  }
  // Resolve these loads before the DMA loads start (the compiler's vmcnt
  // waits do not count those).
#pragma unroll
  for (int ks = 0; ks < SKS; ++ks) asm volatile("" : "+v"(qf[ks]), "+v"(gf[ks]));
  asm volatile("" : "+v"(delta), "+v"(lse2));

  const uint32_t ks_b = static_cast<uint32_t>(a.k.s2) * 2, vs_b = static_cast<uint32_t>(a.v.s2) * 2;
  const u32x4 kdesc = make_desc(head_ptr<T>(a.k, b, hk), static_cast<uint32_t>(kv_end) * ks_b);
  const u32x4 vdesc = make_desc(head_ptr<T>(a.v, b, hk), static_cast<uint32_t>(kv_end) * vs_b);
  const uint32_t lds0 = lds_addr(lds);
  // Wave w loads blocks e = w, w + 4, ... of the tile (K blocks first, then V):
  // block n = (n / QG, n % QG), lane l fetches row 16 (n / QG) + l / 4, chunk
  // 4 (n % QG) + ((l % 4) ^ ((l / 16) % 4)); n % QG = w % QG for all of them.
  const uint32_t lane_chunk = 4 * (w % QG) + ((lane & 3) ^ ((lane >> 4) & 3));
  const uint32_t koff = (lane >> 2) * ks_b + lane_chunk * 16;
  const uint32_t voff = (lane >> 2) * vs_b + lane_chunk * 16;
  auto issue = [&](int tile) {
    const uint32_t st = lds0 + (tile % DQ_NS) * 2 * TILE_B;
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int e = w + NW * u;
      const int n = e < NBLK ? e : e - NBLK;
      const uint32_t row0 = static_cast<uint32_t>(tile * KT + 16 * (n / QG));
      if (e < NBLK) dma16(kdesc, st + n * 1024, koff, row0 * ks_b);
      else dma16(vdesc, st + TILE_B + n * 1024, voff, row0 * vs_b);
    }
  };
  auto in_flight_after = [&](int jn) {
    const int later = min(DQ_PD - 1, n_tiles - 1 - jn);
    return later > 0 ? later * LPT : 0;
  };

  const TileReader<T, D> rd(lane);
  f32x16 acc[PDT];
#pragma unroll
  for (int dt = 0; dt < PDT; ++dt) acc[dt] = f32x16{};
  f32x16 s = f32x16{}, dp = f32x16{};
  u32x4 pd[2];  // dS^T of the previous tile, packed: B operands of its 2 k-steps
  const float sl = a.sl;
  int klim = kv_end;
  if (causal) {
    const int64_t cl = static_cast<int64_t>(qrow) + p.offset + 1;
    if (cl < kv_end) klim = cl < 0 ? 0 : static_cast<int>(cl);
  }
  const uint8_t *kmask_b =
      keymask ? static_cast<const uint8_t *>(p.mask.data) + b * p.mask.s0 : nullptr;

  zero_lds<NT>(lds, sizeof(lds), tid);
  __syncthreads();
  for (int t = 0; t < DQ_PD && t < n_tiles; ++t) issue(t);
  wait_vm(in_flight_after(0));
  __syncthreads();

  // MFMA block of tile j: S_j^T, dP_j^T (k-step i each) and dQ MFMA i of the
  // previous tile (value block i % PDT, key k-step i / PDT); fragments two
  // steps ahead.  One code path for every block keeps the accumulators in
  // place: the first block multiplies a zeroed stage by dS = 0, and past the
  // wave's last tile S and dP are computed and ignored.
  auto mfma_block = [&](int j) {
    const char *kt = lds + (j % DQ_NS) * 2 * TILE_B;
    const char *vt = kt + TILE_B;
    const char *kp = lds + ((j + DQ_NS - 1) % DQ_NS) * 2 * TILE_B;
    constexpr int FD = 2;
    u32x4 kr[FD + 1], vr[FD + 1], kc[FD + 1];
    auto load = [&](int i) {
      kr[i % (FD + 1)] = rd.rows(kt, 0, i);
      vr[i % (FD + 1)] = rd.rows(vt, 0, i);
      kc[i % (FD + 1)] = rd.cols(kp, i / PDT, i % PDT);
    };
    s = f32x16{};
    dp = f32x16{};
#pragma unroll
    for (int i = 0; i < FD; ++i) load(i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < SKS; ++i) {
      s = mfma32<T>(kr[i % (FD + 1)], qf[i], s);
      dp = mfma32<T>(vr[i % (FD + 1)], gf[i], dp);
      acc[i % PDT] = mfma32<T>(kc[i % (FD + 1)], pd[i / PDT], acc[i % PDT]);
      if (i + FD < SKS) load(i + FD);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  auto grad = [&](int j) {
    const int kv0 = j * KT;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = s[i];
    const bool edge = (kv0 + KT > kv_end) || keymask ||
                      (causal && static_cast<int64_t>(kv0 + KT - 1) > qw + p.offset);
    if (edge) {
      const int lim_l = klim - kv0 - 4 * h;
      unsigned kbits = ~0u;
      if (keymask) {
        const int key = kv0 + lane;
        const bool ok = key < p.Sk && kmask_b[static_cast<int64_t>(key) * p.mask.s3];
        kbits = static_cast<unsigned>(__ballot(ok) >> (4 * h));
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int kc = 8 * (i >> 2) + (i & 3);
        const bool ok = (kc < lim_l) & (((kbits >> kc) & 1u) != 0);
        x[i] = ok ? x[i] : -INFINITY;
      }
    }
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      const float p0 = fast_exp2(fmaf(x[i], sl, -lse2));
      const float p1 = fast_exp2(fmaf(x[i + 1], sl, -lse2));
      pd[i >> 3][(i & 7) >> 1] = pack2<T>(p0 * (dp[i] - delta), p1 * (dp[i + 1] - delta));
    }
  };

  auto it_begin = [&](int j) {
    if (j + DQ_PD < n_tiles) issue(j + DQ_PD);
  };
  auto it_end = [&](int j) {
    wait_vm(in_flight_after(j + 1));
    wait_lgkm0();
    phase_barrier();
  };
  int j = 0;
  if (w_tiles > 0) {
    pd[0] = pd[1] = u32x4{0, 0, 0, 0};
    for (; j < w_tiles; ++j) {
      it_begin(j);
      mfma_block(j);
      grad(j);
      it_end(j);
    }
    it_begin(j);
    mfma_block(j);  // dQ of the last tile
    it_end(j);
    ++j;
  }
  for (; j <= n_tiles; ++j) {
    it_begin(j);
    it_end(j);
  }

  if (qrow >= p.Sq) return;
  T *dqp = mut<T>(a.dq) + b * a.dq.s0 + hq * a.dq.s1 + static_cast<int64_t>(qrow) * a.dq.s2;
  const float sc = a.scale;
#pragma unroll
  for (int dt = 0; dt < PDT; ++dt) {
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
  { Probe pr_("bwd_row_prep", st); row_prep_kernel<T, D><<<dim3((rows + RPB - 1) / RPB), dim3(NT), 0, st>>>(a); }
  const int n_kb = (p.Sk + KB - 1) / KB;
  { Probe pr_("bwd_dkdv_mfma", st); dkdv_kernel<T, D><<<dim3(n_kb * p.Hkv * p.B), dim3(NTK), 0, st>>>(a); }
  const int n_qb = (p.Sq + QB - 1) / QB;
  { Probe pr_("bwd_dq_mfma", st); dq_kernel<T, D><<<dim3(n_qb * p.Hq * p.B), dim3(NT), 0, st>>>(a); }
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
