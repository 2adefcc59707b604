// fp32 attention on the fp32 matrix cores (v_mfma_f32_32x32x2_f32): forward,
// backward row values, dQ and dK/dV, for fp32 q / k / v with Dqk = Dv in
// {32, 64, 128}, causal windows with offsets, key-padding lengths and GQA.
// The reference keeps fp32 inputs in fp32 (src/tensorsmith/nn/attention.py:63)
// and fp32 is its default dtype; these kernels follow the same streaming
// algorithm as the 16-bit ones (attention.py:175-198 forward, :200-247 VJP),
// with every product and accumulation in fp32 (P and dS stay fp32: nothing is
// rounded to a narrower type).
//
// MFMA 32x32x2 f32, lane l = 32 h + c: A[m = c][k = h], B[k = h][n = c], C as
// in mfma_common.h.  A contraction over K elements runs K / 2 MFMAs; lane half
// h supplies element k = perm(s, h) of step s, any bijection shared by both
// operands.  Over a head dimension the kernels take d = h D / 2 + s, so each
// lane walks a contiguous half of every row (16-byte LDS reads serve four
// steps); over a 32-row tile of an accumulator layout they take the row
// crow(i, h) of register i, so a C tile feeds the next contraction as it is.
//
// LDS tiles hold 32 rows x D floats, row-major, 16-byte chunk q of row r at
// q ^ fsw(r): 16 lanes reading one chunk each of 16 consecutive rows hit 16
// different bank groups (the operands whose rows are lanes), and 64 lanes
// reading a 32-float segment of rows r and r + 4 (the operands whose rows are
// accumulator rows) hit the two halves of the banks (D >= 64; at D = 32 a row
// is half the banks and the segment reads take two passes).  Tiles reach LDS
// by direct buffer loads (DMA), each lane fetching the global chunk its
// swizzled position holds; rows past the buffer range arrive as zeros.
#include "mfma_common.h"

namespace tsattn {
namespace {

constexpr int NT = 256;
constexpr int NW = NT / 64;
constexpr int BM = 128;  // query rows per forward / dQ workgroup
constexpr int BN = 32;   // keys (forward, dQ) or query rows (dK/dV) per tile
constexpr int KB = 128;  // keys per dK/dV workgroup
constexpr float kTau = 8.f;

__device__ __forceinline__ f32x16 mfma32f(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <int D>
__host__ __device__ __forceinline__ constexpr int fsw(int r) {
  return D >= 64 ? ((r & 3) | ((r & 4) << 1) | ((r & 8) >> 1)) : ((r >> 1) & 7);
}

template <typename X>
__device__ __forceinline__ const X *f32_head(View v, int b, int h) {
  return static_cast<const X *>(v.data) + b * v.s0 + h * v.s1;
}

// A [32 x D] fp32 tile in LDS (see the layout above).
template <int D>
struct FTile {
  static constexpr int CPR = D / 4;                  // 16-byte chunks per row
  static constexpr int BYTES = BN * D * 4;           // per tile
  static constexpr int BLOCKS = BYTES / 1024;        // 1 KiB DMA blocks per tile
  static constexpr int RPB = 1024 / (D * 4);         // rows per DMA block

  // Byte offset (within the block's rows) of the global chunk lane l of a
  // DMA of block n fetches: its LDS slot is 16 l of the block.
  __device__ __forceinline__ static uint32_t dma_off(int n, int lane, uint32_t stride_b) {
    const int rr = lane / CPR, p = lane % CPR, row = n * RPB + rr;
    return static_cast<uint32_t>(rr) * stride_b + static_cast<uint32_t>((p ^ fsw<D>(row)) * 16);
  }
  // 16 bytes of row r, chunk q (d = 4 q .. 4 q + 3).
  __device__ __forceinline__ static float4 chunk(const char *t, int r, int q) {
    return *reinterpret_cast<const float4 *>(t + r * D * 4 + ((q ^ fsw<D>(r)) << 4));
  }
  // One float: row r, column d.
  __device__ __forceinline__ static float elem(const char *t, int r, int d) {
    return *reinterpret_cast<const float *>(t + r * D * 4 + (((d >> 2) ^ fsw<D>(r)) << 4) + ((d & 3) << 2));
  }
};

// Compute units of the current device (cached per device).
int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    int n = 0;
    cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cus[dev];
}

struct F32Args {
  Problem p;
  View q, k, v, o, dout, dq, dk, dv;
  float *lse;
  float *rows;  // backward row values: [rows] -delta, then [rows] -safe(lse) / scale
  float sl;     // scale * log2(e)
  float scale;
};

// ---------------------------------------------------------------------------
// Forward: one workgroup = 128 query rows of one (b, q head), 4 waves x 32
// rows; key tiles of 32 keys double-buffered through LDS (the next tile's DMA
// issued at the start of an iteration, between the S steps).  Per tile a wave
// computes S^T = K Q^T (D / 2 MFMAs, Q in registers, K by 16-byte chunks),
// the online softmax on its lane's query column (lazy rescale, exp2 domain),
// and O^T += V^T P^T (D / 2 MFMAs, V by 32-float row segments, P^T the fp32
// accumulator registers).  Two workgroups per CU.
//
// SPLIT (problems with fewer 128-row workgroups than CUs, D <= 64): one
// workgroup = 32 query rows, all 4 waves on them; wave w takes key tiles w,
// w + 4, ... through its own double-buffered LDS ring (no barrier in the
// loop), and the waves' (max, sum, O) merge through LDS at the end as the
// online softmax merges tiles: the key loop of a row block runs 4 ways
// parallel.  One workgroup per CU.
// ---------------------------------------------------------------------------
template <int D, bool SPLIT>
__global__ __launch_bounds__(NT, SPLIT ? 1 : 2) void fwd_f32_kernel(F32Args a) {
  using TL = FTile<D>;
  constexpr int HD = D / 2;             // MFMA steps over the head dimension
  constexpr int PDT = D / 32;           // 32-row blocks of O^T
  constexpr int STAGE = 2 * TL::BYTES;  // K | V
  constexpr int ROWS = SPLIT ? 32 : BM;  // query rows per workgroup
  constexpr int RINGS = SPLIT ? NW : 1;  // double-buffered rings (one per wave when split)
  constexpr int STRIDE = SPLIT ? NW : 1;  // tiles between a wave's consecutive tiles
  // DMA blocks per wave per tile: a wave loads its whole tile when split
  constexpr int PARTS = SPLIT ? 2 * TL::BLOCKS : 2 * TL::BLOCKS / NW;
  static_assert(SPLIT || (PARTS * NW == 2 * TL::BLOCKS && PARTS >= 1), "tile loads split over the waves");
  static_assert(PARTS <= 2 * (HD / 4), "at most two DMA parts per S step");
  // the rings, then a 1 KiB block the parts of a tile past the last land in
  // (split: then the workgroup's 32 Q rows, staged once for the four waves)
  constexpr int QSTG = SPLIT ? TL::BYTES : 0;
  __shared__ __attribute__((aligned(1024))) char lds[RINGS * 2 * STAGE + 1024 + QSTG];

  const Problem &p = a.p;
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 31, h = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_qb = (p.Sq + ROWS - 1) / ROWS;
  const int total = n_qb * p.Hq * p.B;
  const int logical = xcd_remap(blockIdx.x, total);
  int bh, rank;
  heavy_first(logical, n_qb, p.Hq * p.B, SPLIT ? 32 : 64, bh, rank);
  const int qb = n_qb - 1 - rank;
  const int b = bh / p.Hq, hq = bh - b * p.Hq, hk = hq / p.rep;
  const int q0 = qb * ROWS, qw = SPLIT ? q0 : q0 + 32 * w, qrow = qw + c;
  const int kv_end = kv_end_for(p, b);
  const bool keymask = p.mask.kind == TSATTN_MASK_BOOL && !(p.kv_prefix && p.kv_prefix[b]);

  int64_t lim = kv_end, wlim = kv_end;
  if (p.causal) {
    lim = min(lim, static_cast<int64_t>(min(q0 + ROWS, p.Sq) - 1) + p.offset + 1);
    wlim = min(wlim, static_cast<int64_t>(min(qw + 32, p.Sq) - 1) + p.offset + 1);
  }
  if (qw >= p.Sq) wlim = 0;
  const int n_tiles = __builtin_amdgcn_readfirstlane(lim > 0 ? static_cast<int>((lim + BN - 1) / BN) : 0);
  const int w_tiles = __builtin_amdgcn_readfirstlane(wlim > 0 ? static_cast<int>((wlim + BN - 1) / BN) : 0);
  // this wave's tiles: j = first + STRIDE jj, jj < my_tiles
  const int first = SPLIT ? w : 0;
  const int my_tiles = SPLIT ? (n_tiles > w ? (n_tiles - 1 - w) / NW + 1 : 0) : n_tiles;

  const uint32_t qs_b = static_cast<uint32_t>(a.q.s2) * 4;
  const uint32_t ks_b = static_cast<uint32_t>(a.k.s2) * 4;
  const uint32_t vs_b = static_cast<uint32_t>(a.v.s2) * 4;
  const rsrc_t qrs = make_rsrc(f32_head<float>(a.q, b, hq), static_cast<uint32_t>(p.Sq) * qs_b);
  const u32x4 kdesc = make_desc(f32_head<float>(a.k, b, hk), static_cast<uint32_t>(kv_end) * ks_b);
  const u32x4 vdesc = make_desc(f32_head<float>(a.v, b, hk), static_cast<uint32_t>(kv_end) * vs_b);

  // Q fragments: lane (c, h) holds Q[qrow][h D / 2 .. + D / 2), step s = d - h D / 2.
  // Split: the four waves share the 32 rows, which land in LDS once by DMA
  // (whole lines per instruction) beside the first tile and are read from
  // there; fragment loads straight into registers touch 64 lines each.
  float qf[HD];
  if constexpr (!SPLIT) {
#pragma unroll
    for (int j = 0; j < HD / 4; ++j) {
      const float4 x = __builtin_bit_cast(float4, buf_load16(qrs, static_cast<uint32_t>(qrow) * qs_b +
                                                                      static_cast<uint32_t>((h * HD + 4 * j) * 4)));
      qf[4 * j] = x.x, qf[4 * j + 1] = x.y, qf[4 * j + 2] = x.z, qf[4 * j + 3] = x.w;
    }
  } else {
    static_assert(TL::BLOCKS % NW == 0, "Q blocks split evenly over the waves");
    const u32x4 qd = make_desc(f32_head<float>(a.q, b, hq), static_cast<uint32_t>(p.Sq) * qs_b);
    const uint32_t qst = lds_addr(lds) + RINGS * 2 * STAGE + 1024;
#pragma unroll
    for (int u = 0; u < TL::BLOCKS / NW; ++u) {
      const int n = w + NW * u;
      dma16(qd, qst + n * 1024, TL::dma_off(n, lane, qs_b), static_cast<uint32_t>(q0 + n * TL::RPB) * qs_b);
    }
  }

  const uint32_t lds0 = lds_addr(lds);
  const uint32_t ring = lds0 + (SPLIT ? w * 2 * STAGE : 0);
  const char *ring_p = lds + (SPLIT ? w * 2 * STAGE : 0);
  const uint32_t spare = lds0 + RINGS * 2 * STAGE;
  // Part u of this wave's share of local tile jj (tile first + STRIDE jj):
  // block n = w + NW u of the stage (split: n = u), K blocks first.  A tile
  // past the last one reads past the buffer ranges (zeros, no memory access)
  // into the spare block, so every wave issues the same parts.
  auto issue_part = [&](int jj, int u) {
    const int n = SPLIT ? u : w + NW * u;
    const int tile = first + STRIDE * jj;
    const bool real = tile < n_tiles;
    const uint32_t st = real ? ring + (jj & 1) * STAGE : spare;
    if (n < TL::BLOCKS) {
      const uint32_t so = real ? static_cast<uint32_t>(tile * BN + n * TL::RPB) * ks_b : 0x80000000u;
      dma16(kdesc, st + (real ? n * 1024 : 0), TL::dma_off(n, lane, ks_b), so);
    } else {
      const int m = n - TL::BLOCKS;
      const uint32_t so = real ? static_cast<uint32_t>(tile * BN + m * TL::RPB) * vs_b : 0x80000000u;
      dma16(vdesc, st + (real ? TL::BYTES + m * 1024 : 0), TL::dma_off(m, lane, vs_b), so);
    }
  };

  f32x16 oacc[PDT];
#pragma unroll
  for (int dt = 0; dt < PDT; ++dt) oacc[dt] = f32x16{};
  float m = -INFINITY, l = 0.f, thr = -INFINITY, nbase = 0.f;
  const float sl = a.sl, inv_sl = 1.f / sl;
  int klim = kv_end;
  if (p.causal) {
    const int64_t cl = static_cast<int64_t>(qrow) + p.offset + 1;
    if (cl < kv_end) klim = cl < 0 ? 0 : static_cast<int>(cl);
  }
  const uint8_t *kmask_b = keymask ? static_cast<const uint8_t *>(p.mask.data) + b * p.mask.s0 : nullptr;
  int j_edge = kv_end / BN;
  if (keymask) j_edge = 0;
  if (p.causal) {
    const int64_t dd = static_cast<int64_t>(qw) + p.offset - (BN - 1);
    const int jc = dd < 0 ? 0 : static_cast<int>(min(dd / BN + 1, static_cast<int64_t>(INT32_MAX)));
    j_edge = min(j_edge, jc);
  }

#pragma unroll
  for (int u = 0; u < PARTS; ++u) issue_part(0, u);
  wait_vm_n<0>();  // the query fragments and the first tile
  if constexpr (SPLIT) {
    __syncthreads();  // every wave's Q blocks landed
    const char *qt = lds + RINGS * 2 * STAGE + 1024;
#pragma unroll
    for (int j = 0; j < HD / 4; ++j) {
      const float4 x = TL::chunk(qt, c, h * (HD / 4) + j);
      qf[4 * j] = x.x, qf[4 * j + 1] = x.y, qf[4 * j + 2] = x.z, qf[4 * j + 3] = x.w;
    }
  }
#pragma unroll
  for (int i = 0; i < HD; ++i) asm volatile("" : "+v"(qf[i]));
  if constexpr (!SPLIT) __syncthreads();

  for (int jj = 0; jj < my_tiles; ++jj) {
    const int j = first + STRIDE * jj;
    const char *kt = ring_p + (jj & 1) * STAGE;
    const char *vt = kt + TL::BYTES;
    if (SPLIT || j < w_tiles) {
      // S^T = K Q^T, the next tile's parts spread over the steps; each
      // 16-byte chunk of K serves four steps, read one chunk ahead
      f32x16 s = f32x16{};
      {
        constexpr int NC = HD / 4;
        float4 kc[2];
        kc[0] = TL::chunk(kt, c, h * NC);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < NC; ++q) {
          if (q + 1 < NC) kc[(q + 1) & 1] = TL::chunk(kt, c, h * NC + q + 1);
          const float4 kv = kc[q & 1];
          s = mfma32f(kv.x, qf[4 * q], s);
          s = mfma32f(kv.y, qf[4 * q + 1], s);
          s = mfma32f(kv.z, qf[4 * q + 2], s);
          s = mfma32f(kv.w, qf[4 * q + 3], s);
          if (2 * q < PARTS && PARTS > NC) issue_part(jj + 1, 2 * q);
          if (2 * q + 1 < PARTS && PARTS > NC) issue_part(jj + 1, 2 * q + 1);
          if (q < PARTS && PARTS <= NC) issue_part(jj + 1, q);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      // softmax of this lane's query column: element i is key kv0 + crow(i, h)
      const int kv0 = j * BN;
      if (j >= j_edge) {
        const int lm = klim - kv0 - 4 * h;
        unsigned kbits = ~0u;
        if (keymask) {
          const int key = kv0 + lane;
          const bool ok = key < p.Sk && kmask_b[static_cast<int64_t>(key) * p.mask.s3];
          kbits = static_cast<unsigned>(__ballot(ok) >> (4 * h));
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kc_ = 8 * (i >> 2) + (i & 3);
          s[i] = ((kc_ < lm) & (((kbits >> kc_) & 1u) != 0)) ? s[i] : -INFINITY;
        }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[i]);
      const float mxr = half_swap_max3(mx);
      if (__ballot(mxr > thr) != 0ull) {
        const float m_new = fmaxf(m, mxr * sl);
        const float corr = m_new == -INFINITY ? 1.f : fast_exp2(m - m_new);
        m = m_new;
        thr = (m + kTau) * inv_sl;
        nbase = m == -INFINITY ? 0.f : -m;
        l *= corr;
#pragma unroll
        for (int dt = 0; dt < PDT; ++dt) oacc[dt] *= corr;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        s[i] = fast_exp2(fmaf(s[i], sl, nbase));
        l += s[i];
      }
      // O^T += V^T P^T: step i takes keys crow(i, h) (register i of P^T); the
      // V elements read two steps ahead
      {
        constexpr int NS_ = 16 * PDT, FD = 2;
        float vf[FD + 1];
        auto vload = [&](int t) {
          const int i = t / PDT, dt = t % PDT;
          vf[t % (FD + 1)] = TL::elem(vt, 8 * (i >> 2) + 4 * h + (i & 3), 32 * dt + c);
        };
#pragma unroll
        for (int t = 0; t < FD; ++t) vload(t);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < NS_; ++t) {
          if (t + FD < NS_) vload(t + FD);
          oacc[t % PDT] = mfma32f(vf[t % (FD + 1)], s[t / PDT], oacc[t % PDT]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < PARTS; ++u) issue_part(jj + 1, u);
    }
    wait_vm_n<0>();  // tile jj + 1 has landed
    if constexpr (SPLIT) {
      // this wave's ring only: its LDS reads of the stage the next DMA
      // overwrites are done once they have returned
      wait_lgkm0();
    } else {
      __syncthreads();
    }
  }

  // O rows: lane holds O^T[d = 32 dt + 8 g + 4 h + r][row c], four consecutive
  // channels per (dt, g): one 16-byte store each.
  float *orow = static_cast<float *>(const_cast<void *>(a.o.data)) + b * a.o.s0 + hq * a.o.s1 +
                static_cast<int64_t>(qrow < p.Sq ? qrow : 0) * a.o.s2;
  const float lt = xor32_sum(l);
  if constexpr (!SPLIT) {
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    if (qrow < p.Sq) {
#pragma unroll
      for (int dt = 0; dt < PDT; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<float4 *>(orow + 32 * dt + 8 * g + 4 * h) =
              float4{oacc[dt][4 * g] * inv, oacc[dt][4 * g + 1] * inv, oacc[dt][4 * g + 2] * inv,
                     oacc[dt][4 * g + 3] * inv};
      if (a.lse && h == 0)
        a.lse[(static_cast<int64_t>(b) * p.Hq + hq) * p.Sq + qrow] =
            lt > 0.f ? (m + log2f(lt)) * kLn2 : -INFINITY;
    }
  } else {
    // Merge the waves' partial rows: max mf = max_w m_w, sum L = sum_w l_w
    // 2^(m_w - mf), O = sum_w O_w 2^(m_w - mf) / L, in wave order.  Wave w
    // stores the (dt, g) groups w, w + 4, ...
    wait_vm_n<0>();
    __syncthreads();  // every wave's loop is done (and its past-the-end loads landed)
    float *cm = reinterpret_cast<float *>(lds);  // [NW][32] maxima
    float *cl = cm + NW * 32;                     // [NW][32] sums
    float *co = cl + NW * 32;                     // [NW][PDT][16][64] O^T registers
    if (h == 0) {
      cm[w * 32 + c] = m;
      cl[w * 32 + c] = lt;
    }
#pragma unroll
    for (int dt = 0; dt < PDT; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) co[((w * PDT + dt) * 16 + i) * 64 + lane] = oacc[dt][i];
    __syncthreads();
    float mf = -INFINITY;
#pragma unroll
    for (int v = 0; v < NW; ++v) mf = fmaxf(mf, cm[v * 32 + c]);
    float sc[NW], lsum = 0.f;
#pragma unroll
    for (int v = 0; v < NW; ++v) {
      const float mv = cm[v * 32 + c];
      sc[v] = mv == -INFINITY ? 0.f : fast_exp2(mv - mf);
      lsum += cl[v * 32 + c] * sc[v];
    }
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    if (qrow < p.Sq) {
      for (int grp = w; grp < PDT * 4; grp += NW) {
        const int dt = grp >> 2, g = grp & 3;
        float o4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int v = 0; v < NW; ++v)
#pragma unroll
          for (int r = 0; r < 4; ++r) o4[r] = fmaf(co[((v * PDT + dt) * 16 + 4 * g + r) * 64 + lane], sc[v], o4[r]);
        *reinterpret_cast<float4 *>(orow + 32 * dt + 8 * g + 4 * h) =
            float4{o4[0] * inv, o4[1] * inv, o4[2] * inv, o4[3] * inv};
      }
      if (a.lse && w == 0 && h == 0)
        a.lse[(static_cast<int64_t>(b) * p.Hq + hq) * p.Sq + qrow] =
            lsum > 0.f ? (mf + log2f(lsum)) * kLn2 : -INFINITY;
    }
  }
}

// ---------------------------------------------------------------------------
// Backward row values: nd = -delta (delta = sum_d dO O, attention.py:232) and
// nl = -safe(lse) / scale (safe: 0 for a row that sees no key, :231), the
// layout the 16-bit kernels use: P = exp2((S + nl) sl), dS = P (dP + nd).  A
// row is D / 4 lanes of 16 bytes.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(NT) void rows_f32_kernel(F32Args a) {
  constexpr int G = D / 4, RPW = 64 / G;
  const Problem &p = a.p;
  const int64_t rows = static_cast<int64_t>(p.B) * p.Hq * p.Sq;
  const int lane = threadIdx.x & 63, g = lane % G;
  const int64_t row = (static_cast<int64_t>(blockIdx.x) * NW + (threadIdx.x >> 6)) * RPW + lane / G;
  const bool live = row < rows;
  const int64_t rr = live ? row : rows - 1;
  const int64_t bh = rr / p.Sq, i = rr - bh * p.Sq, b = bh / p.Hq, hq = bh - b * p.Hq;
  const float *go = static_cast<const float *>(a.dout.data) + b * a.dout.s0 + hq * a.dout.s1 + i * a.dout.s2;
  const float *oo = static_cast<const float *>(a.o.data) + b * a.o.s0 + hq * a.o.s1 + i * a.o.s2;
  const float4 x = *reinterpret_cast<const float4 *>(go + 4 * g);
  const float4 y = *reinterpret_cast<const float4 *>(oo + 4 * g);
  float d = x.x * y.x + x.y * y.y + x.z * y.z + x.w * y.w;
#pragma unroll
  for (int o = 1; o < G; o <<= 1) d += __shfl_xor(d, o, 64);
  if (live && g == 0) {
    const float lse = a.lse[rr];
    a.rows[rr] = -d;
    a.rows[rows + rr] = isfinite(lse) ? -lse / a.scale : 0.f;
  }
}

// ---------------------------------------------------------------------------
// dQ: one workgroup = 128 query rows of one (b, q head), 4 waves x 32 rows,
// one workgroup per CU (a wave holds Q, dO and the dQ accumulators).  Key
// tiles double-buffered through LDS as in the forward.  Per tile a wave
// computes S^T = K Q^T and dP^T = V dO^T (K, V by 16-byte chunks; Q, dO in
// registers), P = exp2((S + nl) sl) and dS = P (dP + nd) on its lane's query
// column, then dQ^T += K^T dS^T (K by 32-float row segments, dS^T the
// accumulator registers).  dQ = scale dQ^T^T.
//
// SPLIT (as the forward's): one workgroup = 32 query rows, wave w takes key
// tiles w, w + 4, ... through its own ring, and the waves' dQ^T partial sums
// add up through LDS in wave order at the end.
// ---------------------------------------------------------------------------
template <int D, bool SPLIT>
__global__ __launch_bounds__(NT, 1) void dq_f32_kernel(F32Args a) {
  using TL = FTile<D>;
  constexpr int HD = D / 2, PDT = D / 32;
  constexpr int STAGE = 2 * TL::BYTES;  // K | V
  constexpr int ROWS = SPLIT ? 32 : BM;
  constexpr int RINGS = SPLIT ? NW : 1, STRIDE = SPLIT ? NW : 1;
  constexpr int PARTS = SPLIT ? 2 * TL::BLOCKS : 2 * TL::BLOCKS / NW;
  static_assert(SPLIT || (PARTS * NW == 2 * TL::BLOCKS && PARTS >= 1), "tile loads split over the waves");
  static_assert(PARTS <= 2 * (HD / 4), "at most two DMA parts per S step");
  // (split: after the rings and the spare block, the workgroup's 32 Q and 32
  // dO rows, staged once for the four waves)
  constexpr int QSTG = SPLIT ? 2 * TL::BYTES : 0;
  __shared__ __attribute__((aligned(1024))) char lds[RINGS * 2 * STAGE + 1024 + QSTG];

  const Problem &p = a.p;
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 31, h = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_qb = (p.Sq + ROWS - 1) / ROWS;
  const int total = n_qb * p.Hq * p.B;
  const int logical = xcd_remap(blockIdx.x, total);
  int bh, rank;
  heavy_first(logical, n_qb, p.Hq * p.B, 32, bh, rank);
  const int qb = n_qb - 1 - rank;
  const int b = bh / p.Hq, hq = bh - b * p.Hq, hk = hq / p.rep;
  const int q0 = qb * ROWS, qw = SPLIT ? q0 : q0 + 32 * w, qrow = qw + c;
  const int kv_end = kv_end_for(p, b);
  const bool keymask = p.mask.kind == TSATTN_MASK_BOOL && !(p.kv_prefix && p.kv_prefix[b]);
  int64_t lim = kv_end, wlim = kv_end;
  if (p.causal) {
    lim = min(lim, static_cast<int64_t>(min(q0 + ROWS, p.Sq) - 1) + p.offset + 1);
    wlim = min(wlim, static_cast<int64_t>(min(qw + 32, p.Sq) - 1) + p.offset + 1);
  }
  if (qw >= p.Sq) wlim = 0;
  const int n_tiles = __builtin_amdgcn_readfirstlane(lim > 0 ? static_cast<int>((lim + BN - 1) / BN) : 0);
  const int w_tiles = __builtin_amdgcn_readfirstlane(wlim > 0 ? static_cast<int>((wlim + BN - 1) / BN) : 0);
  const int first = SPLIT ? w : 0;
  const int my_tiles = SPLIT ? (n_tiles > w ? (n_tiles - 1 - w) / NW + 1 : 0) : n_tiles;

  const uint32_t qs_b = static_cast<uint32_t>(a.q.s2) * 4, gs_b = static_cast<uint32_t>(a.dout.s2) * 4;
  const uint32_t ks_b = static_cast<uint32_t>(a.k.s2) * 4, vs_b = static_cast<uint32_t>(a.v.s2) * 4;
  const rsrc_t qrs = make_rsrc(f32_head<float>(a.q, b, hq), static_cast<uint32_t>(p.Sq) * qs_b);
  const rsrc_t grs = make_rsrc(f32_head<float>(a.dout, b, hq), static_cast<uint32_t>(p.Sq) * gs_b);
  const u32x4 kdesc = make_desc(f32_head<float>(a.k, b, hk), static_cast<uint32_t>(kv_end) * ks_b);
  const u32x4 vdesc = make_desc(f32_head<float>(a.v, b, hk), static_cast<uint32_t>(kv_end) * vs_b);
  // Split: the four waves share the rows, which land in LDS once by DMA
  // beside the first tile (as in the forward) and are read from there.
  float qf[HD], gf[HD];
  if constexpr (!SPLIT) {
#pragma unroll
    for (int j = 0; j < HD / 4; ++j) {
      const uint32_t off = static_cast<uint32_t>((h * HD + 4 * j) * 4);
      const float4 x = __builtin_bit_cast(float4, buf_load16(qrs, static_cast<uint32_t>(qrow) * qs_b + off));
      const float4 y = __builtin_bit_cast(float4, buf_load16(grs, static_cast<uint32_t>(qrow) * gs_b + off));
      qf[4 * j] = x.x, qf[4 * j + 1] = x.y, qf[4 * j + 2] = x.z, qf[4 * j + 3] = x.w;
      gf[4 * j] = y.x, gf[4 * j + 1] = y.y, gf[4 * j + 2] = y.z, gf[4 * j + 3] = y.w;
    }
  } else {
    static_assert(TL::BLOCKS % NW == 0, "Q / dO blocks split evenly over the waves");
    const u32x4 qd = make_desc(f32_head<float>(a.q, b, hq), static_cast<uint32_t>(p.Sq) * qs_b);
    const u32x4 gd = make_desc(f32_head<float>(a.dout, b, hq), static_cast<uint32_t>(p.Sq) * gs_b);
    const uint32_t qst = lds_addr(lds) + RINGS * 2 * STAGE + 1024;
#pragma unroll
    for (int u = 0; u < TL::BLOCKS / NW; ++u) {
      const int n = w + NW * u;
      dma16(qd, qst + n * 1024, TL::dma_off(n, lane, qs_b), static_cast<uint32_t>(q0 + n * TL::RPB) * qs_b);
      dma16(gd, qst + TL::BYTES + n * 1024, TL::dma_off(n, lane, gs_b), static_cast<uint32_t>(q0 + n * TL::RPB) * gs_b);
    }
  }
  const int64_t rows = static_cast<int64_t>(p.B) * p.Hq * p.Sq;
  const int64_t rix = static_cast<int64_t>(bh) * p.Sq + (qrow < p.Sq ? qrow : p.Sq - 1);
  const float nd = a.rows[rix], nl = a.rows[rows + rix];

  const uint32_t lds0 = lds_addr(lds);
  const uint32_t ring = lds0 + (SPLIT ? w * 2 * STAGE : 0);
  const char *ring_p = lds + (SPLIT ? w * 2 * STAGE : 0);
  const uint32_t spare = lds0 + RINGS * 2 * STAGE;
  // part u of local tile jj (tile first + STRIDE jj), as in the forward
  auto issue_part = [&](int jj, int u) {
    const int n = SPLIT ? u : w + NW * u;
    const int tile = first + STRIDE * jj;
    const bool real = tile < n_tiles;
    const uint32_t st = real ? ring + (jj & 1) * STAGE : spare;
    if (n < TL::BLOCKS) {
      const uint32_t so = real ? static_cast<uint32_t>(tile * BN + n * TL::RPB) * ks_b : 0x80000000u;
      dma16(kdesc, st + (real ? n * 1024 : 0), TL::dma_off(n, lane, ks_b), so);
    } else {
      const int m = n - TL::BLOCKS;
      const uint32_t so = real ? static_cast<uint32_t>(tile * BN + m * TL::RPB) * vs_b : 0x80000000u;
      dma16(vdesc, st + (real ? TL::BYTES + m * 1024 : 0), TL::dma_off(m, lane, vs_b), so);
    }
  };
  int klim = kv_end;
  if (p.causal) {
    const int64_t cl = static_cast<int64_t>(qrow) + p.offset + 1;
    if (cl < kv_end) klim = cl < 0 ? 0 : static_cast<int>(cl);
  }
  const uint8_t *kmask_b = keymask ? static_cast<const uint8_t *>(p.mask.data) + b * p.mask.s0 : nullptr;
  int j_edge = kv_end / BN;
  if (keymask) j_edge = 0;
  if (p.causal) {
    const int64_t dd = static_cast<int64_t>(qw) + p.offset - (BN - 1);
    const int jc = dd < 0 ? 0 : static_cast<int>(min(dd / BN + 1, static_cast<int64_t>(INT32_MAX)));
    j_edge = min(j_edge, jc);
  }
  const float sl = a.sl;
  f32x16 acc[PDT];
#pragma unroll
  for (int dt = 0; dt < PDT; ++dt) acc[dt] = f32x16{};

#pragma unroll
  for (int u = 0; u < PARTS; ++u) issue_part(0, u);
  wait_vm_n<0>();
  if constexpr (SPLIT) {
    __syncthreads();  // every wave's Q / dO blocks landed
    const char *qt = lds + RINGS * 2 * STAGE + 1024, *gt = qt + TL::BYTES;
#pragma unroll
    for (int j = 0; j < HD / 4; ++j) {
      const float4 x = TL::chunk(qt, c, h * (HD / 4) + j), y = TL::chunk(gt, c, h * (HD / 4) + j);
      qf[4 * j] = x.x, qf[4 * j + 1] = x.y, qf[4 * j + 2] = x.z, qf[4 * j + 3] = x.w;
      gf[4 * j] = y.x, gf[4 * j + 1] = y.y, gf[4 * j + 2] = y.z, gf[4 * j + 3] = y.w;
    }
  }
#pragma unroll
  for (int i = 0; i < HD; ++i) asm volatile("" : "+v"(qf[i]), "+v"(gf[i]));
  if constexpr (!SPLIT) __syncthreads();

  for (int jj = 0; jj < my_tiles; ++jj) {
    const int j = first + STRIDE * jj;
    const char *kt = ring_p + (jj & 1) * STAGE;
    const char *vt = kt + TL::BYTES;
    if (SPLIT || j < w_tiles) {
      f32x16 s = f32x16{}, dp = f32x16{};
      {
        constexpr int NC = HD / 4;
        float4 kc[2], vc[2];
        kc[0] = TL::chunk(kt, c, h * NC);
        vc[0] = TL::chunk(vt, c, h * NC);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < NC; ++q) {
          if (q + 1 < NC) {
            kc[(q + 1) & 1] = TL::chunk(kt, c, h * NC + q + 1);
            vc[(q + 1) & 1] = TL::chunk(vt, c, h * NC + q + 1);
          }
          const float4 kv = kc[q & 1], vv = vc[q & 1];
          s = mfma32f(kv.x, qf[4 * q], s);
          dp = mfma32f(vv.x, gf[4 * q], dp);
          s = mfma32f(kv.y, qf[4 * q + 1], s);
          dp = mfma32f(vv.y, gf[4 * q + 1], dp);
          s = mfma32f(kv.z, qf[4 * q + 2], s);
          dp = mfma32f(vv.z, gf[4 * q + 2], dp);
          s = mfma32f(kv.w, qf[4 * q + 3], s);
          dp = mfma32f(vv.w, gf[4 * q + 3], dp);
          if (PARTS > NC) {
            if (2 * q < PARTS) issue_part(jj + 1, 2 * q);
            if (2 * q + 1 < PARTS) issue_part(jj + 1, 2 * q + 1);
          } else if (q < PARTS) {
            issue_part(jj + 1, q);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      // P = exp2((S + nl) sl), dS = P (dP + nd): element i is key kv0 + crow(i, h)
      const int kv0 = j * BN;
      unsigned kbits = ~0u;
      int lm = 64;
      if (j >= j_edge) {
        lm = klim - kv0 - 4 * h;
        if (keymask) {
          const int key = kv0 + lane;
          const bool ok = key < p.Sk && kmask_b[static_cast<int64_t>(key) * p.mask.s3];
          kbits = static_cast<unsigned>(__ballot(ok) >> (4 * h));
        }
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int kc_ = 8 * (i >> 2) + (i & 3);
        const float pv = ((kc_ < lm) & (((kbits >> kc_) & 1u) != 0)) ? fast_exp2((s[i] + nl) * sl) : 0.f;
        s[i] = pv * (dp[i] + nd);
      }
      // dQ^T += K^T dS^T: step i takes keys crow(i, h) (register i of dS^T)
      {
        constexpr int NS_ = 16 * PDT, FD = 2;
        float kf[FD + 1];
        auto kload = [&](int t) {
          const int i = t / PDT, dt = t % PDT;
          kf[t % (FD + 1)] = TL::elem(kt, 8 * (i >> 2) + 4 * h + (i & 3), 32 * dt + c);
        };
#pragma unroll
        for (int t = 0; t < FD; ++t) kload(t);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < NS_; ++t) {
          if (t + FD < NS_) kload(t + FD);
          acc[t % PDT] = mfma32f(kf[t % (FD + 1)], s[t / PDT], acc[t % PDT]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < PARTS; ++u) issue_part(jj + 1, u);
    }
    wait_vm_n<0>();
    if constexpr (SPLIT) wait_lgkm0();  // (this wave's ring only)
    else __syncthreads();
  }
  float *orow = static_cast<float *>(const_cast<void *>(a.dq.data)) + b * a.dq.s0 + hq * a.dq.s1 +
                static_cast<int64_t>(qrow < p.Sq ? qrow : 0) * a.dq.s2;
  const float sc = a.scale;
  if constexpr (!SPLIT) {
    if (qrow < p.Sq) {
#pragma unroll
      for (int dt = 0; dt < PDT; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<float4 *>(orow + 32 * dt + 8 * g + 4 * h) =
              float4{acc[dt][4 * g] * sc, acc[dt][4 * g + 1] * sc, acc[dt][4 * g + 2] * sc, acc[dt][4 * g + 3] * sc};
    }
  } else {
    // the waves' partial dQ^T, summed in wave order; wave w stores the
    // (dt, g) groups w, w + 4, ...
    __syncthreads();  // every wave's loop (and its last loads) done: the rings are free
    float *co = reinterpret_cast<float *>(lds);  // [NW][PDT][16][64]
#pragma unroll
    for (int dt = 0; dt < PDT; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) co[((w * PDT + dt) * 16 + i) * 64 + lane] = acc[dt][i];
    __syncthreads();
    if (qrow < p.Sq) {
      for (int grp = w; grp < PDT * 4; grp += NW) {
        const int dt = grp >> 2, g = grp & 3;
        float o4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int v = 0; v < NW; ++v)
#pragma unroll
          for (int r = 0; r < 4; ++r) o4[r] += co[((v * PDT + dt) * 16 + 4 * g + r) * 64 + lane];
        *reinterpret_cast<float4 *>(orow + 32 * dt + 8 * g + 4 * h) =
            float4{o4[0] * sc, o4[1] * sc, o4[2] * sc, o4[3] * sc};
      }
    }
  }
}

// ---------------------------------------------------------------------------
// dK / dV: one workgroup = 128 keys of one (b, kv head), 4 waves x 32 keys,
// one workgroup per CU (a wave holds its K and V rows and the dK / dV
// accumulators).  Query tiles of 32 rows -- Q, dO and their row values, for
// every query head of the GQA group (attention.py:245-247) -- double-buffered
// through LDS.  Per tile a wave computes S = Q K^T and dP = dO V^T (Q, dO by
// 16-byte chunks; K, V in registers), P = exp2((S + nl) sl) and dS = P (dP +
// nd) per (row, key), then dV^T += dO^T P and dK^T += Q^T dS (Q, dO by
// 32-float row segments, P and dS the accumulator registers).  dK = scale
// dK^T^T, dV = dV^T^T.
//
// SPLIT (problems with fewer 128-key workgroups than CUs, D <= 64): one
// workgroup = 32 keys, all 4 waves on them; wave w takes tiles w, w + 4, ...
// of the (query head, query tile) walk through its own ring, and the waves'
// dK^T / dV^T partial sums add up through LDS in wave order at the end.
// ---------------------------------------------------------------------------
template <int D, bool SPLIT>
__global__ __launch_bounds__(NT, 1) void dkdv_f32_kernel(F32Args a) {
  using TL = FTile<D>;
  constexpr int HD = D / 2, PDT = D / 32;
  constexpr int RV = 2 * BN * 4;                 // nl | nd of the tile's rows
  constexpr int STAGE = 2 * TL::BYTES + RV;      // Q | dO | row values
  constexpr int KEYS = SPLIT ? 32 : KB;          // keys per workgroup
  constexpr int RINGS = SPLIT ? NW : 1, STRIDE = SPLIT ? NW : 1;
  constexpr int PARTS = SPLIT ? 2 * TL::BLOCKS : 2 * TL::BLOCKS / NW;
  static_assert(SPLIT || (PARTS * NW == 2 * TL::BLOCKS && PARTS >= 1), "tile loads split over the waves");
  // (the prologue first stages the workgroup's K and V rows in the same bytes)
  constexpr int KVB = KEYS * D * 4;  // bytes of the workgroup's K (and of its V) rows
  constexpr int LDS_B = RINGS * 2 * STAGE + 1024 > 2 * KVB ? RINGS * 2 * STAGE + 1024 : 2 * KVB;
  __shared__ __attribute__((aligned(1024))) char lds[LDS_B];

  const Problem &p = a.p;
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 31, h = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_kb = (p.Sk + KEYS - 1) / KEYS;
  const int total = n_kb * p.Hkv * p.B;
  const int logical = xcd_remap(blockIdx.x, total);
  int bh, kb;
  heavy_first(logical, n_kb, p.Hkv * p.B, 32, bh, kb);
  const int b = bh / p.Hkv, hk = bh - b * p.Hkv;
  const int k0 = kb * KEYS, kw = SPLIT ? k0 : k0 + 32 * w, key = kw + c;
  const int kv_end = kv_end_for(p, b);
  const bool keymask = p.mask.kind == TSATTN_MASK_BOOL && !(p.kv_prefix && p.kv_prefix[b]);
  const bool key_live = key < kv_end &&
                        (!keymask || static_cast<const uint8_t *>(p.mask.data)[b * p.mask.s0 + static_cast<int64_t>(key) * p.mask.s3]);
  int q_start = 0;
  if (p.causal) {
    const int64_t s0 = static_cast<int64_t>(k0) - p.offset;
    q_start = s0 <= 0 ? 0 : static_cast<int>(s0 < p.Sq ? s0 : p.Sq);
    q_start = (q_start / BN) * BN;
  }
  const int n_qt = __builtin_amdgcn_readfirstlane(k0 < kv_end ? (p.Sq - q_start + BN - 1) / BN : 0);
  const int n_iter = __builtin_amdgcn_readfirstlane(n_qt * p.rep);
  // this wave's tiles: it = first + STRIDE jj, jj < my_iter
  const int first = SPLIT ? w : 0;
  const int my_iter = SPLIT ? (n_iter > w ? (n_iter - 1 - w) / NW + 1 : 0) : n_iter;
  const int64_t rows = static_cast<int64_t>(p.B) * p.Hq * p.Sq;

  const uint32_t qs_b = static_cast<uint32_t>(a.q.s2) * 4, gs_b = static_cast<uint32_t>(a.dout.s2) * 4;
  const uint32_t ks_b = static_cast<uint32_t>(a.k.s2) * 4, vs_b = static_cast<uint32_t>(a.v.s2) * 4;
  // This wave's K and V rows (key = kw + c, half h of the row): staged
  // through LDS -- the workgroup's rows land there by DMA, whole lines per
  // instruction, as 32-row FTiles, and each wave reads its 32 rows' halves.
  // (Straight into registers each instruction touches 64 cache lines: the
  // address unit, not memory, then bounds the prologue; split workgroups
  // would also load the same rows four times.)  Keys past the cache end
  // read as zeros.
  float kf[HD], vf[HD];
  {
    const uint32_t lds_kv = lds_addr(lds);
    const u32x4 kd = make_desc(f32_head<float>(a.k, b, hk), static_cast<uint32_t>(kv_end) * ks_b);
    const u32x4 vd = make_desc(f32_head<float>(a.v, b, hk), static_cast<uint32_t>(kv_end) * vs_b);
    static_assert(KEYS / 32 * TL::BLOCKS % NW == 0, "K / V blocks split evenly over the waves");
#pragma unroll
    for (int u = 0; u < KEYS / 32 * TL::BLOCKS / NW; ++u) {
      const int m = w + NW * u, t = m / TL::BLOCKS, n = m % TL::BLOCKS;  // tile t (keys k0 + 32 t ..), block n
      const int row = k0 + 32 * t + n * TL::RPB;
      dma16(kd, lds_kv + t * TL::BYTES + n * 1024, TL::dma_off(n, lane, ks_b), static_cast<uint32_t>(row) * ks_b);
      dma16(vd, lds_kv + KVB + t * TL::BYTES + n * 1024, TL::dma_off(n, lane, vs_b), static_cast<uint32_t>(row) * vs_b);
    }
    wait_vm_n<0>();
    __syncthreads();
    const char *kt = lds + (SPLIT ? 0 : w * TL::BYTES), *vt = lds + KVB + (SPLIT ? 0 : w * TL::BYTES);
#pragma unroll
    for (int j = 0; j < HD / 4; ++j) {
      const float4 x = TL::chunk(kt, c, h * (HD / 4) + j), y = TL::chunk(vt, c, h * (HD / 4) + j);
      kf[4 * j] = x.x, kf[4 * j + 1] = x.y, kf[4 * j + 2] = x.z, kf[4 * j + 3] = x.w;
      vf[4 * j] = y.x, vf[4 * j + 1] = y.y, vf[4 * j + 2] = y.z, vf[4 * j + 3] = y.w;
    }
    wait_lgkm0();
    __syncthreads();  // every wave's reads done before the ring takes the first tiles
  }

  // tile it = query tile it % n_qt of query head hk rep + it / n_qt
  const uint32_t lds0 = lds_addr(lds);
  const uint32_t ring = lds0 + (SPLIT ? w * 2 * STAGE : 0);
  const char *ring_p = lds + (SPLIT ? w * 2 * STAGE : 0);
  const uint32_t spare = lds0 + RINGS * 2 * STAGE;
  // the loads of local tile jj (tile first + STRIDE jj): this wave's share of
  // its Q / dO blocks (split: all of them) and row values
  auto issue = [&](int jj) {
    const int it = first + STRIDE * jj;
    const bool real = it < n_iter;
    const int r = real ? it / n_qt : 0, qi = real ? it - r * n_qt : 0;
    const int hq = hk * p.rep + r, q0 = q_start + qi * BN;
    const uint32_t st = real ? ring + (jj & 1) * STAGE : spare;
    const u32x4 qd = make_desc(f32_head<float>(a.q, b, hq), static_cast<uint32_t>(p.Sq) * qs_b);
    const u32x4 gd = make_desc(f32_head<float>(a.dout, b, hq), static_cast<uint32_t>(p.Sq) * gs_b);
#pragma unroll
    for (int u = 0; u < PARTS; ++u) {
      const int n = SPLIT ? u : w + NW * u;
      if (n < TL::BLOCKS) {
        const uint32_t so = real ? static_cast<uint32_t>(q0 + n * TL::RPB) * qs_b : 0x80000000u;
        dma16(qd, st + (real ? n * 1024 : 0), TL::dma_off(n, lane, qs_b), so);
      } else {
        const int m = n - TL::BLOCKS;
        const uint32_t so = real ? static_cast<uint32_t>(q0 + m * TL::RPB) * gs_b : 0x80000000u;
        dma16(gd, st + (real ? TL::BYTES + m * 1024 : 0), TL::dma_off(m, lane, gs_b), so);
      }
    }
    // the rows' nl (wave 0; split: every wave) and nd (wave 1; split: every
    // wave): 8 lanes of 16 bytes each
#pragma unroll
    for (int part = 0; part < (SPLIT ? 2 : 1); ++part) {
      const int which = SPLIT ? part : w;  // 0: nl, 1: nd
      const float *rv = a.rows + (static_cast<int64_t>(b) * p.Hq + hq) * p.Sq + (which == 0 ? rows : 0);
      const u32x4 rd = make_desc(rv, static_cast<uint32_t>(p.Sq) * 4);
      const bool mine = real && which < 2;
      if (lane < BN / 4)
        dma16(rd, mine ? st + 2 * TL::BYTES + which * BN * 4 : spare, static_cast<uint32_t>(lane) * 16,
              mine ? static_cast<uint32_t>(q0) * 4 : 0x80000000u);
    }
  };

  f32x16 dka[PDT], dva[PDT];
#pragma unroll
  for (int dt = 0; dt < PDT; ++dt) dka[dt] = dva[dt] = f32x16{};
  const float sl = a.sl;
  const int64_t kd64 = static_cast<int64_t>(key) - p.offset;
  const int kdiff = kd64 < -(1 << 30) ? -(1 << 30) : static_cast<int>(kd64);

  issue(0);
  wait_vm_n<0>();
#pragma unroll
  for (int i = 0; i < HD; ++i) asm volatile("" : "+v"(kf[i]), "+v"(vf[i]));
  if constexpr (!SPLIT) __syncthreads();

  for (int jj = 0; jj < my_iter; ++jj) {
    const int it = first + STRIDE * jj;
    const char *qt = ring_p + (jj & 1) * STAGE;
    const char *gt = qt + TL::BYTES;
    const float *rvl = reinterpret_cast<const float *>(qt + 2 * TL::BYTES);  // nl [32] | nd [32]
    const int r = it / n_qt, qi = it - r * n_qt;
    const int q0 = q_start + qi * BN;
    issue(jj + 1);
    // S = Q K^T, dP = dO V^T over the tile's 32 rows x this wave's 32 keys
    f32x16 s = f32x16{}, dp = f32x16{};
    {
      constexpr int NC = HD / 4;
      float4 qc[2], gc[2];
      qc[0] = TL::chunk(qt, c, h * NC);
      gc[0] = TL::chunk(gt, c, h * NC);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int jj = 0; jj < NC; ++jj) {
        if (jj + 1 < NC) {
          qc[(jj + 1) & 1] = TL::chunk(qt, c, h * NC + jj + 1);
          gc[(jj + 1) & 1] = TL::chunk(gt, c, h * NC + jj + 1);
        }
        const float4 qv = qc[jj & 1], gv = gc[jj & 1];
        s = mfma32f(qv.x, kf[4 * jj], s);
        dp = mfma32f(gv.x, vf[4 * jj], dp);
        s = mfma32f(qv.y, kf[4 * jj + 1], s);
        dp = mfma32f(gv.y, vf[4 * jj + 1], dp);
        s = mfma32f(qv.z, kf[4 * jj + 2], s);
        dp = mfma32f(gv.z, vf[4 * jj + 2], dp);
        s = mfma32f(qv.w, kf[4 * jj + 3], s);
        dp = mfma32f(gv.w, vf[4 * jj + 3], dp);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // element i: row q0 + crow(i, h), key `key`; allowed iff the key is live,
    // the row exists and (causal) key - offset <= row
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int rr = 8 * (i >> 2) + 4 * h + (i & 3);
      const bool ok = key_live && (q0 + rr < p.Sq) && (!p.causal || kdiff <= q0 + rr);
      const float pv = ok ? fast_exp2((s[i] + rvl[rr]) * sl) : 0.f;
      s[i] = pv;
      dp[i] = pv * (dp[i] + rvl[BN + rr]);
    }
    // dV^T += dO^T P, dK^T += Q^T dS: step i takes rows crow(i, h)
    {
      constexpr int NS_ = 16 * PDT, FD = 2;
      float gfr[FD + 1], qfr[FD + 1];
      auto load = [&](int t) {
        const int i = t / PDT, dt = t % PDT, rr = 8 * (i >> 2) + 4 * h + (i & 3);
        gfr[t % (FD + 1)] = TL::elem(gt, rr, 32 * dt + c);
        qfr[t % (FD + 1)] = TL::elem(qt, rr, 32 * dt + c);
      };
#pragma unroll
      for (int t = 0; t < FD; ++t) load(t);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < NS_; ++t) {
        if (t + FD < NS_) load(t + FD);
        dva[t % PDT] = mfma32f(gfr[t % (FD + 1)], s[t / PDT], dva[t % PDT]);
        dka[t % PDT] = mfma32f(qfr[t % (FD + 1)], dp[t / PDT], dka[t % PDT]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    wait_vm_n<0>();
    if constexpr (SPLIT) wait_lgkm0();  // (this wave's ring only)
    else __syncthreads();
  }
  const int krow_i = key < p.Sk ? key : 0;
  float *krow = static_cast<float *>(const_cast<void *>(a.dk.data)) + b * a.dk.s0 + hk * a.dk.s1 +
                static_cast<int64_t>(krow_i) * a.dk.s2;
  float *vrow = static_cast<float *>(const_cast<void *>(a.dv.data)) + b * a.dv.s0 + hk * a.dv.s1 +
                static_cast<int64_t>(krow_i) * a.dv.s2;
  const float sc = a.scale;
  if constexpr (!SPLIT) {
    if (key < p.Sk) {
#pragma unroll
      for (int dt = 0; dt < PDT; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          *reinterpret_cast<float4 *>(krow + 32 * dt + 8 * g + 4 * h) =
              float4{dka[dt][4 * g] * sc, dka[dt][4 * g + 1] * sc, dka[dt][4 * g + 2] * sc, dka[dt][4 * g + 3] * sc};
          *reinterpret_cast<float4 *>(vrow + 32 * dt + 8 * g + 4 * h) =
              float4{dva[dt][4 * g], dva[dt][4 * g + 1], dva[dt][4 * g + 2], dva[dt][4 * g + 3]};
        }
    }
  } else {
    // the waves' partial dK^T / dV^T, summed in wave order; wave w stores the
    // (dt, g) groups w, w + 4, ... of both
    __syncthreads();  // every wave's loop (and its last loads) done: the rings are free
    float *co = reinterpret_cast<float *>(lds);  // [NW][2 (dK, dV)][PDT][16][64]
#pragma unroll
    for (int dt = 0; dt < PDT; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        co[(((w * 2 + 0) * PDT + dt) * 16 + i) * 64 + lane] = dka[dt][i];
        co[(((w * 2 + 1) * PDT + dt) * 16 + i) * 64 + lane] = dva[dt][i];
      }
    __syncthreads();
    if (key < p.Sk) {
      for (int grp = w; grp < PDT * 4; grp += NW) {
        const int dt = grp >> 2, g = grp & 3;
        float k4[4] = {0.f, 0.f, 0.f, 0.f}, v4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int v = 0; v < NW; ++v)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            k4[r] += co[(((v * 2 + 0) * PDT + dt) * 16 + 4 * g + r) * 64 + lane];
            v4[r] += co[(((v * 2 + 1) * PDT + dt) * 16 + 4 * g + r) * 64 + lane];
          }
        *reinterpret_cast<float4 *>(krow + 32 * dt + 8 * g + 4 * h) =
            float4{k4[0] * sc, k4[1] * sc, k4[2] * sc, k4[3] * sc};
        *reinterpret_cast<float4 *>(vrow + 32 * dt + 8 * g + 4 * h) = float4{v4[0], v4[1], v4[2], v4[3]};
      }
    }
  }
}

template <int D>
void launch_bwd_dims(const F32Args &a, hipStream_t st) {
  const Problem &p = a.p;
  {
    Probe pr_("bwd_rows_f32", st);
    const int64_t rows = static_cast<int64_t>(p.B) * p.Hq * p.Sq;
    const int64_t per_block = NW * (64 / (D / 4));
    rows_f32_kernel<D><<<dim3(static_cast<unsigned>((rows + per_block - 1) / per_block)), dim3(NT), 0, st>>>(a);
  }
  const int64_t qheads = static_cast<int64_t>(p.Hq) * p.B, kheads = static_cast<int64_t>(p.Hkv) * p.B;
  const int64_t n_qb = (p.Sq + BM - 1) / BM, n_kb = (p.Sk + KB - 1) / KB;
  bool split_q = false, split_k = false;
  if constexpr (D <= 64) {  // (the split rings of D = 128 would not fit in LDS)
    split_q = n_qb * qheads < device_cus();
    split_k = n_kb * kheads < device_cus();
  }
  if (split_q) {
    if constexpr (D <= 64) {
      Probe pr_("bwd_dq_mfma_f32_split", st);
      dq_f32_kernel<D, true><<<dim3(static_cast<unsigned>((p.Sq + 31) / 32 * qheads)), dim3(NT), 0, st>>>(a);
    }
  } else {
    Probe pr_("bwd_dq_mfma_f32", st);
    dq_f32_kernel<D, false><<<dim3(static_cast<unsigned>(n_qb * qheads)), dim3(NT), 0, st>>>(a);
  }
  if (split_k) {
    if constexpr (D <= 64) {
      Probe pr_("bwd_dkdv_mfma_f32_split", st);
      dkdv_f32_kernel<D, true><<<dim3(static_cast<unsigned>((p.Sk + 31) / 32 * kheads)), dim3(NT), 0, st>>>(a);
    }
  } else {
    Probe pr_("bwd_dkdv_mfma_f32", st);
    dkdv_f32_kernel<D, false><<<dim3(static_cast<unsigned>(n_kb * kheads)), dim3(NT), 0, st>>>(a);
  }
}

template <int D>
void launch_fwd_dims(const F32Args &a, hipStream_t st) {
  const int64_t heads = static_cast<int64_t>(a.p.Hq) * a.p.B;
  const int64_t n_qb = (a.p.Sq + BM - 1) / BM;
  if constexpr (D <= 64) {  // (the split rings of D = 128 would not fit in LDS)
    if (n_qb * heads < device_cus()) {
      Probe pr_("fwd_mfma_f32_split", st);
      fwd_f32_kernel<D, true><<<dim3(static_cast<unsigned>((a.p.Sq + 31) / 32 * heads)), dim3(NT), 0, st>>>(a);
      return;
    }
  }
  Probe pr_("fwd_mfma_f32", st);
  fwd_f32_kernel<D, false><<<dim3(static_cast<unsigned>(n_qb * heads)), dim3(NT), 0, st>>>(a);
}

}  // namespace

hipError_t launch_mfma_f32_backward(const Problem &p, View q, View k, View v, View o, View dout,
                                    const float *lse, View dq, View dk, View dv, float *rows,
                                    hipStream_t st) {
  F32Args a{};
  a.p = p;
  a.q = q, a.k = k, a.v = v, a.o = o, a.dout = dout, a.dq = dq, a.dk = dk, a.dv = dv;
  a.lse = const_cast<float *>(lse);
  a.rows = rows;
  a.sl = static_cast<float>(p.scale) * kLog2e;
  a.scale = static_cast<float>(p.scale);
  if (p.Dqk == 128) launch_bwd_dims<128>(a, st);
  else if (p.Dqk == 64) launch_bwd_dims<64>(a, st);
  else launch_bwd_dims<32>(a, st);
  return hipGetLastError();
}

bool mfma_f32_supported(const Problem &p, int dtype) {
  if (dtype != TSATTN_F32 || p.Dqk != p.Dv) return false;
  if (p.Dqk != 32 && p.Dqk != 64 && p.Dqk != 128) return false;
  if (!(p.scale > 0.0) || p.drop.on || p.rope.R > 0) return false;
  // masks: none, or a [B,1,1,K] boolean key mask reduced to lengths
  return p.mask.kind == TSATTN_MASK_NONE ||
         (p.mask.kind == TSATTN_MASK_BOOL && p.mask.s1 == 0 && p.mask.s2 == 0 && p.kv_len != nullptr);
}

hipError_t launch_mfma_f32_forward(const Problem &p, View q, View k, View v, View o, float *lse,
                                   hipStream_t st) {
  F32Args a{};
  a.p = p;
  a.q = q, a.k = k, a.v = v, a.o = o;
  a.lse = lse;
  a.sl = static_cast<float>(p.scale) * kLog2e;
  a.scale = static_cast<float>(p.scale);
  if (p.Dqk == 128) launch_fwd_dims<128>(a, st);
  else if (p.Dqk == 64) launch_fwd_dims<64>(a, st);
  else launch_fwd_dims<32>(a, st);
  return hipGetLastError();
}

}  // namespace tsattn
