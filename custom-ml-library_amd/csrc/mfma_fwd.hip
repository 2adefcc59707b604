// Flash-style attention forward for gfx950: MFMA 32x32x16 (f16/bf16 in,
// fp32 accumulate), online softmax in the exp2 domain, row LSE saved.  Head
// dims 64 or 128, q / k and v / o independently (Dqk != Dv, the reference's
// value_dim), or 32 for both.
//
// Algorithm: the reference's streaming forward (src/tensorsmith/nn/
// attention.py:175-198) -- running max m, denominator l and accumulator per
// query row, rescaled by exp(m - m') when the max moves; O = acc / l;
// LSE = m + log l; fully masked rows give O = 0, LSE = -inf.
//
// Work split: one workgroup = 4 wavefronts = 128 query rows of one (b, h),
// two workgroups per CU; each wave owns 32 rows and computes S^T = K Q^T, so
// each lane owns one query column: the softmax statistics stay lane-local,
// and P^T leaves the accumulator registers as the B operand of
// O^T += V^T P^T.  K is read from LDS as row fragments, V^T with LDS
// transpose reads.
//
// Schedule: per key tile of 32 rows a wave runs one MFMA block -- PV of the
// previous tile fused with S of the current one, 16 MFMAs at D = 128, the
// LDS fragments of each step prefetched two steps ahead -- then the softmax
// of the current tile on the VALU.  The two waves sharing a SIMD belong to
// different workgroups, so one's MFMA block overlaps the other's softmax.
// Key/value tiles stream global -> LDS by direct (DMA) buffer loads into a
// 4-stage ring, issued two tiles ahead and spread over the steps of the
// MFMA block (issuing them all at once stalls every wave on the shared
// address unit); the per-tile barrier is a bare s_barrier (no memory fence),
// and each wave waits only for the next tile.
//
// Rescaling is lazy: the reference max m is raised (and O, l rescaled) only
// when a row's max exceeds it by more than kTau (in log2 units), so P <= 2^kTau
// and most tiles skip the rescale.  O / l and the LSE are exact for any m.
//
// Dropout (template DR): the probabilities fed to PV are multiplied by the
// keep mask the problem's Philox stream gives (philox.h), while the softmax
// denominator sums the undropped ones; with DropDesc::bits set the kernel
// also writes the mask as bits (one word per row and 32-key tile it
// computes) for the backward.
//
// RoPE (Problem::rope, R > 0): the prologue rotates the query fragments it
// loads (the keys come rotated), bit-identical to a separate tsattn_rope;
// with rope.qrot set the epilogue also stores them there for the backward.
//
// Masks (template MK): a key mask reduced to per-row lengths costs one ballot
// per tile; a general boolean or additive mask (MK = 1 / 2) is read per
// (query row, key) from its broadcast strides on every tile, an additive one
// entering as scores * scale + mask (attention.py:105-107) in log2 units
// (MK = 2 for an f32 mask, 3 for f16 / bf16; 4..6 the same read as 16-byte
// row pieces when the keys are contiguous and the rows aligned).
#include <type_traits>

#include "mfma_common.h"
#include "philox.h"
#include "rope_math.h"

namespace tsattn {
namespace {

constexpr int BM = 128;  // query rows per workgroup
constexpr int BN = 32;   // keys per tile
constexpr int NT = 256;  // threads
constexpr int NW = NT / 64;
constexpr int PD = 2;    // tiles issued ahead
constexpr int NS = PD + 2;  // K/V ring stages: tile j is read in iterations j and j + 1
constexpr float kTau = 8.f;

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

// DK = head dim of q / k, DV = of v / o (each 64 or 128).
template <typename T, int DK, int DV, int MK, bool DR>
__global__ __launch_bounds__(NT, 2) void fwd_kernel(FwdArgs a) {
  constexpr int TILE_K = BN * DK * 2, TILE_V = BN * DV * 2;  // bytes per K / V tile
  constexpr int STAGE = TILE_K + TILE_V;
  // 1 KiB DMA blocks of a K / V tile; wave w loads blocks w, w + NW, ... of
  // the stage (K blocks, then V blocks).  When both counts are multiples of
  // NW (head dims 64 / 128) the split is the compile-time one below: parts
  // u < KPARTS are K blocks.  At head dim 32 a tile is 2 blocks: waves 0, 1
  // load K, waves 2, 3 load V.
  constexpr int KBLK = TILE_K / 1024, VBLK = TILE_V / 1024;
  constexpr bool EVEN = KBLK % NW == 0 && VBLK % NW == 0;
  constexpr int KPARTS = KBLK / NW;           // K blocks per wave (EVEN split)
  constexpr int VPARTS = VBLK / NW;           // ... V blocks
  constexpr int LPT = (KBLK + VBLK + NW - 1) / NW;  // DMA loads per wave per K+V tile
  constexpr int SKS = DK / 16;                // k-steps of S^T = K Q^T
  constexpr int PDT = DV / 32;                // 32-row blocks of O^T
  constexpr int PVS = 2 * PDT;                // PV MFMAs per tile (two key k-steps each block)
  constexpr int STEPS = SKS > PVS ? SKS : PVS;
  constexpr int QGK = DK / 32, QGV = DV / 32;  // 4-chunk groups per K / V row
  static_assert(EVEN ? (KPARTS >= 1 && VPARTS >= 1 && LPT == KPARTS + VPARTS)
                     : (KBLK + VBLK == NW && LPT == 1 && DK == 32 && DV == 32),
                "tile loads must split over the waves");
  static_assert(2 * LPT <= STEPS, "one DMA part per two MFMA steps");
  // [stage][K | V], then one 1 KiB block that DMA parts past the last tile
  // land in (nothing reads it)
  __shared__ __attribute__((aligned(1024))) char lds[NS * STAGE + 1024];

  const Problem &p = a.p;
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 31, h = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, in an SGPR
  const int logical = xcd_remap(blockIdx.x, a.total);
  int bh, rank;
  heavy_first(logical, a.n_qblocks, a.total / a.n_qblocks, 64, bh, rank);  // 2 WG per CU
  const int qb = a.n_qblocks - 1 - rank;  // long causal rows first
  const int b = bh / p.Hq, hq = bh - b * p.Hq, hk = hq / p.rep;
  const int q0 = qb * BM, qw = q0 + 32 * w, qrow = qw + c;

  const int kv_end = kv_end_for(p, b);
  const bool keymask =
      MK == 0 && p.mask.kind == TSATTN_MASK_BOOL && !(p.kv_prefix && p.kv_prefix[b]);

  // Key tiles of the workgroup (all its rows) and of this wave.
  int64_t lim = kv_end, wlim = kv_end;
  const int last_q = min(q0 + BM, p.Sq) - 1;
  const int last_qw = min(qw + 32, p.Sq) - 1;
  if (p.causal) {
    lim = min(lim, static_cast<int64_t>(last_q) + p.offset + 1);
    wlim = min(wlim, static_cast<int64_t>(last_qw) + p.offset + 1);
  }
  if (qw >= p.Sq) wlim = 0;
  // wave-uniform by construction; readfirstlane keeps them in SGPRs
  const int n_tiles =
      __builtin_amdgcn_readfirstlane(lim > 0 ? static_cast<int>((lim + BN - 1) / BN) : 0);
  const int w_tiles =
      __builtin_amdgcn_readfirstlane(wlim > 0 ? static_cast<int>((wlim + BN - 1) / BN) : 0);

  const uint32_t qs_b = static_cast<uint32_t>(a.q.s2) * 2;
  const uint32_t ks_b = static_cast<uint32_t>(a.k.s2) * 2;
  const uint32_t vs_b = static_cast<uint32_t>(a.v.s2) * 2;
  const rsrc_t qrs = make_rsrc(head_ptr<T>(a.q, b, hq), static_cast<uint32_t>(p.Sq) * qs_b);
  const u32x4 kdesc = make_desc(head_ptr<T>(a.k, b, hk), static_cast<uint32_t>(kv_end) * ks_b);
  const u32x4 vdesc = make_desc(head_ptr<T>(a.v, b, hk), static_cast<uint32_t>(kv_end) * vs_b);

  // Q fragments (B operand of S^T = K Q^T): lane holds Q[qrow][16ks + 8h .. +7].
  // When the workgroup's 128 Q rows fit in ring stages 2 and 3 (DK <= DV)
  // they come through there: by DMA beside the first two tiles (whole
  // lines, eight rows per instruction), then each wave's fragment reads.
  // Otherwise straight into registers (each instruction then touches 32
  // rows, slow to issue).
  constexpr bool QSTAGE = BM * DK * 2 <= 2 * STAGE;
  u32x4 qf[SKS];  // (DK channels)
  if constexpr (!QSTAGE) {
#pragma unroll
    for (int ks = 0; ks < SKS; ++ks)
      qf[ks] = buf_load16(qrs, static_cast<uint32_t>(qrow) * qs_b + (ks * 16 + h * 8) * 2);
  }
  // RoPE folded in: the lane's channels 16 ks + 8 h .. + 7 (pairs 8 ks +
  // 4 h ..) rotate by position qpos0 + qrow, exactly as tsattn_rope would.
  // The table loads and the rotation run after the first tiles' DMA issue,
  // under their latency.
  const bool rope = p.rope.R > 0;
  // Resolve the Q loads here: the compiler's own vmcnt waits do not count the
  // DMA loads below, so a first use of qf inside the main loop would make it
  // wait there for tiles still in flight.
  if constexpr (!QSTAGE) {
#pragma unroll
    for (int ks = 0; ks < SKS; ++ks) asm volatile("" : "+v"(qf[ks]));
  }

  const uint32_t lds0 = lds_addr(lds);
  // DMA of key tile `tile` into its ring stage.  The 1 KiB blocks of the K
  // (then V) tile are numbered n = 0, 1, ...; wave w loads n = w, w + 4, ...
  // Block n = (rg, qg) = (n / QG, n % QG); its lane l fetches row 16 rg + l/4,
  // chunk 4 qg + ((l % 4) ^ ((l / 16) % 4)).  qg = w % QG for all of the
  // wave's blocks, so the per-lane part of the offset is loop-invariant and
  // the row part is wave-uniform.
  const uint32_t swz_chunk = (lane & 3) ^ ((lane >> 4) & 3);
  const uint32_t koff = (lane >> 2) * ks_b + (4 * (w % QGK) + swz_chunk) * 16;
  const uint32_t voff = (lane >> 2) * vs_b + (4 * (w % QGV) + swz_chunk) * 16;
  // Parts u < KPARTS are K blocks, the rest V blocks (a compile-time split).
  // Every iteration issues its LPT parts: those of a tile past the last one
  // read row 0 into the spare LDS block, so the count of loads in flight is
  // the same on every iteration and no branch guards an issue.
  const uint32_t spare = lds0 + NS * STAGE;
  // Per-tile DMA state, computed once per tile: the byte offset of its first
  // row in K and V, and its stage offset from the spare block masked by keep
  // (all ones for a real tile, else 0 -- masks instead of selects, which the
  // compiler turns into branches between the MFMA steps).  A tile past the
  // last one reads past the buffer range (zeros, no memory access) into the
  // spare block.
  struct DmaTile {
    uint32_t krow, vrow, st, keep;
  };
  auto dma_tile = [&](int tile) {
    DmaTile d;
    // all ones iff n_tiles - 1 - tile >= 0 (sign fill of the difference)
    d.keep = ~static_cast<uint32_t>((n_tiles - 1 - tile) >> 31);
    // a tile past the last one reads at offsets >= 2^31, past the range
    const uint32_t far = ~d.keep & 0x80000000u;
    d.krow = (static_cast<uint32_t>(tile * BN) * ks_b) | far;
    d.vrow = (static_cast<uint32_t>(tile * BN) * vs_b) | far;
    d.st = (lds0 + (tile % NS) * STAGE - spare) & d.keep;
    return d;
  };
  auto issue_k = [&](const DmaTile &d, int n) {
    dma16(kdesc, spare + d.st + ((n * 1024) & d.keep), koff,
          d.krow + static_cast<uint32_t>(16 * (n / QGK)) * ks_b);
  };
  auto issue_v = [&](const DmaTile &d, int n) {
    dma16(vdesc, spare + d.st + ((TILE_K + n * 1024) & d.keep), voff,
          d.vrow + static_cast<uint32_t>(16 * (n / QGV)) * vs_b);
  };
  auto issue_part = [&](const DmaTile &d, int u) {
    if constexpr (EVEN) {
      if (u < KPARTS) issue_k(d, w + NW * u);
      else issue_v(d, w + NW * (u - KPARTS));
    } else {
      if (w < KBLK) issue_k(d, w);  // (w is wave-uniform: a scalar branch)
      else issue_v(d, w - KBLK);
    }
  };
  auto issue = [&](int tile) {
    const DmaTile d = dma_tile(tile);
#pragma unroll
    for (int u = 0; u < LPT; ++u) issue_part(d, u);
  };

  const TileReader<T, DK> rdk(lane);
  const TileReader<T, DV> rdv(lane);
  f32x16 oacc[PDT];
#pragma unroll
  for (int dt = 0; dt < PDT; ++dt) oacc[dt] = f32x16{};
  f32x16 s = f32x16{};
  u32x4 pb[2];  // P^T of the previous tile, packed: B operands of its 2 PV k-steps
  float m = -INFINITY, l = 0.f;
  const float sl = a.sl;
  // Kept with m, recomputed only when it moves: raw row maxima above thr =
  // (m + kTau) / scale trigger a rescale, and nbase = -m (0 while m = -inf)
  // is the exponent offset.
  float thr = -INFINITY, nbase = 0.f;
  // This lane's allowed keys are [0, klim) (cache end and causal window),
  // further thinned by the key mask row kmask_b when there is one.
  int klim = kv_end;
  if (p.causal) {
    const int64_t cl = static_cast<int64_t>(qrow) + p.offset + 1;
    if (cl < kv_end) klim = cl < 0 ? 0 : static_cast<int>(cl);
  }
  const uint8_t *kmask_b =
      keymask ? static_cast<const uint8_t *>(p.mask.data) + b * p.mask.s0 : nullptr;
  // General mask: the (b, hq) slice as a buffer; this lane reads row qrow.
  // Rows past Sq use none of what they read.
  constexpr int mes = mask_bytes<MK>();
  u32x4 mdesc{};
  uint32_t mrow = 0, mstep = 0;
  if constexpr (MK != 0) {
    const int64_t extent = ((p.Sq - 1) * p.mask.s2 + (p.Sk - 1) * p.mask.s3 + 1) * mes;
    mdesc = make_desc(static_cast<const char *>(p.mask.data) + (b * p.mask.s0 + hq * p.mask.s1) * mes,
                      static_cast<uint32_t>(extent));
    mrow = static_cast<uint32_t>(static_cast<int64_t>(qrow) * p.mask.s2 * mes);
    mstep = static_cast<uint32_t>(p.mask.s3 * mes);
    if (qrow >= p.Sq) klim = 0;
  }
  // Dropout block index of this lane half's first 16 keys of its row (tile j
  // adds 2 j).
  uint64_t drow = 0;
  if constexpr (DR)
    drow = dropout_block_index(p, (static_cast<int64_t>(b) * p.Hq + hq) * p.Sq + qrow, 16 * h);
  PhiloxPair ph{};  // dropout: the keep words of the tile in flight
  MaskFetch mf;
  // Scores an additive mask has already scaled (x sl + mask log2 e) take 1.
  const float slx = mask_kind(MK) >= 2 ? 1.f : a.sl;
  const float inv_slx = 1.f / slx;

  // The first MFMA block runs PV with P = 0 against the V half of stage
  // NS - 1, which no DMA has written yet: zero it (0 x stale NaN is NaN).
  // Every other LDS byte is written by a DMA load before it is read (lanes
  // past the buffer range write zeros).
  if constexpr (QSTAGE) {
    // Q rows into stages 2 and 3 (blocked layout, as a 128-row K tile: wave
    // w loads blocks w, w + 4, ...), the first two tiles into stages 0 and
    // 1; every wave's fragment reads done before the zeroing below, which
    // falls in the staging area.
    const u32x4 qdesc = make_desc(head_ptr<T>(a.q, b, hq), static_cast<uint32_t>(p.Sq) * qs_b);
    const uint32_t qoff = (lane >> 2) * qs_b + (4 * (w % QGK) + swz_chunk) * 16;
#pragma unroll
    for (int u = 0; u < BM / 16 * QGK / NW; ++u) {
      const int n = w + NW * u;  // block (16 rows (n / QGK), chunk group n % QGK = w % QGK)
      dma16(qdesc, lds0 + 2 * STAGE + n * 1024, qoff, static_cast<uint32_t>(q0 + 16 * (n / QGK)) * qs_b);
    }
    for (int t = 0; t < PD; ++t) issue(t);
    wait_vm_n<0>();
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < SKS; ++ks) qf[ks] = rdk.rows(lds + 2 * STAGE, w, ks);
    wait_lgkm0();
    __syncthreads();
    zero_lds<NT>(lds + (NS - 1) * STAGE + TILE_K, TILE_V, tid);
  } else {
    zero_lds<NT>(lds + (NS - 1) * STAGE + TILE_K, TILE_V, tid);
    __syncthreads();
    for (int t = 0; t < PD; ++t) issue(t);
  }
  if (rope) {
    // (the compiler's wait for the tables also covers the DMA parts issued
    // before them, which the wait below needs anyway)
    int64_t rows[SKS];
    int rp0[SKS];
#pragma unroll
    for (int ks = 0; ks < SKS; ++ks) {
      rows[ks] = p.rope.qpos0 + (qrow < p.Sq ? qrow : p.Sq - 1);  // rows past Sq: unused
      rp0[ks] = 8 * ks + 4 * h;
    }
    rotate_chunks<T, SKS>(qf, p.rope, rows, rp0, false);
  }
  wait_vm_n<(PD - 1) * LPT>();
  __syncthreads();

  // Tiles from j_edge on need masking (the causal diagonal, a ragged end, a
  // key mask or a general mask); those before it are interior.
  int j_edge = kv_end / BN;
  if (MK != 0 || keymask) j_edge = 0;
  if (p.causal) {
    const int64_t d = static_cast<int64_t>(qw) + p.offset - (BN - 1);
    const int jc = d < 0 ? 0 : static_cast<int>(min(d / BN + 1, static_cast<int64_t>(INT32_MAX)));
    j_edge = min(j_edge, jc);
  }

  // MFMA block of key tile j: O^T += V_{j-1}^T P_{j-1}^T and S_j^T = K_j Q^T.
  // Step i issues S k-step i and PV MFMA i (value block i % PDT, key k-step
  // i / PDT), so dependent S MFMAs are two issues apart, while the fragments
  // of step i+1 load.  One code path for every block keeps the accumulators
  // in place: the first block runs PV with P = 0 (its V stage is still the
  // zeroed LDS), and past the wave's last tile S is computed and ignored.
  // fetch: also load tile j's mask elements (before the DMA parts, so that
  // the softmax can wait for them and leave those parts in flight).
  auto mfma_block = [&](int j, int nt, bool fetch) {  // nt: tile whose DMA to issue, or -1
    if constexpr (mask_vec(MK)) {
      if (fetch) mf.issue_vec<mes>(mdesc, mrow + static_cast<uint32_t>(j * BN + 16 * h) * mes);
    } else if constexpr (MK != 0) {
      if (fetch) mf.issue<mes>(mdesc, mrow + static_cast<uint32_t>(j * BN + 4 * h) * mstep, mstep);
    }
    const char *kt = lds + (j % NS) * STAGE;
    const char *vt = lds + ((j + NS - 1) % NS) * STAGE + TILE_K;
    const DmaTile dt_next = dma_tile(nt);
    constexpr int FD = 2;  // fragment prefetch distance, in steps
    u32x4 kf[FD + 1], vf[FD + 1];
    auto load = [&](int i) {
      if (i < SKS) kf[i % (FD + 1)] = rdk.rows(kt, 0, i);
      if (i < PVS) vf[i % (FD + 1)] = rdv.cols(vt, i / PDT, i % PDT);
    };
    s = f32x16{};
    // Dropout: the Philox rounds of tile j's keep words (the softmax after
    // this block takes them) depend on no product, so they run among the
    // MFMA steps, a step's share after its MFMAs, where they execute while
    // the matrix pipe works; after the last tile's block they are not used.
    if constexpr (DR) ph = philox_pair_start(p.drop, drow + static_cast<uint32_t>(j * BN / 16));
#pragma unroll
    for (int i = 0; i < FD; ++i) load(i);
    // sched_barrier fences keep each step's reads FD steps ahead of its use.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < STEPS; ++i) {
      if (i < SKS) s = mfma32<T>(kf[i % (FD + 1)], qf[i], s);
      if (i < PVS) oacc[i % PDT] = mfma32<T>(vf[i % (FD + 1)], pb[i / PDT], oacc[i % PDT]);
      if (i + FD < STEPS) load(i + FD);
      if ((i & 1) && (i >> 1) < LPT) issue_part(dt_next, i >> 1);
      if constexpr (DR) philox_pair_rounds(ph, p.drop, 10 * i / STEPS, 10 * (i + 1) / STEPS);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  auto softmax = [&](int j, int nt) {
    const int kv0 = j * BN;
    float x[16];  // scores of this lane's query row; element i is key kv0 + crow(i, h)
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = s[i];
    if (j >= j_edge) {
      // Key kv0 + 4h + kc(i), kc a compile-time constant.
      const int lim = klim - kv0 - 4 * h;
      if constexpr (MK == 0) {
        unsigned kbits = ~0u;
        if (keymask) {
          const int key = kv0 + lane;
          const bool ok = key < p.Sk && kmask_b[static_cast<int64_t>(key) * p.mask.s3];
          kbits = static_cast<unsigned>(__ballot(ok) >> (4 * h));
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kc = 8 * (i >> 2) + (i & 3);
          const bool ok = (kc < lim) & (((kbits >> kc) & 1u) != 0);
          x[i] = ok ? x[i] : -INFINITY;
        }
      } else {
        wait_vm_n<LPT>();  // the mask loads; tile nt's parts stay in flight
        if constexpr (mask_vec(MK)) {
          mf.resolve_vec<mes>();
          mf.unpack<mes>(h);
        } else {
          mf.resolve();
        }
        mask_scores<MK>(x, mf, p.mask.dtype, -64, lim, sl);
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, x[i]);
    // the partner's max joins in one v_max3 (fmaxf would canonicalise both
    // values the permlane returns)
    const float mxr = half_swap_max3(mx);
    if (__ballot(mxr > thr) != 0ull) {
      const float m_new = fmaxf(m, mxr * slx);
      const float corr = m_new == -INFINITY ? 1.f : fast_exp2(m - m_new);
      m = m_new;
      thr = (m + kTau) * inv_slx;
      nbase = m == -INFINITY ? 0.f : -m;
      l *= corr;
#pragma unroll
      for (int dt = 0; dt < PDT; ++dt) oacc[dt] *= corr;
    }
    // Dropout: the denominator sums the undropped probabilities (the
    // reference normalises first, attention.py:139-144); PV takes P * mask.
    // Pair masks km[k]: 0xFFFF in the half of each kept word of elements 2k,
    // 2k + 1 (the order pack2 gives P), so P * mask is one AND per pair.  A
    // threshold of 65536 keeps nothing: zero multiplier and bits instead.
    uint32_t km[8];
    const bool none_kept = p.drop.thr > 65535u;
    if constexpr (DR) {
      uint64_t dw[4];
      philox_pair_rows(ph, dw);  // (rounds run in the MFMA block of tile j)
      const uint32_t thr2 = (p.drop.thr & 0xFFFFu) * 0x00010001u;
#pragma unroll
      for (int k = 0; k < 8; ++k)
        km[k] = keep_mask_pair(static_cast<uint32_t>(dw[k >> 1] >> (32 * (k & 1))), thr2);
      // keep bits for the backward: lane half h holds keys 8 g + 4 h + r.
      // One buffer store per tile, always (past the range, so dropped, for
      // half 1, rows past Sq and without a bits buffer): the end-of-tile wait
      // counts it and leaves it in flight, where a store it did not count
      // held each tile until the store, or a DMA part issued after the
      // previous tile's, had completed.
      {
        uint32_t bits = none_kept ? 0u : keep_bits16(km) << (4 * h);
        // lanes 0..31 take their partner's half (v_permlane32_swap exchanges
        // the upper half of its first register with the lower half of its
        // second: no LDS round trip)
        uint32_t mine = bits, other = bits;
        asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(mine), "+v"(other));
        bits |= other;
        // the tile's words: rows 0 .. sqp - 1 of key tile kv0 / BN
        const uintptr_t tbase =
            reinterpret_cast<uintptr_t>(p.drop.bits) +
            ((static_cast<uint64_t>(b) * p.Hq + hq) * p.drop.nkt + static_cast<uint64_t>(kv0 / BN)) *
                static_cast<uint64_t>(p.drop.sqp) * 4;
        const rsrc_t br = make_rsrc(reinterpret_cast<const void *>(tbase),
                                    p.drop.bits ? static_cast<uint32_t>(p.drop.sqp) * 4 : 0u);
        const uint32_t boff = (static_cast<uint32_t>(qrow) * 4) | (h == 0 && qrow < p.Sq ? 0u : 0x80000000u);
        __builtin_amdgcn_raw_buffer_store_b32(bits, br, static_cast<int>(boff), 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      float p0 = fast_exp2(fmaf(x[i], slx, nbase));
      float p1 = fast_exp2(fmaf(x[i + 1], slx, nbase));
      l += p0 + p1;  // fp32 sum of the unrounded probabilities, as the reference
      if constexpr (DR) {
        const float dsc = none_kept ? 0.f : p.drop.scale;
        pb[i >> 3][(i & 7) >> 1] = pack2<T>(p0 * dsc, p1 * dsc) & km[i >> 1];
      } else {
        pb[i >> 3][(i & 7) >> 1] = pack2<T>(p0, p1);
      }
    }
  };

  // Iteration j: issue tile j + PD, MFMA block j (PV of tile j - 1, S of tile
  // j), softmax of tile j, then wait for tile j + 1 and barrier (stage
  // (j + PD) % NS last held tile j - 2, read up to iteration j - 1).  Each
  // wave's work is one straight loop, so the accumulators stay in place;
  // iterations past the wave's last tile only keep the barrier count.
  auto next_dma = [&](int j) { return j + PD; };
  // (stored: the iteration issued a dropout keep-bit store after its DMA
  // parts, which may stay in flight)
  auto it_end = [&](auto stored) {
    wait_vm_n<(PD - 1) * LPT + (decltype(stored)::value ? 1 : 0)>();  // tile j + 1 has landed
    wait_lgkm0();
    phase_barrier();
  };
  int j = 0;
  if (w_tiles > 0) {
    pb[0] = pb[1] = u32x4{0, 0, 0, 0};
    for (; j < w_tiles; ++j) {
      mfma_block(j, next_dma(j), true);
      softmax(j, next_dma(j));
      it_end(std::bool_constant<DR>{});
    }
    mfma_block(j, next_dma(j), false);  // PV of the last tile
    it_end(std::false_type{});
    ++j;
  }
  for (; j <= n_tiles; ++j) {
    issue(next_dma(j));
    it_end(std::false_type{});
  }
  wait_vm_n<0>();  // the last (spare-block) loads, before the epilogue reuses the ring

  // RoPE with a rotated-query buffer: the rotated rows, for the backward's
  // dK/dV kernel (which reads Q tiles by DMA and cannot rotate them).
  if (p.rope.qrot && qrow < p.Sq) {
    T *qr = static_cast<T *>(p.rope.qrot) + ((static_cast<int64_t>(b) * p.Hq + hq) * p.Sq + qrow) * DK + 8 * h;
#pragma unroll
    for (int ks = 0; ks < SKS; ++ks) *reinterpret_cast<u32x4 *>(qr + 16 * ks) = qf[ks];
  }

  const float lt = xor32_sum(l);  // lanes c and c+32 share a query row
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  // O rows leave through LDS (free after the last barrier, all loads waited
  // for): each wave rounds its 32 rows into its own slice -- row r at r * 2D
  // bytes, 16-byte chunk q at q ^ (r % CPR), the XOR keeping the row writes
  // off one bank -- then reads back whole 16-byte chunks of rows, so the
  // global stores are coalesced.  Lane holds O^T[d = 32 dt + 8 g + 4 h + r][row c].
  constexpr int CPR = DV / 8;
  static_assert(NW * 32 * 2 * DV <= NS * STAGE, "output slices fit in the ring");
  static_assert(32 * CPR % 64 == 0, "store chunks split evenly over the lanes");
  char *slice = lds + w * 32 * 2 * DV;
#pragma unroll
  for (int dt = 0; dt < PDT; ++dt) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int off = c * 2 * DV + (((4 * dt + g) ^ (c % CPR)) * 16) + 8 * h;
      *reinterpret_cast<u32x2 *>(slice + off) =
          u32x2{pack2<T>(oacc[dt][g * 4 + 0] * inv, oacc[dt][g * 4 + 1] * inv),
                pack2<T>(oacc[dt][g * 4 + 2] * inv, oacc[dt][g * 4 + 3] * inv)};
    }
  }
  T *ob = static_cast<T *>(const_cast<void *>(a.o.data)) + b * a.o.s0 + hq * a.o.s1;
  // every chunk read back before the first store (a read inside each store's
  // row guard waits out one LDS latency per store)
  u32x4 vr[32 * CPR / 64];
#pragma unroll
  for (int u = 0; u < 32 * CPR / 64; ++u) {
    const int idx = u * 64 + lane, r = idx / CPR, q = idx % CPR;
    vr[u] = *reinterpret_cast<const u32x4 *>(slice + r * 2 * DV + ((q ^ (r % CPR)) * 16));
  }
#pragma unroll
  for (int u = 0; u < 32 * CPR / 64; ++u) {
    const int idx = u * 64 + lane, r = idx / CPR, q = idx % CPR;
    if (qw + r < p.Sq) *reinterpret_cast<u32x4 *>(ob + static_cast<int64_t>(qw + r) * a.o.s2 + q * 8) = vr[u];
  }
  if (a.lse && h == 0 && qrow < p.Sq)
    a.lse[(static_cast<int64_t>(b) * p.Hq + hq) * p.Sq + qrow] =
        lt > 0.f ? (m + log2f(lt)) * kLn2 : -INFINITY;
}

template <typename T, int DK, int DV, bool DR>
void launch_dr(const FwdArgs &a, int mk, hipStream_t st) {
  const dim3 g(a.total), blk(NT);
  switch (mk) {
    case 1: fwd_kernel<T, DK, DV, 1, DR><<<g, blk, 0, st>>>(a); break;
    case 2: fwd_kernel<T, DK, DV, 2, DR><<<g, blk, 0, st>>>(a); break;
    case 3: fwd_kernel<T, DK, DV, 3, DR><<<g, blk, 0, st>>>(a); break;
    case 4: fwd_kernel<T, DK, DV, 4, DR><<<g, blk, 0, st>>>(a); break;
    case 5: fwd_kernel<T, DK, DV, 5, DR><<<g, blk, 0, st>>>(a); break;
    case 6: fwd_kernel<T, DK, DV, 6, DR><<<g, blk, 0, st>>>(a); break;
    default: fwd_kernel<T, DK, DV, 0, DR><<<g, blk, 0, st>>>(a); break;
  }
}

template <typename T, int DK, int DV>
void launch_dims(const FwdArgs &a, hipStream_t st) {
  const int mk = mfma_mask_mode_vec(a.p);
  if (a.p.drop.on) launch_dr<T, DK, DV, true>(a, mk, st);
  else launch_dr<T, DK, DV, false>(a, mk, st);
}

template <typename T>
hipError_t launch(const FwdArgs &a, hipStream_t st) {
  const Problem &p = a.p;
  const int mk = mfma_mask_mode(p);
  Probe pr_(p.drop.on ? "fwd_mfma_dropout" : (mk ? "fwd_mfma_masked" : "fwd_mfma"), st);
  if (p.Dqk == 128 && p.Dv == 128) launch_dims<T, 128, 128>(a, st);
  else if (p.Dqk == 64 && p.Dv == 64) launch_dims<T, 64, 64>(a, st);
  else if (p.Dqk == 32) launch_dims<T, 32, 32>(a, st);
  else if (p.Dqk == 128) launch_dims<T, 128, 64>(a, st);
  else launch_dims<T, 64, 128>(a, st);
  return hipGetLastError();
}

}  // namespace

bool mfma_supported(const Problem &p, int dtype) {
  if (dtype != TSATTN_F16 && dtype != TSATTN_BF16) return false;
  // head dims 64 / 128 each, or 32 for both
  const bool d32 = p.Dqk == 32 && p.Dv == 32;
  if (!d32 && ((p.Dqk != 64 && p.Dqk != 128) || (p.Dv != 64 && p.Dv != 128))) return false;
  if (!(p.scale > 0.0)) return false;
  // the backward reads each (b, h) slice of the dropout keep bits with 32-bit offsets
  if (p.drop.on && static_cast<int64_t>((p.Sk + 31) / 32) * ((p.Sq + 3) / 4 * 4) * 4 >= (int64_t(1) << 31))
    return false;
  if (p.mask.kind == TSATTN_MASK_ADDITIVE && p.mask.dtype != TSATTN_F32 &&
      p.mask.dtype != TSATTN_F16 && p.mask.dtype != TSATTN_BF16)
    return false;
  const int mk = mfma_mask_mode(p);
  if (mk == 0) return true;
  // General masks are read with 32-bit byte offsets inside each (b, h) slice,
  // rows and keys padded to whole tiles.
  const MaskDesc &m = p.mask;
  if (m.s0 < 0 || m.s1 < 0 || m.s2 < 0 || m.s3 < 0) return false;
  const int64_t es = mk == 1 ? 1 : (mk == 2 ? 4 : 2);
  return ((p.Sq + 128) * m.s2 + (p.Sk + 128) * m.s3 + 1) * es < (int64_t(1) << 31);
}

hipError_t launch_mfma_forward(const Problem &p, int dtype, View q, View k, View v, View o,
                               float *lse, hipStream_t st) {
  FwdArgs a{p, q, k, v, o, lse, static_cast<float>(p.scale) * kLog2e, (p.Sq + BM - 1) / BM, 0};
  a.total = a.n_qblocks * p.Hq * p.B;
  return dtype == TSATTN_BF16 ? launch<bf16>(a, st) : launch<f16>(a, st);
}

}  // namespace tsattn
