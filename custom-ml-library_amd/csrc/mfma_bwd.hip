// Attention backward for gfx950 with MFMA 32x32x16 (f16/bf16 in, fp32
// accumulate).  Follows the reference's streaming VJP (src/tensorsmith/nn/
// attention.py:220-247):
//   delta_i = sum_d dO_id O_id                     (dq_kernel prologue)
//   P_ij = exp(S_ij - LSE_i), dS_ij = P_ij (dP_ij - delta_i), dP = dO V^T
//   dQ = scale dS K                                (dq_kernel, runs first)
//   dV = P^T dO, dK = scale dS^T Q                 (dkdv_kernel)
// dK/dV and dQ are produced by two kernels that each own their output tile,
// so every gradient element is written exactly once: no atomics, bitwise
// deterministic results (checkpoint recompute reproduces them exactly).
// The dK/dV kernel sums the query heads of a GQA group itself (:245-247).
//
// Tiles reach LDS by direct buffer loads into swizzled row-major layouts;
// transposed operands (Q^T, dO^T, K^T) come from LDS transpose reads.
//
// Dropout (template DR): both kernels read the keep mask as bits (one 32-bit
// word per query row and 32-key tile, DropDesc::bits) -- the forward's, or
// drawn from the problem's Philox stream by dropout_bits_kernel first:
// dV = (P * mask)^T dO and dS = P (dP * mask - delta) (attention.py:210-217;
// delta = rowsum(dO O) already holds the mask through O).  The dQ kernel
// fetches its row's word with each key tile, the dK/dV kernel stages the 32
// words of its key tile through the LDS ring with the Q / dO tiles.
//
// RoPE (Problem::rope, R > 0): the dQ prologue rotates the query fragments
// as the forward did; the dQ and dK epilogues apply the inverse rotation to
// the rounded gradients, so they are those of the unrotated queries and keys
// (bit-identical to a separate inverse tsattn_rope).
//
// Masks (template MK) as in the forward: a key mask reduced to lengths, or a
// general boolean / additive mask read per (query row, key) on every tile
// (additive: P = exp(S scale + mask - LSE)).
#include <type_traits>

#include "mfma_common.h"
#include "rope_math.h"

namespace tsattn {
namespace {

constexpr int NT = 256;
constexpr int NW = NT / 64;

struct BwdArgs {
  Problem p;
  View q, k, v, o, dout, dq, dk, dv;
  // The queries the dK/dV kernel reads: q, or with RoPE folded in the rotated
  // rows the dQ kernel stages in the workspace ([B, Hq, Sq, D] contiguous).
  View qk;
  const float *lse;
  // Row values the dQ kernel writes for the dK/dV kernel: [rows] nd = -delta,
  // then [rows] nl = -safe(lse) / scale, safe(lse) = isfinite(lse) ? lse : 0
  // (the reference's safe_lse, attention.py:231).  Stored negated so the
  // dK/dV kernel starts its S and dP accumulators from them:
  // S + nl = (S scale - lse) / scale and dP + nd = dP - delta (with dropout
  // both absorb the mask value, store_row_values).
  float *delta;
  float sl;      // scale * log2(e)
  float scale;   // final gradient scale
  // Stored dS (NULL: the dQ kernel recomputes S and dP itself).  Per (b, q
  // head) a slice of ds_slice tiles of 32 query rows x 32 keys, query tile qt
  // owning the ds_row_len(qt) tiles from ds_row_start(qt) on (key tiles 0 ..,
  // those of every 128-key block the dK/dV kernel visits for it); tile (qt,
  // kt) at byte (bh ds_slice + ds_row_start(qt) + kt) * 2 KiB, as the dK/dV
  // kernel's lanes hold it: dS[q][k] (q, k within the tile, q = 4 m + r) at
  // (m / 4) KiB + (m % 2) 512 + 16 (k ^ 4 (m % 2) ^ 8 (m / 4)) + ((m / 2) % 2) 8
  // + 2 r.  ds_tri: causal with Sq = Sk and no offset, rows packed (row qt
  // holds 4 (qt / 4 + 1) tiles), so the reads sweep the slice densely; else
  // rows of ds_nkt tiles.
  char *ds;
  int ds_nkt, ds_tri;
  int64_t ds_slice;
  // The KV-head groups (b, kv head), g = b Hkv + hk, this launch covers:
  // [g0, g0 + ng).  With stored dS the backward runs in chunks of groups
  // when the dS of all of them exceeds the region's cap: the region holds
  // the slices of one chunk's query heads (slice index (g - g0) rep + r).
  int g0, ng;
};

// Start of query tile qt's dS row within its slice, in tiles.
__host__ __device__ __forceinline__ int64_t ds_row_start(int tri, int nkt, int qt) {
  if (!tri) return static_cast<int64_t>(qt) * nkt;
  const int64_t g = qt >> 2, r = qt & 3;  // rows 4 g .. 4 g + 3 hold 4 (g + 1) tiles each
  return (g + 1) * (8 * g + 4 * r);
}

constexpr int DS_TILE = 2048;  // bytes of one stored dS tile

// a if B, else c (of another type).
template <bool B, typename X, typename Y>
__device__ __forceinline__ const auto &pick(const X &a, const Y &c) {
  if constexpr (B) return a;
  else return c;
}
constexpr int kStreamStore = 18;  // buffer store cache policy: sc1 (16) | nt (2)

template <typename T>
__device__ __forceinline__ T *mut(View v) {
  return static_cast<T *>(const_cast<void *>(v.data));
}
template <typename T>
__device__ __forceinline__ const T *head_ptr(View v, int b, int h) {
  return static_cast<const T *>(v.data) + b * v.s0 + h * v.s1;
}

// The dK/dV kernel's row values of query row `row`: nd = -delta at [row], nl =
// -lse / scale at [rows + row] (0 for a row that sees no key), so that the
// kernel's S accumulator started from nl gives P = exp2(acc sl).  With
// dropout (mask value m = 1 / (1 - p) where kept) they absorb m: nl + ln(m) /
// scale gives P m, and nd / m gives dS = P m (dP + nd / m) = P (m dP - delta)
// for a kept element and P m (nd / m) = -P delta for a dropped one.
__device__ __forceinline__ void store_row_values(const BwdArgs &a, int64_t rows, int64_t row,
                                                 float nd, float lse) {
  const bool finite = isfinite(lse);
  if (a.p.drop.on) {
    a.delta[row] = nd / a.p.drop.scale;
    a.delta[rows + row] = finite ? (logf(a.p.drop.scale) - lse) / a.scale : 0.f;
  } else {
    a.delta[row] = nd;
    a.delta[rows + row] = finite ? -lse / a.scale : 0.f;
  }
}

// ---------------------------------------------------------------------------
// dK / dV: one workgroup = 128 keys of one (b, kv head), 4 wavefronts, two
// workgroups per CU.  Wave w owns keys k0 + 32 w .. + 31: it holds their K
// and V row fragments in registers for the workgroup's life, next to its
// dK^T / dV^T accumulators, so K and V take no LDS and no wave shares an
// output row.  Query tiles of 32 rows -- Q, dO and their nl / nd row values,
// for every query head of the GQA group -- stream through a 3-stage LDS ring
// by DMA loads issued two tiles ahead (between the first MFMA steps), one
// fence-free barrier per tile.  Per tile a wave computes S = Q K^T and
// dP = dO V^T (16 MFMAs, Q / dO row fragments), P and dS on the VALU, then
// dV^T += dO^T P and dK^T += Q^T dS (16 MFMAs, column fragments).  The two
// workgroups of a CU are not tied by barriers, so one's VALU phase overlaps
// the other's MFMA phases, and each hides the other's prologue and epilogue.
// ---------------------------------------------------------------------------
constexpr int KB = 128;   // keys per workgroup
constexpr int QT = 32;    // query rows per tile
constexpr int KV_NS = 3;  // Q / dO ring stages
constexpr int KV_PD = 2;  // tiles in flight
#ifndef DKDV_FD
#define DKDV_FD 1
#endif

// Workgroups per CU: two, except the general-mask kernel at D = 128, whose
// mask registers do not fit beside the two-workgroup register budget; alone
// on its CU it has the accumulation registers as well.  (The dropout kernel
// at D = 128 spills 13 VGPRs at two per CU -- fragment reloads each tile --
// and is still faster than alone on its CU: 0.88 against 1.07 ms at B16 H16
// S2048 D128.)
// Masks the dK/dV kernel stages through its LDS ring (modes 4 and 6: boolean
// or 16-bit, key-contiguous with 16-byte aligned rows) hold no registers.
constexpr bool mask_staged(int MK) { return MK == 4 || MK == 6; }

template <int DK, int DV, int MK, bool DR>
constexpr int dkdv_wg_per_cu() {
  return (MK != 0 && !mask_staged(MK)) && (DK > 64 || DV > 64) ? 1 : 2;
}

// DK = head dim of q / k (and dK), DV = of v / dO (and dV); each 64 or 128.
template <typename T, int DK, int DV, int MK, bool DR>
__global__ __launch_bounds__(NT, (dkdv_wg_per_cu<DK, DV, MK, DR>())) void dkdv_kernel(BwdArgs a) {
  constexpr int TILE_Q = QT * DK * 2, TILE_G = QT * DV * 2;  // bytes of a Q / dO tile
  // A staged mask: the tile's [QT rows][KB keys] elements, row-major.
  constexpr bool MSTAGE = mask_staged(MK);
  constexpr int MES = MSTAGE ? mask_bytes<MK>() : 0;
  constexpr int MROW = KB * MES, MTILE = QT * MROW;  // bytes per mask row / tile
  constexpr int MPARTS = MTILE / 1024 / NW;          // mask DMA loads per wave per tile
  constexpr int MOFF = TILE_Q + TILE_G + 256;
  // Dropout: each wave's 32 keep-bit words (rows q0 .. q0 + 31 of its key tile)
  constexpr int BOFF = MOFF + MTILE, BSZ = DR ? NW * 128 : 0;
  // Q | dO | nl (QT floats) | nd (QT floats) | mask tile | keep bits
  constexpr int STAGE_B = TILE_Q + TILE_G + 256 + MTILE + BSZ;
  // 1 KiB DMA blocks of a Q / dO tile; wave w loads blocks w, w + NW, ...
  // (Q blocks, then dO blocks): a compile-time split at head dims 64 / 128,
  // and at head dim 32 (two blocks per tile) waves 0, 1 load Q, 2, 3 dO.
  constexpr int QBLK = TILE_Q / 1024, GBLK = TILE_G / 1024;
  constexpr bool EVEN = QBLK % NW == 0 && GBLK % NW == 0;
  constexpr int QPARTS = QBLK / NW, GPARTS = GBLK / NW;
  constexpr int LPT = (QBLK + GBLK + NW - 1) / NW;  // Q + dO DMA loads per wave per tile
  constexpr int SKQ = DK / 16, SKV = DV / 16;     // k-steps of S (over DK) and dP (over DV)
  constexpr int PDK = DK / 32, PDV = DV / 32;     // 32-row blocks of dK^T / dV^T
  constexpr int STEPS = SKQ > SKV ? SKQ : SKV;    // MFMA steps of each block
  constexpr int QGQ = DK / 32, QGG = DV / 32;     // 4-chunk groups per Q / dO row
  constexpr int DMAX = DK > DV ? DK : DV;
  static_assert(EVEN ? (QPARTS >= 1 && GPARTS >= 1 && LPT == QPARTS + GPARTS)
                     : (QBLK + GBLK == NW && LPT == 1 && DK == 32 && DV == 32),
                "tile loads must split over the waves");
  static_assert(2 * LPT <= STEPS, "one tile DMA part per two MFMA steps");
  static_assert(STAGE_B % 256 == 0, "stages keep the bank mapping of the blocked layout");
  // Q / dO ring, then a 1 KiB block that DMA parts of tiles past the last
  // one land in (nothing reads it)
  // The prologue first stages the workgroup's K and V rows (128 keys each)
  // in the same bytes.
  constexpr int KV_STAGE = KB * (DK + DV) * 2;
  constexpr int RING_B = KV_NS * STAGE_B + 1024 > KV_STAGE ? KV_NS * STAGE_B + 1024 : KV_STAGE;
  __shared__ __attribute__((aligned(1024))) char ring[RING_B];

  const Problem &p = a.p;
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 31, h = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_kb = (p.Sk + KB - 1) / KB;
  const int total = n_kb * a.ng;
  const int logical = xcd_remap(blockIdx.x, total);
  int bhc, kb;  // early key blocks see the most queries: run them first
  heavy_first(logical, n_kb, a.ng, 32 * dkdv_wg_per_cu<DK, DV, MK, DR>(), bhc, kb);  // slots per XCD
  const int bh = a.g0 + bhc;  // group (b, kv head); bhc: its index within the chunk
  const int b = bh / p.Hkv, hk = bh - b * p.Hkv;
  const int k0 = kb * KB, kw = k0 + 32 * w, key = kw + c;
  const int kv_end = kv_end_for(p, b);
  const bool keymask =
      MK == 0 && p.mask.kind == TSATTN_MASK_BOOL && !(p.kv_prefix && p.kv_prefix[b]);
  const bool key_live = key < kv_end &&
                        (!keymask || static_cast<const uint8_t *>(p.mask.data)
                                         [b * p.mask.s0 + static_cast<int64_t>(key) * p.mask.s3]);
  const int64_t rows = static_cast<int64_t>(p.B) * p.Hq * p.Sq;
  const bool causal = p.causal != 0;
  // Causal bounds in 32 bits: this lane's key - offset, and the first tile
  // row at which every key of the wave is visible (q0 >= q_diag: no mask).
  const int64_t kd64 = static_cast<int64_t>(key) - p.offset;
  const int kdiff = kd64 < -(1 << 30) ? -(1 << 30) : static_cast<int>(kd64);
  const int64_t qd64 = static_cast<int64_t>(kw) + 31 - p.offset;
  const int q_diag = qd64 < -1 ? -1 : static_cast<int>(qd64);

  // Query tiles: only rows that can see a key of this block (causal).
  int q_start = 0;
  if (causal) {
    const int64_t s0 = static_cast<int64_t>(k0) - p.offset;
    q_start = s0 <= 0 ? 0 : static_cast<int>(s0 < p.Sq ? s0 : p.Sq);
    q_start = (q_start / QT) * QT;
  }
  // wave-uniform by construction; readfirstlane keeps them in SGPRs
  const int n_qt = __builtin_amdgcn_readfirstlane(k0 < kv_end ? (p.Sq - q_start + QT - 1) / QT : 0);
  const int n_iter = __builtin_amdgcn_readfirstlane(n_qt * p.rep);

  const uint32_t qs_b = static_cast<uint32_t>(a.qk.s2) * 2, gs_b = static_cast<uint32_t>(a.dout.s2) * 2;
  const uint32_t ks_b = static_cast<uint32_t>(a.k.s2) * 2, vs_b = static_cast<uint32_t>(a.v.s2) * 2;
  const uint32_t ring0 = lds_addr(ring);
  // Blocked layout: block n = (n / QG, n % QG); its lane l fetches row
  // 16 (n / QG) + l / 4, chunk 4 (n % QG) + ((l % 4) ^ ((l / 16) % 4)).  A
  // wave's blocks are w, w + 4, ..., all with n % QG = w % QG.
  const uint32_t swz_chunk = (lane & 3) ^ ((lane >> 4) & 3);
  const uint32_t lrow = lane >> 2;
  // Tile itn is query tile qi = itn % n_qt of query head hk rep + r, r =
  // itn / n_qt.  Two cursors walk that order without a division or a 64-bit
  // product per tile: the issue cursor (the tile whose DMA loads go out, KV_PD
  // tiles ahead) and the read cursor (the tile being computed).  Per tile a
  // cursor moves its ring stage and its row offsets on by one tile; the move
  // to the next query head, once per n_qt tiles, is a scalar branch that
  // rebuilds the head's buffer descriptors.  Past the last head the issue
  // cursor's descriptors are empty, so the loads issued past the last tile
  // read zeros without touching memory, into the ring stages of tiles already
  // consumed: every iteration issues the same loads, the waits are constants
  // and no branch guards an issue.
  //
  // The dropout kernels keep a per-tile form instead (TileIdx / TileDma
  // below): at D = 128 their registers are full, and the cursors' branches
  // and held descriptors move their spills into the loop (an accumulator
  // block reloaded every tile, 1.9x the dK/dV time).
  const uint64_t qstep = static_cast<uint64_t>(a.qk.s1) * 2, gstep = static_cast<uint64_t>(a.dout.s1) * 2;
  const uint64_t rstep = static_cast<uint64_t>(p.Sq) * 4;
  // With stored dS, da is the byte offset of the tile's head slice.
  const uint64_t dwrap = static_cast<uint64_t>(a.ds_slice) * DS_TILE;
  const uint32_t q_bytes = static_cast<uint32_t>(p.Sq) * qs_b, g_bytes = static_cast<uint32_t>(p.Sq) * gs_b;
  const uint32_t last_stage = ring0 + (KV_NS - 1) * STAGE_B;
  // A 1 KiB block past the ring that nothing reads (dropout kernels: the
  // loads past the last tile; every kernel: the prologue's stand-ins for dS
  // stores).
  const uint32_t spare = ring0 + KV_NS * STAGE_B;
  // nl (waves 0, 2) / nd (waves 1, 3) rows of the group's first query head;
  // waves 2, 3 load the same rows as 0, 1 (the same bytes to the same place;
  // dropout kernels: into the spare block)
  const float *rowv =
      a.delta + (static_cast<int64_t>(b) * p.Hq + hk * p.rep) * p.Sq + ((DR ? w : w & 1) == 0 ? rows : 0);
  struct IssueCur {
    int qi, r;
    uint32_t st;          // LDS address of the tile's ring stage
    uint32_t qo, go, ro;  // byte offsets of the tile's first row in the head's Q, dO, row values
    uint32_t far;         // 0 for a real tile, 2^31 past the last head
    uint64_t qa, ga, ra;  // the head's Q, dO and row-value slices
    u32x4 qdesc, gdesc, rdesc;
  };
  auto set_head = [&](IssueCur &c) {
    const bool real = c.r < p.rep;
    c.far = real ? 0u : 0x80000000u;
    c.qo = static_cast<uint32_t>(q_start) * qs_b;
    c.go = static_cast<uint32_t>(q_start) * gs_b;
    c.ro = static_cast<uint32_t>(q_start) * 4;
    c.qdesc = make_desc(reinterpret_cast<const void *>(c.qa), real ? q_bytes : 0u);
    c.gdesc = make_desc(reinterpret_cast<const void *>(c.ga), real ? g_bytes : 0u);
    c.rdesc = make_desc(reinterpret_cast<const void *>(c.ra), real ? static_cast<uint32_t>(p.Sq) * 4 : 0u);
  };
  auto issue_next = [&](IssueCur &c) {
    c.st = c.st == last_stage ? ring0 : c.st + STAGE_B;
    c.qo += QT * qs_b;
    c.go += QT * gs_b;
    c.ro += QT * 4;
    if (++c.qi == n_qt) {
      asm volatile("");  // (a branch taken once per head, not selects on every tile)
      c.qi = 0;
      ++c.r;
      c.qa += qstep;
      c.ga += gstep;
      c.ra += rstep;
      set_head(c);
    }
  };
  // Dropout kernels: TileIdx walks the order with selects, carrying the
  // head's slice addresses; TileDma holds one tile's load arguments, its
  // stage addressed from the spare block and masked by keep (all ones for a
  // real tile, else 0: tiles past the last one land in the spare block).
  struct TileIdx {
    int itn, r, qi;
    uint64_t qa, ga, ra, da;
  };
  auto tile_next = [&](TileIdx t) {
    ++t.itn;
    const bool wrap = ++t.qi == n_qt;
    t.qi = wrap ? 0 : t.qi;
    t.r += wrap ? 1 : 0;
    t.qa += wrap ? qstep : 0;
    t.ga += wrap ? gstep : 0;
    t.ra += wrap ? rstep : 0;
    t.da += wrap ? dwrap : 0;
    return t;
  };
  struct TileDma {
    uint32_t st, keep, far;
    int q0, hq;
    u32x4 qdesc, gdesc;
    uint64_t ra;
  };
  auto tile_dma = [&](TileIdx x) {
    TileDma t;
    t.hq = hk * p.rep + x.r;
    t.q0 = q_start + x.qi * QT;
    t.keep = ~static_cast<uint32_t>((n_iter - 1 - x.itn) >> 31);  // sign fill
    t.far = ~t.keep & 0x80000000u;
    t.st = (ring0 + (x.itn % KV_NS) * STAGE_B - spare) & t.keep;
    t.qdesc = make_desc(reinterpret_cast<const void *>(x.qa), q_bytes);
    t.gdesc = make_desc(reinterpret_cast<const void *>(x.ga), g_bytes);
    t.ra = x.ra;
    return t;
  };
  // A tile's query head, first row and the LDS address of byte `off` of its
  // stage, from either form.
  auto t_hq = [&](const auto &t) {
    if constexpr (DR) return t.hq;
    else return hk * p.rep + t.r;
  };
  auto t_q0 = [&](const auto &t) {
    if constexpr (DR) return t.q0;
    else return q_start + t.qi * QT;
  };
  auto t_lds = [&](const auto &t, uint32_t off) {
    if constexpr (DR) return spare + t.st + (off & t.keep);
    else return t.st + off;
  };
  // DMA of a tile into its ring stage, in LPT + 1 parts: part u < LPT is
  // this wave's u-th Q / dO block, part LPT the nl / nd rows.
  // Parts u < QPARTS are Q blocks, the rest dO blocks (a compile-time split).
  const uint32_t qvoff = lrow * qs_b + (4 * (w % QGQ) + swz_chunk) * 16;
  const uint32_t gvoff = lrow * gs_b + (4 * (w % QGG) + swz_chunk) * 16;
  auto issue_q = [&](const auto &t, int n) {
    if constexpr (DR)
      dma16(t.qdesc, t_lds(t, n * 1024), qvoff, (static_cast<uint32_t>(t.q0 + 16 * (n / QGQ)) * qs_b) | t.far);
    else
      dma16(t.qdesc, t_lds(t, n * 1024), qvoff, t.qo + static_cast<uint32_t>(16 * (n / QGQ)) * qs_b);
  };
  auto issue_g = [&](const auto &t, int n) {
    if constexpr (DR)
      dma16(t.gdesc, t_lds(t, TILE_Q + n * 1024), gvoff, (static_cast<uint32_t>(t.q0 + 16 * (n / QGG)) * gs_b) | t.far);
    else
      dma16(t.gdesc, t_lds(t, TILE_Q + n * 1024), gvoff, t.go + static_cast<uint32_t>(16 * (n / QGG)) * gs_b);
  };
  auto issue_part = [&](const auto &t, int u) {
    if (u < LPT) {
      if constexpr (EVEN) {
        if (u < QPARTS) issue_q(t, w + NW * u);
        else issue_g(t, w + NW * (u - QPARTS));
      } else {
        if (w < QBLK) issue_q(t, w);  // (w is wave-uniform: a scalar branch)
        else issue_g(t, w - QBLK);
      }
    } else if constexpr (DR) {
      const u32x4 rdesc = make_desc(reinterpret_cast<const void *>(t.ra), static_cast<uint32_t>(p.Sq) * 4);
      // lane * 16, recomputed here rather than held in a register all loop
      uint32_t loff;
      asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0\n\t"
                   "v_lshlrev_b32 %0, 4, %0"
                   : "=v"(loff));
      const uint32_t mine = w < 2 ? t.keep : 0u;  // waves 2, 3: the spare block
      if (lane < QT / 4)
        dma16(rdesc, spare + (t.st & mine) + ((TILE_Q + TILE_G + w * QT * 4) & mine), loff,
              (static_cast<uint32_t>(t.q0) * 4) | (~mine & 0x80000000u));
    } else {
      uint32_t loff;
      asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0\n\t"
                   "v_lshlrev_b32 %0, 4, %0"
                   : "=v"(loff));
      if (lane < QT / 4) dma16(t.rdesc, t.st + TILE_Q + TILE_G + (w & 1) * QT * 4, loff, t.ro);
    }
  };
  // Staged mask: 1 KiB block n = w + NW u of the tile holds rows
  // n * 1024 / MROW ..; lane l fetches 16 bytes at byte 16 l of the block.
  // The lane's offset is recomputed at each issue (no register held all loop:
  // the two-workgroup budget is full).
  auto issue_mask = [&](const auto &t) {
    if constexpr (MSTAGE) {
      const uint32_t ms2 = static_cast<uint32_t>(p.mask.s2 * MES);  // bytes between mask rows
      uint32_t l16;
      asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0\n\t"
                   "v_lshlrev_b32 %0, 4, %0"
                   : "=v"(l16));
      const uint32_t mvoff = (l16 / MROW) * ms2 + l16 % MROW;
      const int64_t extent = ((p.Sq - 1) * p.mask.s2 + (p.Sk - 1) * p.mask.s3 + 1) * MES;
      const u32x4 mdesc = make_desc(
          static_cast<const char *>(p.mask.data) + (b * p.mask.s0 + t_hq(t) * p.mask.s1) * MES,
          static_cast<uint32_t>(extent));
#pragma unroll
      for (int u = 0; u < MPARTS; ++u) {
        const int n = w + NW * u;
        dma16(mdesc, t_lds(t, MOFF + n * 1024), mvoff,
              (static_cast<uint32_t>(t_q0(t) + n * (1024 / MROW)) * ms2 +
               static_cast<uint32_t>(k0 * MES)) | t.far);
      }
    }
  };
  // Dropout: this wave's 32 keep-bit words (key tile kb * 4 + w, rows q0 ..
  // q0 + 31) as one 8-lane DMA part; past the slice they read as zero.
  auto issue_bits = [&](const auto &t) {
    if constexpr (DR) {
      const DropDesc &d = p.drop;
      const u32x4 bdesc = make_desc(d.bits + (static_cast<int64_t>(b) * p.Hq + t.hq) * d.nkt * d.sqp,
                                    static_cast<uint32_t>(d.nkt * d.sqp * 4));
      uint32_t loff;
      asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0\n\t"
                   "v_lshlrev_b32 %0, 4, %0"
                   : "=v"(loff));
      if (lane < 8)
        dma16(bdesc, spare + t.st + ((BOFF + w * 128) & t.keep), loff,
              ((static_cast<uint32_t>(kb * (KB / 32) + w) * d.sqp + t.q0) * 4) | t.far);
    }
  };
  auto issue = [&](const auto &t) {
#pragma unroll
    for (int u = 0; u <= LPT; ++u) issue_part(t, u);
    issue_mask(t);
    issue_bits(t);
  };
  // DMA loads per wave per tile; a wave leaves those of the (KV_PD - 1) later
  // tiles already issued in flight once a tile has landed.
  constexpr int PARTS = LPT + 1 + MPARTS + (DR ? 1 : 0);

  const TileReader<T, DK> rdq(lane);
  const TileReader<T, DV> rdg(lane);
  // This wave's K / V row fragments (B operands of S = Q K^T, dP = dO V^T):
  // lane (c, h) holds row key, columns 16 i + 8 h .. +7.  Keys past the cache
  // end read as zeros.  They come through LDS: the workgroup's 128 K rows
  // and 128 V rows land there by DMA in the Q / dO tiles' blocked layout
  // (as one 128-row tile each; wave w loads its blocks w, w + 4, ..., whole
  // 128-byte lines, eight rows per instruction), then each wave reads its
  // 32 rows' fragments.  Loaded straight into registers instead, every
  // fragment instruction touches 32 rows, and the address unit takes 5 us
  // per workgroup to issue them.
  u32x4 kf[SKQ], vf[SKV];
  {
    const u32x4 kdesc = make_desc(head_ptr<T>(a.k, b, hk), static_cast<uint32_t>(kv_end) * ks_b);
    const u32x4 vdesc = make_desc(head_ptr<T>(a.v, b, hk), static_cast<uint32_t>(kv_end) * vs_b);
    const uint32_t kvoff = lrow * ks_b + (4 * (w % QGQ) + swz_chunk) * 16;
    const uint32_t vvoff = lrow * vs_b + (4 * (w % QGG) + swz_chunk) * 16;
    const uint32_t vst = ring0 + KB * DK * 2;
#pragma unroll
    for (int u = 0; u < KB / 16 * QGQ / NW; ++u) {
      const int n = w + NW * u;  // block (16 rows (n / QGQ), chunk group n % QGQ = w % QGQ)
      dma16(kdesc, ring0 + n * 1024, kvoff, static_cast<uint32_t>(k0 + 16 * (n / QGQ)) * ks_b);
    }
#pragma unroll
    for (int u = 0; u < KB / 16 * QGG / NW; ++u) {
      const int n = w + NW * u;
      dma16(vdesc, vst + n * 1024, vvoff, static_cast<uint32_t>(k0 + 16 * (n / QGG)) * vs_b);
    }
    wait_vm_n<0>();
    __syncthreads();
#pragma unroll
    for (int i = 0; i < STEPS; ++i) {
      if (i < SKQ) kf[i] = rdq.rows(ring, w, i);
      if (i < SKV) vf[i] = rdg.rows(ring + KB * DK * 2, w, i);
    }
    // every wave's reads done before the ring takes the first Q / dO tiles
    wait_lgkm0();
    __syncthreads();
  }

  f32x16 dk_acc[PDK], dv_acc[PDV];
#pragma unroll
  for (int dt = 0; dt < (PDK > PDV ? PDK : PDV); ++dt) {
    if (dt < PDK) dk_acc[dt] = f32x16{};
    if (dt < PDV) dv_acc[dt] = f32x16{};
  }
  const float sl = a.sl;

  // No zeroing: every LDS byte the loop reads is written by a DMA load first
  // (lanes past a buffer's range write zeros).
  IssueCur icur;
  icur.qi = 0;
  icur.r = n_qt > 0 ? 0 : p.rep;  // no tile at all: empty descriptors from the start
  icur.st = ring0;
  icur.qa = reinterpret_cast<uint64_t>(head_ptr<T>(a.qk, b, hk * p.rep));
  icur.ga = reinterpret_cast<uint64_t>(head_ptr<T>(a.dout, b, hk * p.rep));
  icur.ra = reinterpret_cast<uint64_t>(rowv);
  const TileIdx first{0, 0, 0, icur.qa, icur.ga, icur.ra, static_cast<uint64_t>(bhc) * p.rep * dwrap};
  TileIdx nxt_idx = first;
  if constexpr (DR) {
    for (int t = 0; t < KV_PD; ++t) {
      issue(tile_dma(nxt_idx));
      nxt_idx = tile_next(nxt_idx);
    }
  } else {
    set_head(icur);
    for (int t = 0; t < KV_PD; ++t) {
      issue(icur);
      issue_next(icur);
    }
  }
  wait_vm_n<(KV_PD - 1) * PARTS>();
#pragma unroll
  for (int i = 0; i < STEPS; ++i) {
    if (i < SKQ && i < SKV) asm volatile("" : "+v"(kf[i]), "+v"(vf[i]));
    else if (i < SKQ) asm volatile("" : "+v"(kf[i]));
    else asm volatile("" : "+v"(vf[i]));
  }
  if (a.ds) {
    // two loads past the range (zeros into the spare block, no memory
    // access) in place of a previous tile's two dS stores: the loop's waits
    // then count the same on every tile
    dma16(make_desc(a.ds, 0), spare, qvoff, 0x80000000u);
    dma16(make_desc(a.ds, 0), spare, qvoff, 0x80000000u);
  }
  __syncthreads();

  // Read cursor: the tile's ring stage, query head, first row and (stored
  // dS) its dS row within the head's slice, advanced like the issue cursor.
  const int ds_row0 = static_cast<int>(ds_row_start(a.ds_tri, a.ds_nkt, q_start / QT));
  int cur_st = 0, cur_r = 0, cur_qi = 0, cur_q0 = q_start, cur_row = ds_row0;
  uint64_t cur_da = first.da;
  TileIdx cur_idx = first;
  for (int itn = 0; itn < n_iter; ++itn) {
    // Tile itn + 2 is issued between the S / dP MFMA steps below, so a wave
    // never stalls on the address unit before its first MFMA.
    // (not an immediately-invoked lambda: one taking nxt_idx by reference
    // moves the dropout kernels' spills into this loop)
    TileDma tdma;
    if constexpr (DR) {
      tdma = tile_dma(nxt_idx);
      nxt_idx = tile_next(nxt_idx);
    }
    const auto &nxt = pick<DR>(tdma, icur);
    int st_off, hq, q0;
    uint64_t cur_idx_da;
    uint32_t ds_tile;
    if constexpr (DR) {
      st_off = (itn % KV_NS) * STAGE_B;
      hq = hk * p.rep + cur_idx.r;
      q0 = q_start + cur_idx.qi * QT;
      cur_idx_da = cur_idx.da;
      ds_tile = static_cast<uint32_t>((ds_row_start(a.ds_tri, a.ds_nkt, q0 / QT) + kw / 32) * DS_TILE);
      cur_idx = tile_next(cur_idx);
    } else {
      st_off = cur_st;
      hq = hk * p.rep + cur_r;
      q0 = cur_q0;
      cur_idx_da = cur_da;
      ds_tile = static_cast<uint32_t>(cur_row + kw / 32) * DS_TILE;
      cur_st = cur_st == (KV_NS - 1) * STAGE_B ? 0 : cur_st + STAGE_B;
      cur_q0 += QT;
      // dS rows: row qt holds 4 (qt / 4 + 1) tiles (packed causal) or ds_nkt
      cur_row += a.ds_tri ? 4 * static_cast<int>(static_cast<uint32_t>(q0) / (4 * QT) + 1) : a.ds_nkt;
      if (++cur_qi == n_qt) {
        asm volatile("");  // (a branch taken once per head)
        cur_qi = 0;
        ++cur_r;
        cur_q0 = q_start;
        cur_row = ds_row0;
        cur_da += dwrap;
      }
    }
    const char *qt = ring + st_off;
    const char *gt = qt + TILE_Q;
    const float *rv = reinterpret_cast<const float *>(qt + TILE_Q + TILE_G);

    constexpr int FD = DKDV_FD;
    // A general mask: this tile's elements (b, hq, q0 + 4h + kc, key), kc
    // along the rows, fetched before the S / dP MFMAs (their latency hides
    // under them) and before the next tile's DMA parts issued among those, so
    // that the wait for them leaves the parts in flight.
    MaskFetch mf;
    if constexpr (MK != 0 && !MSTAGE) {
      constexpr int mes = mask_bytes<MK>();
      const int64_t extent = ((p.Sq - 1) * p.mask.s2 + (p.Sk - 1) * p.mask.s3 + 1) * mes;
      const u32x4 mdesc = make_desc(
          static_cast<const char *>(p.mask.data) + (b * p.mask.s0 + hq * p.mask.s1) * mes,
          static_cast<uint32_t>(extent));
      const int64_t off0 = (static_cast<int64_t>(q0 + 4 * h) * p.mask.s2 +
                            static_cast<int64_t>(key) * p.mask.s3) * mes;
      mf.issue<mes>(mdesc, static_cast<uint32_t>(off0), static_cast<uint32_t>(p.mask.s2 * mes));
    }
    // S = Q K^T + nl, dP = dO V^T + nd over the tile's 32 rows x this wave's
    // 32 keys, the accumulators starting from the rows' nl / nd values:
    // sacc[e] = (S[q0 + crow(e, h)][key] scale - lse) / scale.
    f32x16 sacc, dpacc;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 l4 = *reinterpret_cast<const float4 *>(rv + 8 * g + 4 * h);
      const float4 d4 = DR ? float4{0.f, 0.f, 0.f, 0.f}  // dropout: dP alone, nd added later
                           : *reinterpret_cast<const float4 *>(rv + QT + 8 * g + 4 * h);
      sacc[4 * g] = l4.x, sacc[4 * g + 1] = l4.y, sacc[4 * g + 2] = l4.z, sacc[4 * g + 3] = l4.w;
      dpacc[4 * g] = d4.x, dpacc[4 * g + 1] = d4.y, dpacc[4 * g + 2] = d4.z, dpacc[4 * g + 3] = d4.w;
    }
    {
      u32x4 qa[FD + 1], ga[FD + 1];
      auto load = [&](int i) {
        if (i < SKQ) qa[i % (FD + 1)] = rdq.rows(qt, 0, i);
        if (i < SKV) ga[i % (FD + 1)] = rdg.rows(gt, 0, i);
      };
#pragma unroll
      for (int i = 0; i < FD; ++i) load(i);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < STEPS; ++i) {
        if (i < SKQ) sacc = mfma32<T>(qa[i % (FD + 1)], kf[i], sacc);
        if (i < SKV) dpacc = mfma32<T>(ga[i % (FD + 1)], vf[i], dpacc);
        if (i + FD < STEPS) load(i + FD);
        if ((i & 1) && (i >> 1) < LPT) issue_part(nxt, i >> 1);
        if (i == 0) {
          issue_part(nxt, LPT);
          issue_mask(nxt);
          issue_bits(nxt);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      __builtin_amdgcn_s_setprio(0);
    }
    if constexpr (!DR) issue_next(icur);

    // P = exp2(sacc sl), dS = P dpacc; rows crow(e, h) = 8 g + 4 h + e % 4.
    const bool edge = MK != 0 || keymask || kw + 32 > kv_end || q0 + QT > p.Sq ||
                      (causal && q0 < q_diag);
    int lo = -64, hi = 64;
    if (edge) {
      hi = key_live ? p.Sq - q0 - 4 * h : -64;
      if (causal) lo = min(64, max(-64, kdiff - q0 - 4 * h));
    }
    u32x4 pp[2], pd[2];
    // Dropout: the staged keep bits; lane (c, h) reads rows 8 g + 4 h + r
    // (four words per g) and takes bit c.  dV takes P * mask, dS = P (dP *
    // mask - delta), m = 1 / (1 - p) folded into the row values.
    const char *btile = qt + BOFF + w * 128;
    // (an offset the compiler cannot see through: otherwise it keeps the nd
    // values it read to start dpacc live across the MFMA steps)
    int nd_off = QT;
    if constexpr (DR) asm volatile("" : "+v"(nd_off));
    // Staged mask: this lane's column (key 32 w + c) at row 4 h of the tile.
    const char *mrow_base = nullptr;
    if constexpr (MSTAGE) {
      uint32_t l;
      asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
      mrow_base = qt + MOFF + (l >> 5) * 4 * MROW + (32 * w + (l & 31)) * MES;
    }
    // Interior tiles skip the per-element bounds (three VALU ops each).
    auto grad = [&](auto masked) {
      float xs[16];
      if constexpr (MK != 0 && !MSTAGE) {
        // The mask loads; the next tile's Q / dO parts stay in flight (waves 0
        // and 1 also wait for their row-value part, the first one issued).
        wait_vm_n<LPT>();
        mf.resolve();
#pragma unroll
        for (int e = 0; e < 16; ++e) xs[e] = sacc[e];
        mask_scores<MK>(xs, mf, p.mask.dtype, lo, hi, sl);
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float pv[4], dsv[4];
        // (read word by word where used: four words held at once spill)
        const uint32_t *bw = reinterpret_cast<const uint32_t *>(btile + (8 * g + 4 * h) * 4);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int e = 4 * g + r, kc = 8 * g + r;
          if constexpr (MK == 0) {
            pv[r] = fast_exp2(sacc[e] * sl);
            if (masked) pv[r] = ((kc >= lo) & (kc < hi)) ? pv[r] : 0.f;
          } else if constexpr (MSTAGE) {
            // element (row 8 g + 4 h + r, key 32 w + c) of the staged tile
            const bool in = (kc >= lo) & (kc < hi);
            const char *me = mrow_base + (8 * g + r) * MROW;
            if constexpr (mask_kind(MK) == 1) {
              pv[r] = in && *reinterpret_cast<const uint8_t *>(me) ? fast_exp2(sacc[e] * sl) : 0.f;
            } else {
              const uint32_t bits = *reinterpret_cast<const uint16_t *>(me);
              const float mv = p.mask.dtype == TSATTN_BF16
                                   ? __builtin_bit_cast(float, bits << 16)
                                   : static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(bits)));
              pv[r] = in ? fast_exp2(fmaf(sacc[e], sl, mv * kLog2e)) : 0.f;
            }
          } else {
            // -inf where disallowed; additive-masked scores arrive scaled
            pv[r] = fast_exp2(mask_kind(MK) >= 2 ? xs[e] : xs[e] * sl);
          }
          if constexpr (DR) {
            // pv = P m and dpacc = dP + nd / m (the row values absorb m)
            const bool keep = (bw[r] >> c) & 1u;
            const float nd = rv[nd_off + 8 * g + 4 * h + r];
            dsv[r] = pv[r] * (keep ? dpacc[e] + nd : nd);
            pv[r] = keep ? pv[r] : 0.f;
          } else {
            dsv[r] = pv[r] * dpacc[e];
          }
        }
        pp[g >> 1][(g & 1) * 2] = pack2<T>(pv[0], pv[1]);
        pp[g >> 1][(g & 1) * 2 + 1] = pack2<T>(pv[2], pv[3]);
        pd[g >> 1][(g & 1) * 2] = pack2<T>(dsv[0], dsv[1]);
        pd[g >> 1][(g & 1) * 2 + 1] = pack2<T>(dsv[2], dsv[3]);
        // staged masks: four LDS reads in flight at a time, not sixteen (the
        // register budget of two workgroups per CU has no room for them)
        if constexpr (MSTAGE || DR) __builtin_amdgcn_sched_barrier(0);
      }
    };
    if (edge) grad(std::true_type{});
    else grad(std::false_type{});

    // dV^T += dO^T P, dK^T += Q^T dS over the tile's rows; step i: value
    // block i % PDT, query k-step i / PDT (rows 16 (i / PDT) ..).
    {
      u32x4 gc[FD + 1], qc[FD + 1];
      auto load = [&](int i) {
        if (i < 2 * PDV) gc[i % (FD + 1)] = rdg.cols(gt, i / PDV, i % PDV);
        if (i < 2 * PDK) qc[i % (FD + 1)] = rdq.cols(qt, i / PDK, i % PDK);
      };
#pragma unroll
      for (int i = 0; i < FD; ++i) load(i);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < STEPS; ++i) {
        if (i < 2 * PDV) dv_acc[i % PDV] = mfma32<T>(gc[i % (FD + 1)], pp[i / PDV], dv_acc[i % PDV]);
        if (i < 2 * PDK) dk_acc[i % PDK] = mfma32<T>(qc[i % (FD + 1)], pd[i / PDK], dk_acc[i % PDK]);
        if (i + FD < STEPS) load(i + FD);
        __builtin_amdgcn_sched_barrier(0);
      }
      __builtin_amdgcn_s_setprio(0);
    }

    // Stored dS (dQ as one GEMM after this kernel): the wave's packed dS
    // registers as they are, pd[0] then pd[1], 1 KiB per wave store, lane
    // (c, h) of pd[gg] at 16 (c ^ 4 h ^ 8 gg) + 512 h (the dQ kernel's
    // transpose reads of them are then free of bank conflicts).  Stores
    // count in vmcnt: the tile wait leaves these two in flight too.
    if (a.ds) {
      // lane * 16 ^ (h * 64), recomputed here rather than held in a
      // register all loop
      uint32_t l16;
      asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0\n\t"
                   "v_lshlrev_b32 %0, 4, %0"
                   : "=v"(l16));
      l16 ^= (l16 >> 9) << 6;
      // streaming stores (cache policy sc1 nt): written once, read once by
      // the dQ kernel, kept from evicting the Q / dO rows other key blocks
      // reuse.  Offsets within the head slice (below 2^31 bytes).
      const rsrc_t dsr = make_rsrc(a.ds + cur_idx_da, static_cast<uint32_t>(a.ds_slice * DS_TILE));
      const uint32_t o = static_cast<uint32_t>(ds_tile);
      __builtin_amdgcn_raw_buffer_store_b128(pd[0], dsr, static_cast<int>(o + l16), 0, kStreamStore);
      __builtin_amdgcn_raw_buffer_store_b128(pd[1], dsr, static_cast<int>(o + 1024 + (l16 ^ 128)), 0,
                                             kStreamStore);
      // tile itn + 1 has landed; the previous tile's stores may still be in
      // flight (they were issued after its loads; before the first tile two
      // empty loads stand in for them)
      wait_vm_n<(KV_PD - 1) * PARTS + 4>();
    } else {
      wait_vm_n<(KV_PD - 1) * PARTS>();  // tile itn + 1 has landed
    }
    wait_lgkm0();
    phase_barrier();
  }
  // The loads issued past the last tile land in the ring (dropout kernels:
  // the spare block): every wave's have landed before any wave's epilogue
  // writes there.
  wait_vm_n<0>();
  if constexpr (!DR) __syncthreads();

  // Epilogue.  The ring is free.  Each wave rounds its rows and stages them in its own
  // slice of the ring -- key row r (0..31) at r * 2DX bytes, 16-byte chunk q
  // at q ^ (r % CPR), the XOR keeping the row writes off one bank -- then
  // reads them back as whole 16-byte chunks of rows, so the global stores are
  // coalesced.  dK (DX = DK) first, then dV (DX = DV) through the same slice.
  static_assert(NW * 32 * 2 * DMAX <= KV_NS * STAGE_B, "epilogue slices fit in the ring");
  char *slice = ring + w * 32 * 2 * DMAX;
  auto store_rows = [&](auto dx, const auto &acc, const View &ov, float f, bool rope_back) {
    constexpr int DX = decltype(dx)::value, PD = DX / 32;
    constexpr int CPR = DX / 8;  // 16-byte chunks per row
    static_assert(32 * CPR % 64 == 0, "store chunks split evenly over the lanes");
    // lane holds X^T[d = 32 dt + 8 g + 4 h + r][key row c]: 4 consecutive d
#pragma unroll
    for (int dt = 0; dt < PD; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int off = c * 2 * DX + (((4 * dt + g) ^ (c % CPR)) * 16) + 8 * h;
        *reinterpret_cast<u32x2 *>(slice + off) =
            u32x2{pack2<T>(acc[dt][4 * g] * f, acc[dt][4 * g + 1] * f),
                  pack2<T>(acc[dt][4 * g + 2] * f, acc[dt][4 * g + 3] * f)};
      }
    T *ob = mut<T>(ov) + b * ov.s0 + hk * ov.s1;
    u32x4 vr[32 * CPR / 64];
#pragma unroll
    for (int u = 0; u < 32 * CPR / 64; ++u) {
      const int idx = u * 64 + lane, r = idx / CPR, q = idx % CPR;
      vr[u] = *reinterpret_cast<const u32x4 *>(slice + r * 2 * DX + ((q ^ (r % CPR)) * 16));
    }
    // RoPE folded in: dK of the unrotated keys = the inverse rotation of the
    // rounded dK, key position kpos0 + kw + r, one 16-byte row chunk at a time.
    if (rope_back) {
      int64_t rows[32 * CPR / 64];
      int p0[32 * CPR / 64];
#pragma unroll
      for (int u = 0; u < 32 * CPR / 64; ++u) {
        const int idx = u * 64 + lane, r = idx / CPR, q = idx % CPR;
        rows[u] = p.rope.kpos0 + (kw + r < p.Sk ? kw + r : p.Sk - 1);  // rows past Sk: not stored
        p0[u] = 4 * q;
      }
      rotate_chunks<T, 32 * CPR / 64>(vr, p.rope, rows, p0, true);
    }
#pragma unroll
    for (int u = 0; u < 32 * CPR / 64; ++u) {
      const int idx = u * 64 + lane, r = idx / CPR, q = idx % CPR;
      if (kw + r < p.Sk) __builtin_nontemporal_store(vr[u], reinterpret_cast<u32x4 *>(ob + static_cast<int64_t>(kw + r) * ov.s2 + q * 8));
    }
  };
  if constexpr (DK == DV) {
    // one loop over the two passes (same dims: the register allocation of the
    // tuned equal-dim kernels)
    constexpr int CPR = DK / 8, PD = DK / 32;
    const float sc = a.scale;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      const f32x16 *acc = pass == 0 ? dk_acc : dv_acc;
      const float f = pass == 0 ? sc : 1.f;
#pragma unroll
      for (int dt = 0; dt < PD; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int off = c * 2 * DK + (((4 * dt + g) ^ (c % CPR)) * 16) + 8 * h;
          *reinterpret_cast<u32x2 *>(slice + off) =
              u32x2{pack2<T>(acc[dt][4 * g] * f, acc[dt][4 * g + 1] * f),
                    pack2<T>(acc[dt][4 * g + 2] * f, acc[dt][4 * g + 3] * f)};
        }
      const View &ov = pass == 0 ? a.dk : a.dv;
      T *ob = mut<T>(ov) + b * ov.s0 + hk * ov.s1;
      u32x4 vr[32 * CPR / 64];
#pragma unroll
      for (int u = 0; u < 32 * CPR / 64; ++u) {
        const int idx = u * 64 + lane, r = idx / CPR, q = idx % CPR;
        vr[u] = *reinterpret_cast<const u32x4 *>(slice + r * 2 * DK + ((q ^ (r % CPR)) * 16));
      }
      if (pass == 0 && p.rope.R > 0) {
        int64_t rows[32 * CPR / 64];
        int p0[32 * CPR / 64];
#pragma unroll
        for (int u = 0; u < 32 * CPR / 64; ++u) {
          const int idx = u * 64 + lane, r = idx / CPR, q = idx % CPR;
          rows[u] = p.rope.kpos0 + (kw + r < p.Sk ? kw + r : p.Sk - 1);  // rows past Sk: not stored
          p0[u] = 4 * q;
        }
        rotate_chunks<T, 32 * CPR / 64>(vr, p.rope, rows, p0, true);
      }
#pragma unroll
      for (int u = 0; u < 32 * CPR / 64; ++u) {
        const int idx = u * 64 + lane, r = idx / CPR, q = idx % CPR;
        if (kw + r < p.Sk) __builtin_nontemporal_store(vr[u], reinterpret_cast<u32x4 *>(ob + static_cast<int64_t>(kw + r) * ov.s2 + q * 8));
      }
    }
  } else {
    store_rows(std::integral_constant<int, DK>{}, dk_acc, a.dk, a.scale, p.rope.R > 0);
    store_rows(std::integral_constant<int, DV>{}, dv_acc, a.dv, 1.f, false);
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

// DK = head dim of q / k (and dQ), DV = of v / dO; each 64 or 128.
template <typename T, int DK, int DV, int MK, bool DR>
__global__ __launch_bounds__(NT, 2) void dq_kernel(BwdArgs a) {
  constexpr int TILE_K = KT * DK * 2, TILE_V = KT * DV * 2;  // bytes per K / V tile
  // K | V | with dropout each wave's 32 keep-bit words (its rows, this key tile)
  constexpr int STAGE = TILE_K + TILE_V + (DR ? NW * 128 : 0);
  // 1 KiB DMA blocks of a K / V tile, split over the waves as in dkdv_kernel
  constexpr int KBLK = TILE_K / 1024, VBLK = TILE_V / 1024;
  constexpr bool EVEN = KBLK % NW == 0 && VBLK % NW == 0;
  constexpr int KPARTS = KBLK / NW, VPARTS = VBLK / NW;
  constexpr int LPT = (KBLK + VBLK + NW - 1) / NW;  // DMA loads per wave per K+V tile
  constexpr int PPT = LPT + (DR ? 1 : 0);     // all DMA loads per wave per tile
  constexpr int SKQ = DK / 16, SKV = DV / 16;  // k-steps of S (over DK), dP (over DV)
  constexpr int PDQ = DK / 32;                 // 32-row blocks of dQ^T (2 key k-steps each)
  constexpr int STEPS = SKQ > SKV ? SKQ : SKV;
  constexpr int QGK = DK / 32, QGV = DV / 32;
  static_assert(EVEN ? (KPARTS >= 1 && VPARTS >= 1 && LPT == KPARTS + VPARTS)
                     : (KBLK + VBLK == NW && LPT == 1 && DK == 32 && DV == 32),
                "tile loads must split over the waves");
  static_assert(2 * LPT <= STEPS, "one DMA part per two MFMA steps");
  // [stage][K | V (| bits)], then a 1 KiB block that DMA parts past the last
  // tile land in (nothing reads it)
  __shared__ __attribute__((aligned(1024))) char lds[DQ_NS * STAGE + 1024];

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
  const bool keymask =
      MK == 0 && p.mask.kind == TSATTN_MASK_BOOL && !(p.kv_prefix && p.kv_prefix[b]);
  const bool causal = p.causal != 0;

  int64_t lim = kv_end, wlim = kv_end;
  if (causal) {
    lim = min(lim, static_cast<int64_t>(min(q0 + QB, p.Sq) - 1) + p.offset + 1);
    wlim = min(wlim, static_cast<int64_t>(min(qw + 32, p.Sq) - 1) + p.offset + 1);
  }
  if (qw >= p.Sq) wlim = 0;
  // wave-uniform by construction; readfirstlane keeps them in SGPRs
  const int n_tiles =
      __builtin_amdgcn_readfirstlane(lim > 0 ? static_cast<int>((lim + KT - 1) / KT) : 0);
  const int w_tiles =
      __builtin_amdgcn_readfirstlane(wlim > 0 ? static_cast<int>((wlim + KT - 1) / KT) : 0);

  // The rows' Q, dO and O fragments (lane holds row qrow, channels 16 ks +
  // 8 h .. +7) and LSE, issued here; consumed after the first tiles' DMA
  // issue below, so the two latencies overlap.
  u32x4 qf[SKQ], gf[SKV], of[SKV];
  float lse2, delta;  // -safe(lse) in exp2 units, -delta
  const int64_t row = (static_cast<int64_t>(b) * p.Hq + hq) * p.Sq + qrow;
  const float lrow_lse = qrow < p.Sq ? a.lse[row] : 0.f;
  {
    const uint32_t qs_b = static_cast<uint32_t>(a.q.s2) * 2, gs_b = static_cast<uint32_t>(a.dout.s2) * 2;
    const uint32_t os_b = static_cast<uint32_t>(a.o.s2) * 2;
    const rsrc_t qrs = make_rsrc(head_ptr<T>(a.q, b, hq), static_cast<uint32_t>(p.Sq) * qs_b);
    const rsrc_t grs = make_rsrc(head_ptr<T>(a.dout, b, hq), static_cast<uint32_t>(p.Sq) * gs_b);
    const rsrc_t ors = make_rsrc(head_ptr<T>(a.o, b, hq), static_cast<uint32_t>(p.Sq) * os_b);
#pragma unroll
    for (int ks = 0; ks < STEPS; ++ks) {
      if (ks < SKQ) qf[ks] = buf_load16(qrs, static_cast<uint32_t>(qrow) * qs_b + (ks * 16 + h * 8) * 2);
      if (ks < SKV) {
        gf[ks] = buf_load16(grs, static_cast<uint32_t>(qrow) * gs_b + (ks * 16 + h * 8) * 2);
        of[ks] = buf_load16(ors, static_cast<uint32_t>(qrow) * os_b + (ks * 16 + h * 8) * 2);
      }
    }
  }

  const uint32_t ks_b = static_cast<uint32_t>(a.k.s2) * 2, vs_b = static_cast<uint32_t>(a.v.s2) * 2;
  const u32x4 kdesc = make_desc(head_ptr<T>(a.k, b, hk), static_cast<uint32_t>(kv_end) * ks_b);
  const u32x4 vdesc = make_desc(head_ptr<T>(a.v, b, hk), static_cast<uint32_t>(kv_end) * vs_b);
  const uint32_t lds0 = lds_addr(lds);
  // Wave w loads blocks e = w, w + 4, ... of the tile (K blocks first, then V):
  // block n = (n / QG, n % QG), lane l fetches row 16 (n / QG) + l / 4, chunk
  // 4 (n % QG) + ((l % 4) ^ ((l / 16) % 4)); n % QG = w % QG for all of them.
  const uint32_t swz_chunk = (lane & 3) ^ ((lane >> 4) & 3);
  const uint32_t koff = (lane >> 2) * ks_b + (4 * (w % QGK) + swz_chunk) * 16;
  const uint32_t voff = (lane >> 2) * vs_b + (4 * (w % QGV) + swz_chunk) * 16;
  // Every iteration issues its parts: those of a tile past the last one read
  // past the buffer range (zeros, no memory access) into the spare LDS
  // block, so the count of loads in flight is the same on every iteration
  // and no branch guards an issue.  Per tile, computed once: its first row's
  // byte offset in K and V and its stage offset from the spare block, masked
  // by keep (all ones for a real tile, else 0 -- masks, not selects, which
  // the compiler would turn into branches between the MFMA steps).
  const uint32_t spare = lds0 + DQ_NS * STAGE;
  struct DmaTile {
    uint32_t krow, vrow, st, keep, far;
    int tile;
  };
  auto dma_tile = [&](int tile) {
    DmaTile d;
    d.tile = tile;
    d.keep = ~static_cast<uint32_t>((n_tiles - 1 - tile) >> 31);  // sign fill
    d.far = ~d.keep & 0x80000000u;  // offsets >= 2^31 are past every range
    d.krow = (static_cast<uint32_t>(tile * KT) * ks_b) | d.far;
    d.vrow = (static_cast<uint32_t>(tile * KT) * vs_b) | d.far;
    d.st = (lds0 + (tile % DQ_NS) * STAGE - spare) & d.keep;
    return d;
  };
  // Parts u < KPARTS are K blocks, the rest V blocks (a compile-time split;
  // at head dim 32 waves 0, 1 load K and waves 2, 3 V).
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
  // Dropout: the wave's 32 keep-bit words of the tile as one 8-lane part
  // (rows past the (b, hq) slice read as zero; rows past Sq are unused).
  auto issue_bits = [&](const DmaTile &t) {
    if constexpr (DR) {
      const DropDesc &d = p.drop;
      const u32x4 bdesc = make_desc(d.bits + (static_cast<int64_t>(b) * p.Hq + hq) * d.nkt * d.sqp,
                                    static_cast<uint32_t>(d.nkt * d.sqp * 4));
      uint32_t loff;
      asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0\n\t"
                   "v_lshlrev_b32 %0, 4, %0"
                   : "=v"(loff));
      if (lane < 8)
        dma16(bdesc, spare + t.st + ((TILE_K + TILE_V + w * 128) & t.keep), loff,
              ((static_cast<uint32_t>(t.tile) * d.sqp + qw) * 4) | t.far);
    }
  };
  auto issue = [&](int tile) {
    const DmaTile d = dma_tile(tile);
#pragma unroll
    for (int u = 0; u < LPT; ++u) issue_part(d, u);
    issue_bits(d);
  };

  const TileReader<T, DK> rdk(lane);
  const TileReader<T, DV> rdv(lane);
  f32x16 acc[PDQ];
#pragma unroll
  for (int dt = 0; dt < PDQ; ++dt) acc[dt] = f32x16{};
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
  MaskFetch mf;
  const float slx = mask_kind(MK) >= 2 ? 1.f : sl;  // additive-masked scores arrive scaled

  // The first MFMA block multiplies the K half of stage DQ_NS - 1 (no DMA has
  // written it yet) by dS = 0: zero it (0 x stale NaN is NaN).  Every other
  // LDS byte is written by a DMA load before it is read (lanes past the
  // buffer range write zeros).
  // (no barrier between the zeroing and the DMA loads: they write other
  // stages; the barrier below orders both before the loop)
  zero_lds<NT>(lds + (DQ_NS - 1) * STAGE, TILE_K, tid);
  for (int t = 0; t < DQ_PD; ++t) issue(t);
  {
    // RoPE folded in: rotate the query fragments as the forward did, and
    // stage the rotated rows for the dK/dV kernel.
    if (p.rope.R > 0) {
      int64_t rows[SKQ];
      int p0[SKQ];
#pragma unroll
      for (int ks = 0; ks < SKQ; ++ks) {
        rows[ks] = p.rope.qpos0 + (qrow < p.Sq ? qrow : p.Sq - 1);  // rows past Sq: unused
        p0[ks] = 8 * ks + 4 * h;
      }
      rotate_chunks<T, SKQ>(qf, p.rope, rows, p0, false);
      if (qrow < p.Sq && !p.rope.qrot) {  // (qrot: the forward stored them)
        T *qk = mut<T>(a.qk) + b * a.qk.s0 + hq * a.qk.s1 + static_cast<int64_t>(qrow) * a.qk.s2;
#pragma unroll
        for (int ks = 0; ks < SKQ; ++ks) *reinterpret_cast<u32x4 *>(qk + ks * 16 + h * 8) = qf[ks];
      }
    }
    const float l = lrow_lse;
    // delta = sum_d dO O in fp32; lanes c and c + 32 hold the row's two halves
    float dsum = 0.f;
#pragma unroll
    for (int ks = 0; ks < SKV; ++ks) {
      const T *ge = reinterpret_cast<const T *>(&gf[ks]);
      const T *oe = reinterpret_cast<const T *>(&of[ks]);
#pragma unroll
      for (int e = 0; e < 8; ++e) dsum += static_cast<float>(ge[e]) * static_cast<float>(oe[e]);
    }
    delta = -xor32_sum(dsum);
    lse2 = isfinite(l) ? -l * kLog2e : 0.f;
    if (h == 0 && qrow < p.Sq) store_row_values(a, static_cast<int64_t>(p.B) * p.Hq * p.Sq, row, delta, l);
  }
  // (the compiler's wait for these loads -- it does not count the DMA
  // loads, so it waits for everything in flight -- also covers the first
  // tiles; resolved here, no use inside the main loop can make it wait for
  // tiles in flight)
#pragma unroll
  for (int ks = 0; ks < STEPS; ++ks) {
    if (ks < SKQ && ks < SKV) asm volatile("" : "+v"(qf[ks]), "+v"(gf[ks]));
    else if (ks < SKQ) asm volatile("" : "+v"(qf[ks]));
    else asm volatile("" : "+v"(gf[ks]));
  }
  asm volatile("" : "+v"(delta), "+v"(lse2));
  wait_vm_n<(DQ_PD - 1) * PPT>();
  __syncthreads();

  // Tiles from j_edge on need masking (the causal diagonal, a ragged end, a
  // key mask or a general mask); those before it are interior.
  int j_edge = kv_end / KT;
  if (MK != 0 || keymask) j_edge = 0;
  if (causal) {
    const int64_t d = static_cast<int64_t>(qw) + p.offset - (KT - 1);
    const int jc = d < 0 ? 0 : static_cast<int>(min(d / KT + 1, static_cast<int64_t>(INT32_MAX)));
    j_edge = min(j_edge, jc);
  }

  // MFMA block of tile j: S_j^T, dP_j^T (k-step i each) and dQ MFMA i of the
  // previous tile (value block i % PDT, key k-step i / PDT); fragments two
  // steps ahead.  One code path for every block keeps the accumulators in
  // place: the first block multiplies a zeroed stage by dS = 0, and past the
  // wave's last tile S and dP are computed and ignored.
  // fetch: also load tile j's mask elements, before the DMA parts.
  auto mfma_block = [&](int j, int nt, bool fetch) {  // nt: tile whose DMA to issue, or -1
    if constexpr (mask_vec(MK)) {
      if (fetch) mf.issue_vec<mes>(mdesc, mrow + static_cast<uint32_t>(j * KT + 16 * h) * mes);
    } else if constexpr (MK != 0) {
      if (fetch) mf.issue<mes>(mdesc, mrow + static_cast<uint32_t>(j * KT + 4 * h) * mstep, mstep);
    }
    const char *kt = lds + (j % DQ_NS) * STAGE;
    const char *vt = kt + TILE_K;
    const char *kp = lds + ((j + DQ_NS - 1) % DQ_NS) * STAGE;
    const DmaTile dt_next = dma_tile(nt);
    constexpr int FD = 2;
    u32x4 kr[FD + 1], vr[FD + 1], kc[FD + 1];
    auto load = [&](int i) {
      if (i < SKQ) kr[i % (FD + 1)] = rdk.rows(kt, 0, i);
      if (i < SKV) vr[i % (FD + 1)] = rdv.rows(vt, 0, i);
      if (i < SKQ) kc[i % (FD + 1)] = rdk.cols(kp, i / PDQ, i % PDQ);
    };
    s = f32x16{};
    dp = f32x16{};
    issue_bits(dt_next);
#pragma unroll
    for (int i = 0; i < FD; ++i) load(i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < STEPS; ++i) {
      if (i < SKQ) s = mfma32<T>(kr[i % (FD + 1)], qf[i], s);
      if (i < SKV) dp = mfma32<T>(vr[i % (FD + 1)], gf[i], dp);
      if (i < SKQ) acc[i % PDQ] = mfma32<T>(kc[i % (FD + 1)], pd[i / PDQ], acc[i % PDQ]);
      if (i + FD < STEPS) load(i + FD);
      if ((i & 1) && (i >> 1) < LPT) issue_part(dt_next, i >> 1);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  auto grad = [&](int j, int) {
    const int kv0 = j * KT;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = s[i];
    if (j >= j_edge) {
      const int lim_l = klim - kv0 - 4 * h;
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
          const bool ok = (kc < lim_l) & (((kbits >> kc) & 1u) != 0);
          x[i] = ok ? x[i] : -INFINITY;
        }
      } else {
        wait_vm_n<LPT>();  // the mask loads; the next tile's parts stay in flight
        if constexpr (mask_vec(MK)) {
          mf.resolve_vec<mes>();
          mf.unpack<mes>(h);
        } else {
          mf.resolve();
        }
        mask_scores<MK>(x, mf, p.mask.dtype, -64, lim_l, sl);
      }
    }
    // Dropout: dS = P (dP * mask - delta) (attention.py:215-217), the mask
    // from row qrow's keep-bit word of the tile, staged with it.
    uint32_t kbits = 0;
    if constexpr (DR)
      kbits = *reinterpret_cast<const uint32_t *>(lds + (j % DQ_NS) * STAGE + TILE_K + TILE_V +
                                                  w * 128 + c * 4);
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      const float p0 = fast_exp2(fmaf(x[i], slx, lse2));
      const float p1 = fast_exp2(fmaf(x[i + 1], slx, lse2));
      float d0 = dp[i], d1 = dp[i + 1];
      if constexpr (DR) {
        d0 = (kbits >> (8 * (i >> 2) + 4 * h + (i & 3))) & 1u ? d0 * p.drop.scale : 0.f;
        d1 = (kbits >> (8 * (i >> 2) + 4 * h + (i & 3) + 1)) & 1u ? d1 * p.drop.scale : 0.f;
      }
      pd[i >> 3][(i & 7) >> 1] = pack2<T>(p0 * (d0 + delta), p1 * (d1 + delta));
    }
  };

  auto next_dma = [&](int j) { return j + DQ_PD; };
  auto it_end = [&](int) {
    wait_vm_n<(DQ_PD - 1) * PPT>();  // tile j + 1 has landed
    wait_lgkm0();
    phase_barrier();
  };
  int j = 0;
  if (w_tiles > 0) {
    pd[0] = pd[1] = u32x4{0, 0, 0, 0};
    for (; j < w_tiles; ++j) {
      mfma_block(j, next_dma(j), true);
      grad(j, next_dma(j));
      it_end(j);
    }
    mfma_block(j, next_dma(j), false);  // dQ of the last tile
    it_end(j);
    ++j;
  }
  for (; j <= n_tiles; ++j) {
    issue(next_dma(j));
    it_end(j);
  }
  wait_vm_n<0>();  // the last (spare-block) loads, before the epilogue reuses the ring

  // dQ rows leave through LDS (free after the last barrier, all loads waited
  // for): each wave rounds its 32 rows into its own slice -- row r at r * 2D
  // bytes, 16-byte chunk q at q ^ (r % CPR) -- then reads back whole 16-byte
  // chunks of rows for coalesced stores.  Lane holds dQ^T[d = 32 dt + 8 g +
  // 4 h + r][row c].
  constexpr int CPR = DK / 8;
  static_assert(NW * 32 * 2 * DK <= DQ_NS * STAGE, "output slices fit in the ring");
  static_assert(32 * CPR % 64 == 0, "store chunks split evenly over the lanes");
  char *slice = lds + w * 32 * 2 * DK;
  const float sc = a.scale;
#pragma unroll
  for (int dt = 0; dt < PDQ; ++dt) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int off = c * 2 * DK + (((4 * dt + g) ^ (c % CPR)) * 16) + 8 * h;
      *reinterpret_cast<u32x2 *>(slice + off) =
          u32x2{pack2<T>(acc[dt][g * 4] * sc, acc[dt][g * 4 + 1] * sc),
                pack2<T>(acc[dt][g * 4 + 2] * sc, acc[dt][g * 4 + 3] * sc)};
    }
  }
  T *ob = mut<T>(a.dq) + b * a.dq.s0 + hq * a.dq.s1;
  u32x4 vr[32 * CPR / 64];
#pragma unroll
  for (int u = 0; u < 32 * CPR / 64; ++u) {
    const int idx = u * 64 + lane, r = idx / CPR, q = idx % CPR;
    vr[u] = *reinterpret_cast<const u32x4 *>(slice + r * 2 * DK + ((q ^ (r % CPR)) * 16));
  }
  // RoPE folded in: dQ of the unrotated queries = the inverse rotation of the
  // rounded dQ (rotary_embedding's VJP), one 16-byte row chunk at a time.
  if (p.rope.R > 0) {
    int64_t rows[32 * CPR / 64];
    int p0[32 * CPR / 64];
#pragma unroll
    for (int u = 0; u < 32 * CPR / 64; ++u) {
      const int idx = u * 64 + lane, r = idx / CPR, q = idx % CPR;
      rows[u] = p.rope.qpos0 + (qw + r < p.Sq ? qw + r : p.Sq - 1);  // rows past Sq: not stored
      p0[u] = 4 * q;
    }
    rotate_chunks<T, 32 * CPR / 64>(vr, p.rope, rows, p0, true);
  }
#pragma unroll
  for (int u = 0; u < 32 * CPR / 64; ++u) {
    const int idx = u * 64 + lane, r = idx / CPR, q = idx % CPR;
    if (qw + r < p.Sq) __builtin_nontemporal_store(vr[u], reinterpret_cast<u32x4 *>(ob + static_cast<int64_t>(qw + r) * a.dq.s2 + q * 8));
  }
}

// ---------------------------------------------------------------------------
// Row values when the dK/dV kernel runs first (stored dS): nd = -delta, the
// fp32 sum over the row of dO O, and nl = -safe(lse) / scale, the values the
// dQ kernel's prologue writes otherwise; with RoPE folded in, also the
// rotated query rows the dK/dV kernel reads.  A row is G = DV / 8 lanes, one
// 16-byte piece each, 64 / G rows per wave.
// ---------------------------------------------------------------------------
constexpr int ROWS_U = 4;  // row groups per wave in the row-value kernel

template <typename T, int DK, int DV>
__global__ __launch_bounds__(NT) void bwd_rows_kernel(BwdArgs a, int nqb) {
  // Workgroup = block qb of the query rows of head bh (blockIdx = bh nqb +
  // qb: 32-bit index arithmetic only); a wave takes ROWS_U groups of RPW
  // rows, a row G = DV / 8 lanes, and issues all its loads before any math.
  constexpr int G = DV / 8, RPW = 64 / G, RPB = (NT / 64) * RPW * ROWS_U;
  const Problem &p = a.p;
  const int64_t rows = static_cast<int64_t>(p.B) * p.Hq * p.Sq;
  const int lane = threadIdx.x & 63, g = lane % G, w = threadIdx.x >> 6;
  const int bh = blockIdx.x / nqb, qb = blockIdx.x - bh * nqb;
  const int b = bh / p.Hq, hq = bh - b * p.Hq;
  const T *gh = head_ptr<T>(a.dout, b, hq) + 8 * g;
  const T *oh = head_ptr<T>(a.o, b, hq) + 8 * g;
  int qr[ROWS_U];
  u32x4 gv[ROWS_U], ov[ROWS_U];
  float lv[ROWS_U];  // the rows' LSE, loaded with the rows (its latency under theirs)
#pragma unroll
  for (int u = 0; u < ROWS_U; ++u) {
    qr[u] = qb * RPB + (u * (NT / 64) + w) * RPW + lane / G;
    const int r = qr[u] < p.Sq ? qr[u] : p.Sq - 1;  // past the head: reload its last row, store nothing
    // (read once here: non-temporal, 49 -> 44 us at B16 H16 S2048 D128)
    gv[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(gh + static_cast<int64_t>(r) * a.dout.s2));
    ov[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(oh + static_cast<int64_t>(r) * a.o.s2));
    lv[u] = a.lse[static_cast<int64_t>(bh) * p.Sq + r];
  }
#pragma unroll
  for (int u = 0; u < ROWS_U; ++u) {
    const T *ge = reinterpret_cast<const T *>(&gv[u]);
    const T *oe = reinterpret_cast<const T *>(&ov[u]);
    float dsum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) dsum += static_cast<float>(ge[e]) * static_cast<float>(oe[e]);
#pragma unroll
    for (int o = 1; o < G; o <<= 1) dsum += __shfl_xor(dsum, o, 64);
    if (g == 0 && qr[u] < p.Sq) {
      const int64_t row = static_cast<int64_t>(bh) * p.Sq + qr[u];
      store_row_values(a, rows, row, -dsum, lv[u]);
    }
  }
  if (p.rope.R > 0 && !p.rope.qrot) {  // (qrot: the forward stored them)
#pragma unroll
    for (int u = 0; u < ROWS_U; ++u) {
      if (qr[u] >= p.Sq) continue;
      const int qrow = qr[u];
      const T *qi = head_ptr<T>(a.q, b, hq) + static_cast<int64_t>(qrow) * a.q.s2;
      T *qk = mut<T>(a.qk) + b * a.qk.s0 + hq * a.qk.s1 + static_cast<int64_t>(qrow) * a.qk.s2;
#pragma unroll
      for (int ch = g; ch < DK / 8; ch += G) {
        u32x4 v = ld16(qi + 8 * ch);
        rotate_chunk<T>(v, p.rope, p.rope.qpos0 + qrow, 4 * ch, false);
        *reinterpret_cast<u32x4 *>(qk + 8 * ch) = v;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// dQ from stored dS: dQ^T = scale K^T dS^T over the key tiles of each row
// (one GEMM; the dK/dV kernel left dS in the workspace).  One workgroup = 512
// query rows of one (b, q head), 8 waves x two 32-row subtiles (w and 15 - w,
// sharing every K^T fragment), one workgroup per CU: each K tile fetched
// serves 512 rows (two 4-wave workgroups of 256 rows fetched it twice, 5%
// slower at B16 H16 S2048 D128).  Per 32-key tile, K
// (shared) and each wave's two dS tiles stream global -> LDS by DMA loads
// into 3-stage rings, issued two tiles ahead; K^T and dS^T fragments come
// from LDS transpose reads; one fence-free barrier per tile.  dS tiles past a
// subtile's causal end, or past the rows, read as zeros (offsets past the
// buffer range).
// ---------------------------------------------------------------------------
constexpr int DQ_NT = 512, DQ_NW = DQ_NT / 64;  // one 8-wave workgroup per CU
constexpr int QB2 = 64 * DQ_NW;   // query rows per workgroup
constexpr int DS_PD = 2;          // tiles issued ahead
constexpr int DS_NS = DS_PD + 1;  // ring stages: tile j is read in iteration j only

template <typename T, int DK>
__global__ __launch_bounds__(DQ_NT, 1) void dq_ds_kernel(BwdArgs a) {
  constexpr int TILE_K = KT * DK * 2;
  // K DMA loads per wave per tile (D = 64: one, the waves past the tile's
  // four blocks loading nothing into the spare block, so that every wave
  // issues the same count)
  constexpr int KPARTS = TILE_K / 1024 > DQ_NW ? TILE_K / 1024 / DQ_NW : 1;
  constexpr int LPT = KPARTS + 4;             // all DMA loads per wave per tile
  constexpr int PDQ = DK / 32;                // 32-row blocks of dQ^T
  constexpr int QGK = DK / 32;
  constexpr int STEPS = 2 * PDQ;              // K^T fragments per tile (2 key k-steps)
  constexpr int KRING = DS_NS * TILE_K;
  constexpr int SRING = DS_NS * 2 * DS_TILE;  // per wave: two dS tiles per stage
  constexpr int RINGS = KRING + DQ_NW * SRING;
  constexpr int EPI = DQ_NW * 32 * 2 * DK;       // epilogue: 32 rows per wave at a time
  static_assert(EPI <= RINGS, "epilogue slices fit in the rings");
  static_assert(KPARTS * DQ_NW * 1024 == TILE_K || (KPARTS == 1 && TILE_K <= DQ_NW * 1024),
                "tile loads split evenly over the waves");
  // K ring, the waves' dS rings, then a 1 KiB block that DMA parts past the
  // last tile land in
  __shared__ __attribute__((aligned(1024))) char lds[RINGS + 1024];

  const Problem &p = a.p;
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 31, h = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_qb = (p.Sq + QB2 - 1) / QB2;
  const int n_bh = a.ng * p.rep;  // query heads of the chunk's groups
  const int total = n_qb * n_bh;
  const int logical = xcd_remap(blockIdx.x, total);
  int bhc, rank;
  heavy_first(logical, n_qb, n_bh, 32, bhc, rank);  // 1 WG per CU
  const int qb = n_qb - 1 - rank;  // long causal rows first
  const int bh = a.g0 * p.rep + bhc;  // (b, q head); bhc: its dS slice in the region
  const int b = bh / p.Hq, hq = bh - b * p.Hq, hk = hq / p.rep;
  // Wave w takes the block's 32-row subtiles w and 15 - w, so that the
  // causal work of the four waves is alike (the subtiles share every K^T
  // fragment; the shorter one's operands past its end read as zeros).
  const int q0 = qb * QB2, qa = q0 + 32 * w, qz = q0 + 32 * (2 * DQ_NW - 1 - w);
  const int kv_end = kv_end_for(p, b);
  // key tiles up to query row `last` (its cache end and causal window)
  auto tiles_to = [&](int last) {
    int64_t lim = kv_end;
    if (p.causal) lim = min(lim, static_cast<int64_t>(last) + p.offset + 1);
    return lim > 0 ? static_cast<int>((lim + KT - 1) / KT) : 0;
  };
  const int n_tiles = __builtin_amdgcn_readfirstlane(tiles_to(min(q0 + QB2, p.Sq) - 1));
  const int s_tiles = __builtin_amdgcn_readfirstlane(qa < p.Sq ? tiles_to(min(qa + 32, p.Sq) - 1) : 0);
  const int z_tiles = __builtin_amdgcn_readfirstlane(qz < p.Sq ? tiles_to(min(qz + 32, p.Sq) - 1) : 0);
  const int w_tiles = max(s_tiles, z_tiles);

  const uint32_t ks_b = static_cast<uint32_t>(a.k.s2) * 2;
  const u32x4 kdesc = make_desc(head_ptr<T>(a.k, b, hk), static_cast<uint32_t>(kv_end) * ks_b);
  // dS of this (b, q head); the wave's subtiles are query tiles qa / 32, qz / 32
  const int64_t slice = a.ds_slice * DS_TILE;
  const u32x4 sdesc = make_desc(a.ds + static_cast<int64_t>(bhc) * slice, static_cast<uint32_t>(slice));
  // (rows past Sq: past the slice, or masked off below)
  const uint32_t dsa = static_cast<uint32_t>(ds_row_start(a.ds_tri, a.ds_nkt, qa / 32) * DS_TILE);
  const uint32_t dsz = static_cast<uint32_t>(ds_row_start(a.ds_tri, a.ds_nkt, qz / 32) * DS_TILE);
  const uint32_t lds0 = lds_addr(lds);
  const uint32_t swz_chunk = (lane & 3) ^ ((lane >> 4) & 3);
  const uint32_t koff = (lane >> 2) * ks_b + (4 * (w % QGK) + swz_chunk) * 16;
  const uint32_t loff = lane * 16;
  const uint32_t spare = lds0 + RINGS;
  const uint32_t sring = lds0 + KRING + w * SRING;
  // Per tile, as in the forward: every iteration issues the same loads; those
  // of a tile past the last one read past the range into the spare block.
  // Part u < KPARTS: this wave's u-th K block; then its dS tiles in four
  // 1 KiB parts (subtile u / 2, half u % 2), past the range (zeros) beyond the
  // subtile's causal end.
  struct DmaTile {
    uint32_t krow, kst, sst, keep, far0, far1, srow0, srow1;
  };
  auto dma_tile = [&](int tile) {
    DmaTile d;
    d.keep = ~static_cast<uint32_t>((n_tiles - 1 - tile) >> 31);  // sign fill
    const uint32_t far = ~d.keep & 0x80000000u;
    d.krow = (static_cast<uint32_t>(tile * KT) * ks_b) | far;
    d.kst = (lds0 + (tile % DS_NS) * TILE_K - spare) & d.keep;
    d.sst = (sring + (tile % DS_NS) * 2 * DS_TILE - spare) & d.keep;
    d.far0 = tile < s_tiles ? 0u : 0x80000000u;
    d.far1 = tile < z_tiles ? 0u : 0x80000000u;
    d.srow0 = (dsa + static_cast<uint32_t>(tile) * DS_TILE) | d.far0;
    d.srow1 = (dsz + static_cast<uint32_t>(tile) * DS_TILE) | d.far1;
    return d;
  };
  auto issue_part = [&](const DmaTile &d, int u) {
    if (u < KPARTS) {
      const int n = w + DQ_NW * u;  // wave-uniform
      if (n * 1024 < TILE_K)
        dma16(kdesc, spare + d.kst + ((n * 1024) & d.keep), koff,
              d.krow + static_cast<uint32_t>(16 * (n / QGK)) * ks_b);
      else
        dma16(kdesc, spare, koff, 0x80000000u);  // past the range: zeros into the spare block
    } else {
      const int s = (u - KPARTS) >> 1, half = (u - KPARTS) & 1;
      dma16_nt(sdesc, spare + d.sst + ((s * DS_TILE + half * 1024) & d.keep), loff,
               (s ? d.srow1 : d.srow0) + half * 1024);
    }
  };
  // dS^T operand (16 keys of k-step ks x 32 queries) of one stored tile by
  // transpose reads: the 16 lanes of a read group each name 4 queries of one
  // key row (dS[4 m .. 4 m + 3][k] is 8 contiguous bytes of the tile), and
  // lane (c, h) receives query c at keys 16 ks + 4 h .. + 3 (then + 8 ..),
  // the key order of TileReader::cols.  Lane (i, g) of the read (i = lane %
  // 16, g = lane / 16) names m = 4 (g % 2) + i % 4 and key row kb + i / 4,
  // kb = 16 ks + 4 h (+ 8): the stored layout's key swizzle turns into
  // per-lane bases for the two halves.
  const int i16 = lane & 15, gg = (lane >> 4) & 1, hp = i16 & 1;
  const uint32_t s_base = gg * 1024 + hp * 512 + ((i16 >> 1) & 1) * 8 + (i16 >> 2) * 16 +
                          ((h ^ hp) * 4) * 16;
  const uint32_t s_lo = s_base + (gg * 8) * 16, s_hi = s_base + ((gg ^ 1) * 8) * 16;
  auto ds_frag = [&](const char *tile, int ks) {
    const u32x2 lo = ds_read_tr<T>(reinterpret_cast<const T *>(tile + s_lo + ks * 256));
    const u32x2 hi = ds_read_tr<T>(reinterpret_cast<const T *>(tile + s_hi + ks * 256));
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };

  const TileReader<T, DK> rdk(lane);
  f32x16 acc[PDQ][2];
#pragma unroll
  for (int dt = 0; dt < PDQ; ++dt) acc[dt][0] = acc[dt][1] = f32x16{};

  for (int t = 0; t < DS_PD; ++t) {
    const DmaTile d = dma_tile(t);
#pragma unroll
    for (int u = 0; u < LPT; ++u) issue_part(d, u);
  }
  wait_vm_n<(DS_PD - 1) * LPT>();  // tile 0
  __syncthreads();

  // Iteration j: issue tile j + 2 among the MFMA steps, dQ^T += K_j^T dS_j^T
  // for both subtiles, then wait for tile j + 1 and barrier.
  auto iteration = [&](int j) {
    const DmaTile dn = dma_tile(j + DS_PD);
    const char *kt = lds + (j % DS_NS) * TILE_K;
    const char *st = lds + KRING + w * SRING + (j % DS_NS) * 2 * DS_TILE;
    u32x4 sf[2][2];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) sf[s][ks] = ds_frag(st + s * DS_TILE, ks);
    constexpr int FD = 2;
    u32x4 kf[FD + 1];
    auto load = [&](int i) { kf[i % (FD + 1)] = rdk.cols(kt, i / PDQ, i % PDQ); };
#pragma unroll
    for (int i = 0; i < FD; ++i) load(i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < STEPS; ++i) {
      const int ks = i / PDQ, dt = i % PDQ;
      acc[dt][0] = mfma32<T>(kf[i % (FD + 1)], sf[0][ks], acc[dt][0]);
      acc[dt][1] = mfma32<T>(kf[i % (FD + 1)], sf[1][ks], acc[dt][1]);
      if (i + FD < STEPS) load(i + FD);
      if (i < LPT) issue_part(dn, i);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int u = STEPS; u < LPT; ++u) issue_part(dn, u);  // D = 64: one MFMA step short
    wait_vm_n<(DS_PD - 1) * LPT>();  // tile j + 1 has landed
    wait_lgkm0();
    phase_barrier();
  };
  // Iterations past the wave's last tile only keep the DMA and barrier count.
  auto idle = [&](int j) {
    const DmaTile dn = dma_tile(j + DS_PD);
#pragma unroll
    for (int u = 0; u < LPT; ++u) issue_part(dn, u);
    wait_vm_n<(DS_PD - 1) * LPT>();
    wait_lgkm0();
    phase_barrier();
  };
  int j = 0;
  for (; j < w_tiles; ++j) iteration(j);
  for (; j < n_tiles; ++j) idle(j);
  wait_vm_n<0>();  // the last (spare-block) loads, before the epilogue reuses the rings

  // dQ rows leave through LDS, 32 rows (one subtile) per wave at a time:
  // each wave rounds them into its own slice -- row r at r * 2D bytes,
  // 16-byte chunk q at q ^ (r % CPR) -- then reads back whole 16-byte chunks
  // of rows for coalesced stores.  Lane holds dQ^T[d = 32 dt + 8 g + 4 h +
  // r][row c] of each subtile.
  constexpr int CPR = DK / 8;
  static_assert(32 * CPR % 64 == 0, "store chunks split evenly over the lanes");
  char *wslice = lds + w * 32 * 2 * DK;
  const float sc = a.scale;
  T *ob = mut<T>(a.dq) + b * a.dq.s0 + hq * a.dq.s1;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int qs = s ? qz : qa;
#pragma unroll
    for (int dt = 0; dt < PDQ; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int off = c * 2 * DK + (((4 * dt + g) ^ (c % CPR)) * 16) + 8 * h;
        *reinterpret_cast<u32x2 *>(wslice + off) =
            u32x2{pack2<T>(acc[dt][s][g * 4] * sc, acc[dt][s][g * 4 + 1] * sc),
                  pack2<T>(acc[dt][s][g * 4 + 2] * sc, acc[dt][s][g * 4 + 3] * sc)};
      }
    }
    u32x4 vr[32 * CPR / 64];
#pragma unroll
    for (int u = 0; u < 32 * CPR / 64; ++u) {
      const int idx = u * 64 + lane, r = idx / CPR, q = idx % CPR;
      vr[u] = *reinterpret_cast<const u32x4 *>(wslice + r * 2 * DK + ((q ^ (r % CPR)) * 16));
    }
    // RoPE folded in: the inverse rotation of the rounded dQ.
    if (p.rope.R > 0) {
      int64_t rows[32 * CPR / 64];
      int p0[32 * CPR / 64];
#pragma unroll
      for (int u = 0; u < 32 * CPR / 64; ++u) {
        const int idx = u * 64 + lane, r = idx / CPR, q = idx % CPR;
        rows[u] = p.rope.qpos0 + (qs + r < p.Sq ? qs + r : p.Sq - 1);  // rows past Sq: not stored
        p0[u] = 4 * q;
      }
      rotate_chunks<T, 32 * CPR / 64>(vr, p.rope, rows, p0, true);
    }
    // dQ is written once and not read back here: non-temporal stores keep
    // it from evicting the dS / K stream (255 -> 225 us at B16 H16 S2048
    // D128; the dK/dV and recomputing dQ epilogues store the same way)
#pragma unroll
    for (int u = 0; u < 32 * CPR / 64; ++u) {
      const int idx = u * 64 + lane, r = idx / CPR, q = idx % CPR;
      if (qs + r < p.Sq) __builtin_nontemporal_store(vr[u], reinterpret_cast<u32x4 *>(ob + static_cast<int64_t>(qs + r) * a.dq.s2 + q * 8));
    }
  }
}

// MKQ: the dQ kernel's mask mode (0..6), MK the dK/dV kernel's: element reads
// (1..3), or boolean / 16-bit row-piece masks staged through its LDS ring
// (4, 6); f32 row-piece masks (5) read element by element there.
template <typename T, int DK, int DV, int MKQ, int MK, bool DR>
void launch_mk(const BwdArgs &a0, hipStream_t st) {
  const Problem &p = a0.p;
  BwdArgs a = a0;
  // (stored dS only with a 128-wide head: the sizing gives the others none)
  if constexpr (DK == 128 || DV == 128) {
  if (a.ds) {
    // Stored dS: row values, then per chunk of KV-head groups (one chunk
    // unless the dS of every group exceeds the region's cap) dK/dV storing
    // the chunk's dS, then its dQ as one GEMM.
    {
      Probe pr_("bwd_rows", st);
      const int per_block = (NT / 64) * (64 / (DV / 8)) * ROWS_U;
      const int nqb = (p.Sq + per_block - 1) / per_block;
      bwd_rows_kernel<T, DK, DV><<<dim3(static_cast<unsigned>(static_cast<int64_t>(nqb) * p.B * p.Hq)),
                                  dim3(NT), 0, st>>>(a, nqb);
    }
    const int groups = p.B * p.Hkv, per_chunk = mfma_ds_chunk_groups(p);
    const int n_kb = (p.Sk + KB - 1) / KB, n_qb = (p.Sq + QB2 - 1) / QB2;
    for (a.g0 = 0; a.g0 < groups; a.g0 += per_chunk) {
      a.ng = min(per_chunk, groups - a.g0);
      {
        Probe pr_(DR ? "bwd_dkdv_mfma_dropout" : (MK ? "bwd_dkdv_mfma_masked" : "bwd_dkdv_mfma"), st);
        dkdv_kernel<T, DK, DV, MK, DR><<<dim3(n_kb * a.ng), dim3(NT), 0, st>>>(a);
      }
      {
        Probe pr_(DR ? "bwd_dq_ds_dropout" : (MK ? "bwd_dq_ds_masked" : "bwd_dq_ds"), st);
        dq_ds_kernel<T, DK><<<dim3(n_qb * a.ng * p.rep), dim3(DQ_NT), 0, st>>>(a);
      }
    }
    return;
  }
  }
  a.ds = nullptr;  // (the recomputing pipeline stores no dS)
  // dQ first: its prologue writes the nd / nl row values the dK/dV kernel reads.
  const int n_qb = (p.Sq + QB - 1) / QB;
  {
    Probe pr_(DR ? "bwd_dq_mfma_dropout" : (MK ? "bwd_dq_mfma_masked" : "bwd_dq_mfma"), st);
    dq_kernel<T, DK, DV, MKQ, DR><<<dim3(n_qb * p.Hq * p.B), dim3(NT), 0, st>>>(a);
  }
  const int n_kb = (p.Sk + KB - 1) / KB;
  {
    Probe pr_(DR ? "bwd_dkdv_mfma_dropout" : (MK ? "bwd_dkdv_mfma_masked" : "bwd_dkdv_mfma"), st);
    dkdv_kernel<T, DK, DV, MK, DR><<<dim3(n_kb * a.ng), dim3(NT), 0, st>>>(a);
  }
}

template <typename T, int DK, int DV, bool DR>
void launch_dr(const BwdArgs &a, int mkq, hipStream_t st) {
  switch (mkq) {
    case 1: launch_mk<T, DK, DV, 1, 1, DR>(a, st); break;
    case 2: launch_mk<T, DK, DV, 2, 2, DR>(a, st); break;
    case 3: launch_mk<T, DK, DV, 3, 3, DR>(a, st); break;
    case 4: launch_mk<T, DK, DV, 4, 4, DR>(a, st); break;
    case 5: launch_mk<T, DK, DV, 5, 2, DR>(a, st); break;  // f32 tiles: too much LDS to stage
    case 6: launch_mk<T, DK, DV, 6, 6, DR>(a, st); break;
    default: launch_mk<T, DK, DV, 0, 0, DR>(a, st); break;
  }
}

template <typename T, int DK, int DV>
void launch_dims(const BwdArgs &a, hipStream_t st) {
  const int mkq = mfma_mask_mode_vec(a.p);
  if (a.p.drop.on) launch_dr<T, DK, DV, true>(a, mkq, st);
  else launch_dr<T, DK, DV, false>(a, mkq, st);
}

template <typename T>
hipError_t launch(const BwdArgs &a, hipStream_t st) {
  const Problem &p = a.p;
  if (p.Dqk == 128 && p.Dv == 128) launch_dims<T, 128, 128>(a, st);
  else if (p.Dqk == 64 && p.Dv == 64) launch_dims<T, 64, 64>(a, st);
  else if (p.Dqk == 32) launch_dims<T, 32, 32>(a, st);
  else if (p.Dqk == 128) launch_dims<T, 128, 64>(a, st);
  else launch_dims<T, 64, 128>(a, st);
  return hipGetLastError();
}

}  // namespace

size_t mfma_rope_stage_offset(const Problem &p) {
  const size_t rows = static_cast<size_t>(p.B) * p.Hq * p.Sq;
  return (2 * rows * sizeof(float) + 255) / 256 * 256;
}

// Key tiles of stored dS per query tile: every 32-key tile of the dK/dV
// kernel's 128-key blocks, including those past the keys (zeros, never read).
static int ds_key_tiles(const Problem &p) { return (p.Sk + KB - 1) / KB * (KB / 32); }

static int ds_packed(const Problem &p) { return p.causal && p.offset == 0 && p.Sq == p.Sk; }

static int64_t ds_slice_tiles(const Problem &p) {
  return ds_row_start(ds_packed(p), ds_key_tiles(p), (p.Sq + 31) / 32);
}

// The stored-dS region holds at most 8 GiB, and each (b, q head) slice stays
// within 2^31 bytes (32-bit buffer offsets, bit 31 marking a zero read).
// When the dS of every KV-head group (its rep query heads) does not fit, the
// backward runs over chunks of groups that reuse one region: as few chunks
// as fit the cap, of (nearly) equal size.  0: no stored dS (a slice alone is
// too large).
//
// Stored dS pays only with a 128-wide head: its HBM round trip (written by
// dK/dV, read by dQ) does not shrink with the head dim, while the recomputing
// dQ kernel's S and dP products do.  With both dims 64 or below the
// recomputing kernel is the faster backward (B16 H16 S2048 causal bf16: D32
// 0.37 against 0.49 ms, D64 0.54 against 0.63 ms; D128 0.96 against 0.89 ms
// the other way; 128 / 64 mixed within 1%), so those problems store none.
static int ds_chunk_groups(const Problem &p, int64_t *bytes) {
  constexpr int64_t kCap = int64_t(8) << 30;
  const int64_t slice = ds_slice_tiles(p) * DS_TILE;
  const int64_t per_group = slice * p.rep;
  const int groups = p.B * p.Hkv;
  if ((p.Dqk < 128 && p.Dv < 128) || slice > (int64_t(1) << 31) || per_group > kCap || groups <= 0) {
    *bytes = 0;
    return 0;
  }
  const int64_t max_groups = kCap / per_group;
  const int64_t chunks = (groups + max_groups - 1) / max_groups;
  const int per_chunk = static_cast<int>((groups + chunks - 1) / chunks);
  *bytes = per_chunk * per_group;
  return per_chunk;
}

int mfma_ds_chunk_groups(const Problem &p) {
  int64_t bytes;
  return ds_chunk_groups(p, &bytes);
}

size_t mfma_ds_bytes(const Problem &p) {
  int64_t bytes;
  ds_chunk_groups(p, &bytes);
  return static_cast<size_t>(bytes);
}

hipError_t launch_mfma_backward(const Problem &p, int dtype, View q, View k, View v, View o,
                                View dout, const float *lse, View dq, View dk, View dv,
                                float *delta, void *ds, hipStream_t st) {
  View qk = q;
  if (p.rope.R > 0) {
    // rotated query rows: the forward's (rope.qrot), or staged after the row
    // values, 256-byte aligned
    const int64_t D = p.Dqk;
    void *rows = p.rope.qrot ? p.rope.qrot : reinterpret_cast<char *>(delta) + mfma_rope_stage_offset(p);
    qk = View{rows, static_cast<int64_t>(p.Hq) * p.Sq * D, static_cast<int64_t>(p.Sq) * D, D};
  }
  BwdArgs a{p, q, k, v, o, dout, dq, dk, dv, qk, lse, delta,
            static_cast<float>(p.scale) * kLog2e, static_cast<float>(p.scale),
            static_cast<char *>(ds), ds_key_tiles(p), ds_packed(p), ds_slice_tiles(p),
            0, p.B * p.Hkv};
  return dtype == TSATTN_BF16 ? launch<bf16>(a, st) : launch<f16>(a, st);
}

}  // namespace tsattn
