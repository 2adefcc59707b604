// Internal declarations shared by the libtsattn.so translation units.
// Everything here is gfx950-only HIP; nothing is exported except through
// include/tsattn.h.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "tsattn.h"

namespace tsattn {

// ---------------------------------------------------------------------------
// Element types and conversions (storage T <-> accumulator A).
// ---------------------------------------------------------------------------
using bf16 = __bf16;
using f16 = _Float16;

template <typename A, typename T>
__device__ __forceinline__ A to_acc(T x) {
  return static_cast<A>(static_cast<float>(x));
}
template <>
__device__ __forceinline__ double to_acc<double, double>(double x) {
  return x;
}
template <>
__device__ __forceinline__ float to_acc<float, float>(float x) {
  return x;
}

template <typename T, typename A>
__device__ __forceinline__ T from_acc(A x) {
  return static_cast<T>(x);  // RNE on gfx950 (v_cvt_pk_bf16_f32 / v_cvt_f16_f32)
}

// Reads one element of a mask of runtime dtype as the accumulator type.
template <typename A>
__device__ __forceinline__ A load_additive(const void *base, int64_t idx, int dtype) {
  switch (dtype) {
    case TSATTN_F64: return static_cast<A>(static_cast<const double *>(base)[idx]);
    case TSATTN_F16: return static_cast<A>(static_cast<float>(static_cast<const f16 *>(base)[idx]));
    case TSATTN_BF16:
      return static_cast<A>(static_cast<float>(static_cast<const bf16 *>(base)[idx]));
    default: return static_cast<A>(static_cast<const float *>(base)[idx]);
  }
}

// ---------------------------------------------------------------------------
// Launch descriptors (plain structs passed by value to kernels).
// ---------------------------------------------------------------------------
struct View {
  const void *data;
  int64_t s0, s1, s2;  // batch, head, sequence strides (elements); dim stride is 1
};

inline View make_view(const tsattn_view *v) {
  return View{v->data, v->stride[0], v->stride[1], v->stride[2]};
}

struct MaskDesc {
  int kind;   // tsattn_mask_kind
  int dtype;  // TSATTN_BOOL or a float type
  const void *data;
  int64_t s0, s1, s2, s3;
};

// RoPE folded into the MFMA attention kernels: cos / sin tables [*, R / 2]
// in the tensor dtype; query row i at position qpos0 + i, key row j at
// kpos0 + j.  R = 0: none.
struct RopeDesc {
  const void *cos, *sin;
  int R;
  int64_t qpos0, kpos0;
  void *qrot;  // rotated query rows [B, Hq, Sq, Dqk]: written by the forward, read by the backward
};

// Attention dropout (on = 0: none): keep a 16-bit word w iff w >= thr, kept
// probabilities times `scale` (f32 compute) / `scale64` (f64 compute), the
// reference's keep.astype(compute dtype) / (1 - p); Philox4x32 key k0 (two
// 32-bit words), stream words k1 (the high half of every block counter) and
// stream counter c0 (philox.h); c1 unused.
struct DropDesc {
  int on;
  uint32_t thr;
  float scale;
  double scale64;
  uint64_t k0, k1, c0, c1;
  // keep bits (tsattn_problem.dropout_bits layout): word ((b Hq + h) nkt + t)
  // sqp + i holds keys 32 t .. 32 t + 31 of row i; nkt = ceil(Sk / 32),
  // sqp = Sq rounded up to 4
  uint32_t *bits;
  int nkt, sqp;
};

struct Problem {
  int B, Hq, Hkv, Sq, Sk, Dqk, Dv, rep;
  double scale;
  int causal;
  int64_t offset;
  const int32_t *kv_len;
  const int32_t *kv_prefix;
  MaskDesc mask;
  RopeDesc rope;
  DropDesc drop;
};

// Mask handling of the MFMA kernels (a template parameter): 0 = none, or a
// key mask [B,1,1,K] reduced to kv_len / kv_prefix; 1 = any other boolean
// mask, read per (row, key) from its strides; 2 / 3 = an additive f32 /
// (f16 or bf16) mask, read the same way and added to the scaled scores.
inline int mfma_mask_mode(const Problem &p) {
  if (p.mask.kind == TSATTN_MASK_BOOL)
    return p.mask.s1 == 0 && p.mask.s2 == 0 && p.kv_len != nullptr ? 0 : 1;
  if (p.mask.kind != TSATTN_MASK_ADDITIVE) return 0;
  return p.mask.dtype == TSATTN_F32 ? 2 : 3;
}
// The same, read as 16-byte row pieces (modes 4..6) where the keys are
// contiguous and every row starts 16-byte aligned.
inline int mfma_mask_mode_vec(const Problem &p) {
  const int mk = mfma_mask_mode(p);
  if (mk == 0) return 0;
  const int64_t es = mk == 1 ? 1 : (mk == 2 ? 4 : 2);
  const MaskDesc &m = p.mask;
  const bool ok = m.s3 == 1 && (m.s0 * es) % 16 == 0 && (m.s1 * es) % 16 == 0 &&
                  (m.s2 * es) % 16 == 0 && reinterpret_cast<uintptr_t>(m.data) % 16 == 0;
  return ok ? mk + 3 : mk;
}

// Valid keys for batch row b: [0, kv_end).
__device__ __forceinline__ int kv_end_for(const Problem &p, int b) {
  int e = p.Sk;
  if (p.kv_len) {
    int l = p.kv_len[b];
    e = l < e ? l : e;
    e = e < 0 ? 0 : e;
  }
  return e;
}

// ---------------------------------------------------------------------------
// Kernel timing probes: when enabled (tsattn_profile_enable), every kernel
// launch is bracketed by hipEvents recorded on its own stream; durations are
// aggregated per kernel name by tsattn_profile_read.  Disabled: one relaxed
// atomic load per launch.
// ---------------------------------------------------------------------------
bool probes_on();
void probe_begin(const char *name, hipStream_t st);
void probe_end(hipStream_t st);

struct Probe {
  bool on;
  hipStream_t st;
  Probe(const char *name, hipStream_t s) : on(probes_on()), st(s) {
    if (on) probe_begin(name, st);
  }
  ~Probe() {
    if (on) probe_end(st);
  }
};

// ---------------------------------------------------------------------------
// Launchers (each returns hipSuccess or the launch error).
// ---------------------------------------------------------------------------
hipError_t launch_generic_forward(const Problem &p, int dtype, View q, View k, View v, View o,
                                  void *lse, hipStream_t st);
hipError_t launch_generic_backward(const Problem &p, int dtype, View q, View k, View v, View o,
                                   View dout, const void *lse, View dq, View dk, View dv,
                                   void *delta, hipStream_t st);

// MFMA kernels: f16 / bf16, dim_qk and dim_v each in {64, 128}, scale > 0; any
// boolean mask, or an additive mask in f32 / f16 / bf16.
bool mfma_supported(const Problem &p, int dtype);
hipError_t launch_mfma_forward(const Problem &p, int dtype, View q, View k, View v, View o,
                               float *lse, hipStream_t st);
// ds: NULL, or mfma_ds_bytes(p) bytes in which the dK/dV kernel stores dS
// for the dQ product (then it runs first and dQ takes one GEMM).
hipError_t launch_mfma_backward(const Problem &p, int dtype, View q, View k, View v, View o,
                                View dout, const float *lse, View dq, View dk, View dv,
                                float *delta, void *ds, hipStream_t st);
// Bytes of the stored-dS region (bf16 / f16 32 x 32 tiles of the (b, q
// head) slices of one chunk of KV-head groups; every group when they fit the
// cap the backward keeps on its workspace), or 0 when one slice is too large.
size_t mfma_ds_bytes(const Problem &p);
// KV-head groups (b, kv head) per chunk of the stored-dS backward.
int mfma_ds_chunk_groups(const Problem &p);
// With RoPE folded in (p.rope.R > 0) the backward workspace also holds the
// rotated query rows [B, Hq, Sq, Dqk] (16-bit) from this byte offset on.
size_t mfma_rope_stage_offset(const Problem &p);

// fp32 MFMA kernels (mfma_f32.hip): fp32, Dqk = Dv in {32, 64, 128}, no
// dropout / folded RoPE, masks none or a key mask reduced to lengths.
bool mfma_f32_supported(const Problem &p, int dtype);
hipError_t launch_mfma_f32_forward(const Problem &p, View q, View k, View v, View o, float *lse,
                                   hipStream_t st);
// rows: the backward workspace's row values (2 B Hq Sq floats).
hipError_t launch_mfma_f32_backward(const Problem &p, View q, View k, View v, View o, View dout,
                                    const float *lse, View dq, View dk, View dv, float *rows,
                                    hipStream_t st);

// Split-K decode.
bool decode_supported(const Problem &p, int dtype);
size_t decode_workspace_bytes(const Problem &p, int split_len);
// Device address of this GPU's decode scratch array (TSATTN_DECODE_SCRATCH_BYTES),
// looked up once per device with that device current.
hipError_t decode_scratch(void **ptr);
hipError_t launch_decode(const Problem &p, int dtype, View q, View k, View v, View o,
                         int split_len, void *workspace, hipStream_t st);
// The same over an int8 cache with fp32 row scales ks / vs [B, Hkv, capacity, 1].
hipError_t launch_decode_int8(const Problem &p, int dtype, View q, View k, View v, View ks,
                              View vs, View o, int split_len, void *workspace, hipStream_t st);

// int8 KV-cache append: rows src[b, h, t, :] (dtype f32 / f16 / bf16) are
// quantised into dst[b, h, pos + t, :] with their scale at scale[b, h, pos + t].
hipError_t launch_kv_append_int8(int dtype, int B, int H, int T, int D, View src, View dst,
                                 View scale, int64_t pos, hipStream_t st);

// Interleaved-pair RoPE of x [B, H, T, D] into out (may alias x), cos / sin
// tables [*, R / 2] in the tensor dtype, rows pos0 .. pos0 + T - 1.
hipError_t launch_rope(int dtype, int B, int H, int T, int D, int R, View x, View out,
                       const void *cos, const void *sin, int64_t pos0, int inverse, hipStream_t st);
// RoPE of the new K rows (R = 0: none) fused with the K/V cache append at
// `pos`; ks / vs non-null for int8 caches (then quantised as the int8 append).
hipError_t launch_rope_append(int dtype, int B, int H, int T, int D, int R, View k, View v, View kc,
                              View vc, const View *ks, const View *vs, const void *cos,
                              const void *sin, int64_t pos, hipStream_t st);

// The q / k / v projections of the `batch x len` rows of x (embed wide; a
// [batch, 1, len, embed] view) with
// RoPE of q and k at rows pos .. (cos == nullptr: none) and the k / v cache
// append at pos; ks / vs non-null for int8 caches.  dim is 64 or 128.
hipError_t launch_qkv_rope_append(int dtype, int batch, int len, int embed, int heads_q, int heads_kv,
                                  int dim, View x, const void *const w[3], const void *const bias[3],
                                  View q, View kc, View vc, const View *ks, const View *vs, const void *cos,
                                  const void *sin, int64_t pos, hipStream_t st);

// The dropout keep mask of problem p as a contiguous [B, Hq, Sq, Sk] uint8 array.
hipError_t launch_dropout_keep(const Problem &p, uint8_t *out, hipStream_t st);
// The keep bits of the problem's dropout stream into `out` (DropDesc::bits
// layout, dropout_bits_bytes long).
hipError_t launch_dropout_bits(const Problem &p, uint32_t *out, hipStream_t st);
inline size_t dropout_bits_bytes(const Problem &p) {
  return static_cast<size_t>(p.B) * p.Hq * ((p.Sk + 31) / 32) * ((p.Sq + 3) / 4 * 4) *
         sizeof(uint32_t);
}

hipError_t launch_key_mask_lengths(const uint8_t *mask, int64_t sb, int64_t sk, int B, int K,
                                   int32_t *kv_len, int32_t *kv_prefix, hipStream_t st);

}  // namespace tsattn
