// C-ABI entry points of libtsattn.so (declared in include/tsattn.h).
//
// Validation mirrors the contract checks of the reference's
// scaled_dot_product_attention (src/tensorsmith/nn/attention.py:36-62) so a
// caller binding the library directly gets the same refusals; the Python
// host layer maps TSATTN_ERR_INVALID to ValueError / TypeError.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

#include "mfma_common.h"

namespace {

thread_local char g_error[512] = "";
std::atomic<int> g_policy{0};     // 0 auto, 1 generic kernels only
thread_local int g_last_path = 0; // 0 none, 1 generic, 2 mfma, 3 decode

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char *where) {
  if (e == hipSuccess) return TSATTN_OK;
  return fail(TSATTN_ERR_HIP, "%s: %s", where, hipGetErrorString(e));
}

bool is_float_dtype(int d) {
  return d == TSATTN_F32 || d == TSATTN_F16 || d == TSATTN_BF16 || d == TSATTN_F64;
}

int check_view(const tsattn_view *v, const char *name) {
  if (!v) return fail(TSATTN_ERR_INVALID, "%s view is NULL", name);
  if (!v->data) return fail(TSATTN_ERR_INVALID, "%s data pointer is NULL", name);
  if (v->stride[3] != 1) return fail(TSATTN_ERR_INVALID, "%s innermost stride must be 1", name);
  return TSATTN_OK;
}

int check_problem(const tsattn_problem *p, tsattn::Problem *out) {
  if (!p) return fail(TSATTN_ERR_INVALID, "problem is NULL");
  if (!is_float_dtype(p->dtype))
    return fail(TSATTN_ERR_INVALID, "attention inputs must have the same floating-point dtype");
  if (p->batch <= 0 || p->heads_q <= 0 || p->heads_kv <= 0 || p->len_q <= 0 || p->len_kv <= 0 ||
      p->dim_qk <= 0 || p->dim_v <= 0)
    return fail(TSATTN_ERR_INVALID, "query/key head dimensions must match and sequences must be nonempty");
  if (p->heads_q % p->heads_kv)
    return fail(TSATTN_ERR_INVALID,
                "grouped-query attention requires enable_gqa and query heads divisible by KV heads");
  if (!isfinite(p->scale)) return fail(TSATTN_ERR_INVALID, "attention scale must be finite");
  if (p->causal_offset < 0)
    return fail(TSATTN_ERR_INVALID, "invalid dropout probability, block size, or causal offset");
  if (p->mask_kind != TSATTN_MASK_NONE) {
    if (p->mask_kind != TSATTN_MASK_BOOL && p->mask_kind != TSATTN_MASK_ADDITIVE)
      return fail(TSATTN_ERR_INVALID, "unknown mask kind %d", p->mask_kind);
    if (!p->mask.data) return fail(TSATTN_ERR_INVALID, "mask data pointer is NULL");
    if (p->mask_kind == TSATTN_MASK_BOOL && p->mask_dtype != TSATTN_BOOL)
      return fail(TSATTN_ERR_INVALID, "boolean masks must have dtype TSATTN_BOOL");
    if (p->mask_kind == TSATTN_MASK_ADDITIVE && !is_float_dtype(p->mask_dtype))
      return fail(TSATTN_ERR_INVALID, "attention masks must be boolean or floating point");
  }
  if (!(p->dropout_p >= 0.0 && p->dropout_p < 1.0))
    return fail(TSATTN_ERR_INVALID, "invalid dropout probability, block size, or causal offset");
  if (p->dim_qk > 512 || p->dim_v > 512)
    return fail(TSATTN_ERR_UNSUPPORTED, "head dims above 512 are not supported (got %d/%d)",
                p->dim_qk, p->dim_v);
  tsattn::Problem q{};
  q.B = p->batch;
  q.Hq = p->heads_q;
  q.Hkv = p->heads_kv;
  q.Sq = p->len_q;
  q.Sk = p->len_kv;
  q.Dqk = p->dim_qk;
  q.Dv = p->dim_v;
  q.rep = p->heads_q / p->heads_kv;
  q.scale = p->scale;
  q.causal = p->is_causal ? 1 : 0;
  q.offset = p->causal_offset;
  q.kv_len = p->kv_len;
  q.kv_prefix = p->kv_prefix;
  q.mask.kind = p->mask_kind;
  q.mask.dtype = p->mask_dtype;
  q.mask.data = p->mask.data;
  // A stride along a dimension of extent 1 is never applied; zeroing it lets
  // the kernels recognise a [B,1,1,K] key-padding mask by its strides alone
  // (e.g. a decode step's query dimension of length 1).
  q.mask.s0 = p->batch == 1 ? 0 : p->mask.stride[0];
  q.mask.s1 = p->heads_q == 1 ? 0 : p->mask.stride[1];
  q.mask.s2 = p->len_q == 1 ? 0 : p->mask.stride[2];
  q.mask.s3 = p->len_kv == 1 ? 0 : p->mask.stride[3];
  if (p->dropout_p > 0.0) {
    // keep iff word >= round-half-even(65536 p); kept values times f32(1) / f32(1 - p)
    q.drop.on = 1;
    q.drop.thr = static_cast<uint32_t>(fmin(nearbyint(p->dropout_p * 65536.0), 65536.0));
    q.drop.scale = 1.0f / static_cast<float>(1.0 - p->dropout_p);
    q.drop.scale64 = 1.0 / (1.0 - p->dropout_p);
    q.drop.k0 = p->dropout_key[0];
    q.drop.k1 = p->dropout_key[1];
    q.drop.c0 = p->dropout_counter;
    q.drop.c1 = 0;
    q.drop.bits = p->dropout_bits;
    q.drop.nkt = (q.Sk + 31) / 32;
    q.drop.sqp = (q.Sq + 3) / 4 * 4;
  }
  *out = q;
  return TSATTN_OK;
}

size_t acc_size(int dtype) { return dtype == TSATTN_F64 ? sizeof(double) : sizeof(float); }

// The MFMA kernels address each (b, h) slice of a view with 32-bit buffer
// offsets and a 32-bit range bound: route only 16-byte aligned views whose
// slice of `len` rows, plus a margin for padded tiles, stays below 2^31 bytes.
// A zero sequence stride (a broadcast row) would make the range bound zero.
bool mfma_view_ok(const tsattn::View &v, int64_t len) {
  return tsattn::aligned16(v) && v.s2 > 0 && (len + 256) * v.s2 * 2 < (int64_t(1) << 31);
}

// The same for the fp32 MFMA kernels (4-byte elements).
bool mfma_f32_view_ok(const tsattn::View &v, int64_t len) {
  return reinterpret_cast<uintptr_t>(v.data) % 16 == 0 && v.s0 % 4 == 0 && v.s1 % 4 == 0 &&
         v.s2 % 4 == 0 && v.s2 > 0 && (len + 256) * v.s2 * 4 < (int64_t(1) << 31);
}

// The forward / backward behind the plain and the RoPE entry points.  With a
// RoPE descriptor only the MFMA kernels apply (they fold the rotation in).
int check_rope(const tsattn_rope_desc *r, const tsattn::Problem &pr, tsattn::RopeDesc *out) {
  if (!r->cos || !r->sin) return fail(TSATTN_ERR_INVALID, "RoPE needs cos / sin tables");
  if (r->rotary_dim <= 0 || r->rotary_dim % 2 || r->rotary_dim > pr.Dqk || r->q_pos0 < 0 ||
      r->k_pos0 < 0)
    return fail(TSATTN_ERR_INVALID,
                "RoPE requires a positive even rotary dimension and valid positions/base");
  if (r->rotary_dim % 8)
    return fail(TSATTN_ERR_UNSUPPORTED,
                "RoPE folded into attention needs a rotary dim divisible by 8 (got %d); rotate "
                "with tsattn_rope instead", r->rotary_dim);
  if (reinterpret_cast<uintptr_t>(r->cos) % 8 || reinterpret_cast<uintptr_t>(r->sin) % 8)
    return fail(TSATTN_ERR_UNSUPPORTED, "RoPE tables must be 8-byte aligned; rotate with tsattn_rope instead");
  if (reinterpret_cast<uintptr_t>(r->q_rotated) % 16)
    return fail(TSATTN_ERR_INVALID, "the rotated-query buffer must be 16-byte aligned");
  *out = tsattn::RopeDesc{r->cos, r->sin, r->rotary_dim, r->q_pos0, r->k_pos0, r->q_rotated};
  return TSATTN_OK;
}

int rope_unsupported() {
  return fail(TSATTN_ERR_UNSUPPORTED,
              "RoPE folded into attention needs the MFMA kernels (f16/bf16, dim_qk and dim_v in "
              "{64, 128}, 16-byte aligned views); rotate with tsattn_rope instead");
}

int sdpa_forward(const tsattn_problem *p, const tsattn_rope_desc *rope, const tsattn_view *q,
                 const tsattn_view *k, const tsattn_view *v, const tsattn_view *out, void *lse,
                 void *stream) {
  tsattn::Problem pr;
  int rc = check_problem(p, &pr);
  if (rc) return rc;
  if ((rc = check_view(q, "query")) || (rc = check_view(k, "key")) ||
      (rc = check_view(v, "value")) || (rc = check_view(out, "output")))
    return rc;
  if (rope && (rc = check_rope(rope, pr, &pr.rope))) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  tsattn::View vq = tsattn::make_view(q), vk = tsattn::make_view(k), vv = tsattn::make_view(v),
               vo = tsattn::make_view(out);
  if (g_policy.load() == 0 && tsattn::mfma_supported(pr, p->dtype) && mfma_view_ok(vq, pr.Sq) &&
      mfma_view_ok(vk, pr.Sk) && mfma_view_ok(vv, pr.Sk) && mfma_view_ok(vo, pr.Sq)) {
    g_last_path = 2;
    return hip_status(tsattn::launch_mfma_forward(pr, p->dtype, vq, vk, vv, vo,
                                                  static_cast<float *>(lse), st),
                      "mfma forward launch");
  }
  if (rope) return rope_unsupported();
  if (g_policy.load() == 0 && tsattn::mfma_f32_supported(pr, p->dtype) && mfma_f32_view_ok(vq, pr.Sq) &&
      mfma_f32_view_ok(vk, pr.Sk) && mfma_f32_view_ok(vv, pr.Sk) && mfma_f32_view_ok(vo, pr.Sq)) {
    g_last_path = 2;
    return hip_status(tsattn::launch_mfma_f32_forward(pr, vq, vk, vv, vo, static_cast<float *>(lse), st),
                      "fp32 mfma forward launch");
  }
  g_last_path = 1;
  rc = hip_status(tsattn::launch_generic_forward(pr, p->dtype, vq, vk, vv, vo, lse, st),
                  "generic forward launch");
  // the generic kernels draw their keep bits on the fly: write them out too
  if (!rc && pr.drop.on && pr.drop.bits)
    rc = hip_status(tsattn::launch_dropout_bits(pr, pr.drop.bits, st), "dropout bits launch");
  return rc;
}

size_t round256(size_t n) { return (n + 255) / 256 * 256; }

// Row deltas, then (MFMA path) the row LSE terms.
size_t rows_workspace(const tsattn_problem *p) {
  if (!p || p->batch <= 0 || p->heads_q <= 0 || p->len_q <= 0) return 0;
  return 2 * static_cast<size_t>(p->batch) * p->heads_q * p->len_q * acc_size(p->dtype);
}

// Row values (as above), then the rotated query rows the dK/dV kernel reads.
size_t rope_rows_workspace(const tsattn::Problem &pr) {
  return tsattn::mfma_rope_stage_offset(pr) +
         static_cast<size_t>(pr.B) * pr.Hq * pr.Sq * pr.Dqk * 2;
}

// When dropping, room after those for the keep bits the MFMA backward draws
// when the problem brings none from its forward.
size_t with_bits(size_t base, const tsattn::Problem &pr) {
  return pr.drop.on ? round256(base) + tsattn::dropout_bits_bytes(pr) : base;
}

// Then (MFMA kernels) room for stored dS, with which the dK/dV kernel runs
// first and dQ takes one GEMM instead of recomputing S and dP; a smaller
// workspace runs the recomputing dQ kernel.
size_t with_ds(size_t base, const tsattn::Problem &pr, int dtype) {
  if (!tsattn::mfma_supported(pr, dtype)) return base;
  const size_t ds = tsattn::mfma_ds_bytes(pr);
  return ds ? round256(base) + ds : base;
}

size_t backward_workspace(const tsattn_problem *p) {
  const size_t base = rows_workspace(p);
  tsattn::Problem pr;
  if (!base || check_problem(p, &pr)) return base;
  return with_ds(with_bits(base, pr), pr, p->dtype);
}

size_t rope_backward_workspace(const tsattn::Problem &pr, int dtype) {
  return with_ds(with_bits(rope_rows_workspace(pr), pr), pr, dtype);
}

int sdpa_backward(const tsattn_problem *p, const tsattn_rope_desc *rope, const tsattn_view *q,
                  const tsattn_view *k, const tsattn_view *v, const tsattn_view *out,
                  const tsattn_view *dout, const void *lse, const tsattn_view *dq,
                  const tsattn_view *dk, const tsattn_view *dv, void *workspace,
                  size_t workspace_bytes, void *stream) {
  tsattn::Problem pr;
  int rc = check_problem(p, &pr);
  if (rc) return rc;
  if ((rc = check_view(q, "query")) || (rc = check_view(k, "key")) ||
      (rc = check_view(v, "value")) || (rc = check_view(out, "output")) ||
      (rc = check_view(dout, "upstream gradient")) || (rc = check_view(dq, "dq")) ||
      (rc = check_view(dk, "dk")) || (rc = check_view(dv, "dv")))
    return rc;
  if (!lse) return fail(TSATTN_ERR_INVALID, "backward needs the saved LSE");
  if (rope && (rc = check_rope(rope, pr, &pr.rope))) return rc;
  const size_t rows_need = rope ? rope_rows_workspace(pr) : rows_workspace(p);
  if (!workspace || workspace_bytes < rows_need)
    return fail(TSATTN_ERR_INVALID, "backward workspace too small: %zu < %zu bytes",
                workspace_bytes, rows_need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  tsattn::View vq = tsattn::make_view(q), vk = tsattn::make_view(k), vv = tsattn::make_view(v),
               vo = tsattn::make_view(out), vg = tsattn::make_view(dout),
               vdq = tsattn::make_view(dq), vdk = tsattn::make_view(dk),
               vdv = tsattn::make_view(dv);
  if (g_policy.load() == 0 && tsattn::mfma_supported(pr, p->dtype) && mfma_view_ok(vq, pr.Sq) &&
      mfma_view_ok(vk, pr.Sk) && mfma_view_ok(vv, pr.Sk) && mfma_view_ok(vo, pr.Sq) &&
      mfma_view_ok(vg, pr.Sq) && mfma_view_ok(vdq, pr.Sq) && mfma_view_ok(vdk, pr.Sk) &&
      mfma_view_ok(vdv, pr.Sk)) {
    if (pr.drop.on && !pr.drop.bits) {
      // no bits from the forward: draw them into the workspace, after the rows
      const size_t need = with_bits(rows_need, pr);
      if (workspace_bytes < need)
        return fail(TSATTN_ERR_INVALID,
                    "backward workspace too small for the dropout bits: %zu < %zu bytes",
                    workspace_bytes, need);
      pr.drop.bits = reinterpret_cast<uint32_t *>(static_cast<char *>(workspace) + round256(rows_need));
      if ((rc = hip_status(tsattn::launch_dropout_bits(pr, pr.drop.bits, st), "dropout bits launch")))
        return rc;
    }
    // stored dS when the workspace has room for it (as sized by the query)
    void *ds = nullptr;
    const size_t ds_bytes = tsattn::mfma_ds_bytes(pr);
    const size_t ds_off = round256(with_bits(rows_need, pr));
    if (ds_bytes && workspace_bytes >= ds_off + ds_bytes) ds = static_cast<char *>(workspace) + ds_off;
    g_last_path = 2;
    return hip_status(tsattn::launch_mfma_backward(pr, p->dtype, vq, vk, vv, vo, vg,
                                                   static_cast<const float *>(lse), vdq, vdk,
                                                   vdv, static_cast<float *>(workspace), ds, st),
                      "mfma backward launch");
  }
  if (rope) return rope_unsupported();
  if (g_policy.load() == 0 && tsattn::mfma_f32_supported(pr, p->dtype) && mfma_f32_view_ok(vq, pr.Sq) &&
      mfma_f32_view_ok(vk, pr.Sk) && mfma_f32_view_ok(vv, pr.Sk) && mfma_f32_view_ok(vo, pr.Sq) &&
      mfma_f32_view_ok(vg, pr.Sq) && mfma_f32_view_ok(vdq, pr.Sq) && mfma_f32_view_ok(vdk, pr.Sk) &&
      mfma_f32_view_ok(vdv, pr.Sk)) {
    g_last_path = 2;
    return hip_status(tsattn::launch_mfma_f32_backward(pr, vq, vk, vv, vo, vg, static_cast<const float *>(lse),
                                                       vdq, vdk, vdv, static_cast<float *>(workspace), st),
                      "fp32 mfma backward launch");
  }
  g_last_path = 1;
  return hip_status(tsattn::launch_generic_backward(pr, p->dtype, vq, vk, vv, vo, vg, lse, vdq,
                                                    vdk, vdv, workspace, st),
                    "generic backward launch");
}

// Decode over a 16-bit cache (k_scale == v_scale == NULL) or an int8 one,
// with the query rotation folded in when `rope` is given.
int decode_forward(const tsattn_problem *p, const tsattn_rope_desc *rope, const tsattn_view *q,
                   const tsattn_view *k, const tsattn_view *v, const tsattn_view *k_scale,
                   const tsattn_view *v_scale, const tsattn_view *out, int32_t split_len,
                   void *workspace, size_t workspace_bytes, void *stream) {
  const bool q8 = k_scale != nullptr;
  tsattn::Problem pr;
  int rc = check_problem(p, &pr);
  if (rc) return rc;
  if (pr.drop.on)
    return fail(TSATTN_ERR_UNSUPPORTED, "the decode kernel does not drop (inference only)");
  if ((rc = check_view(q, "query")) || (rc = check_view(k, "key")) ||
      (rc = check_view(v, "value")) || (rc = check_view(out, "output")))
    return rc;
  if (q8 && ((rc = check_view(k_scale, "key scale")) || (rc = check_view(v_scale, "value scale"))))
    return rc;
  if (split_len < 0) return fail(TSATTN_ERR_INVALID, "split_len must be >= 0");
  if (rope && (rc = check_rope(rope, pr, &pr.rope))) return rc;
  const tsattn::View vq = tsattn::make_view(q), vk = tsattn::make_view(k), vv = tsattn::make_view(v);
  if (q8) {
    if (p->mask_kind != TSATTN_MASK_NONE && !p->kv_len)
      return fail(TSATTN_ERR_UNSUPPORTED, "int8 decode takes key-padding lengths, not general masks");
    // int8 rows are read as 8-byte chunks: 8-byte aligned bases and row strides
    auto aligned8 = [](const tsattn::View &x) {
      return reinterpret_cast<uintptr_t>(x.data) % 8 == 0 && x.s0 % 8 == 0 && x.s1 % 8 == 0 &&
             x.s2 % 8 == 0;
    };
    if (p->dtype == TSATTN_F32 || !tsattn::decode_supported(pr, p->dtype) || !tsattn::aligned16(vq) ||
        !aligned8(vk) || !aligned8(vv))
      return fail(TSATTN_ERR_UNSUPPORTED,
                  "int8 decode needs <= 8 query rows per KV head, f16/bf16 queries, equal head "
                  "dims in {64,128,256} and 8-byte aligned cache rows");
  } else if (!tsattn::decode_supported(pr, p->dtype) || !tsattn::aligned16(vq) ||
             !tsattn::aligned16(vk) || !tsattn::aligned16(vv)) {
    return fail(TSATTN_ERR_UNSUPPORTED,
                "decode kernel needs <= 8 query rows per KV head, f16/bf16/f32 (f32: no folded "
                "rotation), equal head dims in "
                "{64,128,256} and 16-byte aligned rows");
  }
  const size_t need = tsattn::decode_workspace_bytes(pr, split_len);
  if (need && (!workspace || workspace_bytes < need))
    return fail(TSATTN_ERR_INVALID, "decode workspace too small: %zu < %zu bytes",
                workspace_bytes, need);
  g_last_path = 3;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (q8)
    return hip_status(tsattn::launch_decode_int8(pr, p->dtype, vq, vk, vv,
                                                 tsattn::make_view(k_scale),
                                                 tsattn::make_view(v_scale),
                                                 tsattn::make_view(out), split_len, workspace, st),
                      "int8 decode launch");
  return hip_status(tsattn::launch_decode(pr, p->dtype, vq, vk, vv, tsattn::make_view(out),
                                          split_len, workspace, st),
                    "decode launch");
}

}  // namespace

extern "C" {

int tsattn_abi_version(void) { return TSATTN_ABI_VERSION; }

const char *tsattn_last_error(void) { return g_error; }

int tsattn_set_kernel_policy(int policy) {
  if (policy < 0 || policy > 1) return fail(TSATTN_ERR_INVALID, "unknown kernel policy %d", policy);
  g_policy.store(policy);
  return TSATTN_OK;
}

int tsattn_last_kernel_path(void) { return g_last_path; }

int tsattn_sdpa_forward(const tsattn_problem *p, const tsattn_view *q, const tsattn_view *k,
                        const tsattn_view *v, const tsattn_view *out, void *lse, void *stream) {
  return sdpa_forward(p, nullptr, q, k, v, out, lse, stream);
}

int tsattn_sdpa_forward_rope(const tsattn_problem *p, const tsattn_rope_desc *rope,
                             const tsattn_view *q, const tsattn_view *k, const tsattn_view *v,
                             const tsattn_view *out, void *lse, void *stream) {
  if (!rope) return fail(TSATTN_ERR_INVALID, "RoPE descriptor is NULL");
  return sdpa_forward(p, rope, q, k, v, out, lse, stream);
}

size_t tsattn_sdpa_backward_workspace(const tsattn_problem *p) { return backward_workspace(p); }

size_t tsattn_sdpa_backward_rope_workspace(const tsattn_problem *p) {
  tsattn::Problem pr;
  if (check_problem(p, &pr)) return 0;
  return rope_backward_workspace(pr, p->dtype);
}

int tsattn_sdpa_backward(const tsattn_problem *p, const tsattn_view *q, const tsattn_view *k,
                         const tsattn_view *v, const tsattn_view *out, const tsattn_view *dout,
                         const void *lse, const tsattn_view *dq, const tsattn_view *dk,
                         const tsattn_view *dv, void *workspace, size_t workspace_bytes,
                         void *stream) {
  return sdpa_backward(p, nullptr, q, k, v, out, dout, lse, dq, dk, dv, workspace,
                       workspace_bytes, stream);
}

int tsattn_sdpa_backward_rope(const tsattn_problem *p, const tsattn_rope_desc *rope,
                              const tsattn_view *q, const tsattn_view *k, const tsattn_view *v,
                              const tsattn_view *out, const tsattn_view *dout, const void *lse,
                              const tsattn_view *dq, const tsattn_view *dk, const tsattn_view *dv,
                              void *workspace, size_t workspace_bytes, void *stream) {
  if (!rope) return fail(TSATTN_ERR_INVALID, "RoPE descriptor is NULL");
  return sdpa_backward(p, rope, q, k, v, out, dout, lse, dq, dk, dv, workspace, workspace_bytes,
                       stream);
}

size_t tsattn_dropout_bits_bytes(const tsattn_problem *p) {
  tsattn::Problem pr;
  if (check_problem(p, &pr)) return 0;
  return tsattn::dropout_bits_bytes(pr);
}

int tsattn_dropout_keep(const tsattn_problem *p, uint8_t *out, void *stream) {
  tsattn::Problem pr;
  int rc = check_problem(p, &pr);
  if (rc) return rc;
  if (!out) return fail(TSATTN_ERR_INVALID, "output pointer is NULL");
  return hip_status(tsattn::launch_dropout_keep(pr, out, static_cast<hipStream_t>(stream)),
                    "dropout keep launch");
}

size_t tsattn_decode_workspace(const tsattn_problem *p, int32_t split_len) {
  tsattn::Problem pr;
  if (check_problem(p, &pr)) return 0;
  return tsattn::decode_workspace_bytes(pr, split_len);
}

int tsattn_decode_forward(const tsattn_problem *p, const tsattn_view *q, const tsattn_view *k,
                          const tsattn_view *v, const tsattn_view *out, int32_t split_len,
                          void *workspace, size_t workspace_bytes, void *stream) {
  return decode_forward(p, nullptr, q, k, v, nullptr, nullptr, out, split_len, workspace,
                        workspace_bytes, stream);
}

int tsattn_decode_forward_noalloc(const tsattn_problem *p, const tsattn_view *q,
                                  const tsattn_view *k, const tsattn_view *v,
                                  const tsattn_view *out, int32_t split_len, void *stream) {
  tsattn::Problem pr;
  int rc = check_problem(p, &pr);
  if (rc) return rc;
  if (split_len < 0) return fail(TSATTN_ERR_INVALID, "split_len must be >= 0");
  const size_t need = tsattn::decode_workspace_bytes(pr, split_len);
  if (need > TSATTN_DECODE_SCRATCH_BYTES)
    return fail(TSATTN_ERR_INVALID,
                "decode needs %zu bytes of scratch; the allocation-free entry point holds %zu "
                "(use tsattn_decode_forward with a workspace)",
                need, static_cast<size_t>(TSATTN_DECODE_SCRATCH_BYTES));
  void *ws = nullptr;
  if ((rc = hip_status(tsattn::decode_scratch(&ws), "decode scratch address"))) return rc;
  return decode_forward(p, nullptr, q, k, v, nullptr, nullptr, out, split_len, ws,
                        TSATTN_DECODE_SCRATCH_BYTES, stream);
}

int tsattn_decode_forward_int8(const tsattn_problem *p, const tsattn_view *q, const tsattn_view *k,
                               const tsattn_view *v, const tsattn_view *k_scale,
                               const tsattn_view *v_scale, const tsattn_view *out, int32_t split_len,
                               void *workspace, size_t workspace_bytes, void *stream) {
  if (!k_scale || !v_scale) return fail(TSATTN_ERR_INVALID, "int8 decode needs both row-scale views");
  return decode_forward(p, nullptr, q, k, v, k_scale, v_scale, out, split_len, workspace,
                        workspace_bytes, stream);
}

int tsattn_decode_forward_rope(const tsattn_problem *p, const tsattn_rope_desc *rope,
                               const tsattn_view *q, const tsattn_view *k, const tsattn_view *v,
                               const tsattn_view *k_scale, const tsattn_view *v_scale,
                               const tsattn_view *out, int32_t split_len, void *workspace,
                               size_t workspace_bytes, void *stream) {
  if (!rope) return fail(TSATTN_ERR_INVALID, "RoPE descriptor is NULL");
  if (!k_scale != !v_scale)
    return fail(TSATTN_ERR_INVALID, "pass both row-scale views (int8 cache) or neither");
  return decode_forward(p, rope, q, k, v, k_scale, v_scale, out, split_len, workspace,
                        workspace_bytes, stream);
}

int tsattn_kv_append_int8(int32_t dtype, int32_t batch, int32_t heads, int32_t len, int32_t dim,
                          const tsattn_view *src, const tsattn_view *dst, const tsattn_view *scale,
                          int64_t pos, void *stream) {
  int rc;
  if ((rc = check_view(src, "source rows")) || (rc = check_view(dst, "int8 cache")) ||
      (rc = check_view(scale, "cache scales")))
    return rc;
  if (dtype != TSATTN_F32 && dtype != TSATTN_F16 && dtype != TSATTN_BF16)
    return fail(TSATTN_ERR_INVALID, "cache rows must be f32, f16 or bf16 (got dtype %d)", dtype);
  if (batch <= 0 || heads <= 0 || len <= 0 || dim <= 0 || pos < 0)
    return fail(TSATTN_ERR_INVALID, "append needs positive sizes and a nonnegative position");
  if (dim > 512) return fail(TSATTN_ERR_UNSUPPORTED, "head dims above 512 are not supported");
  return hip_status(tsattn::launch_kv_append_int8(dtype, batch, heads, len, dim,
                                                  tsattn::make_view(src), tsattn::make_view(dst),
                                                  tsattn::make_view(scale), pos,
                                                  static_cast<hipStream_t>(stream)),
                    "int8 append launch");
}

int tsattn_rope(int32_t dtype, int32_t batch, int32_t heads, int32_t len, int32_t dim,
                int32_t rotary_dim, const tsattn_view *x, const tsattn_view *out, const void *cos,
                const void *sin, int64_t pos0, int32_t inverse, void *stream) {
  int rc;
  if ((rc = check_view(x, "input")) || (rc = check_view(out, "output"))) return rc;
  if (dtype != TSATTN_F32 && dtype != TSATTN_F16 && dtype != TSATTN_BF16)
    return fail(TSATTN_ERR_INVALID, "RoPE rows must be f32, f16 or bf16 (got dtype %d)", dtype);
  if (batch <= 0 || heads <= 0 || len <= 0 || dim <= 0 || pos0 < 0)
    return fail(TSATTN_ERR_INVALID, "RoPE needs positive sizes and a nonnegative position");
  if (rotary_dim <= 0 || rotary_dim % 2 || rotary_dim > dim || dim % 2)
    return fail(TSATTN_ERR_INVALID, "RoPE requires a positive even rotary dimension and valid positions/base");
  if (!cos || !sin) return fail(TSATTN_ERR_INVALID, "RoPE needs cos / sin tables");
  return hip_status(tsattn::launch_rope(dtype, batch, heads, len, dim, rotary_dim,
                                        tsattn::make_view(x), tsattn::make_view(out), cos, sin,
                                        pos0, inverse, static_cast<hipStream_t>(stream)),
                    "RoPE launch");
}

int tsattn_rope_append(int32_t dtype, int32_t batch, int32_t heads, int32_t len, int32_t dim,
                       int32_t rotary_dim, const tsattn_view *k, const tsattn_view *v,
                       const tsattn_view *k_cache, const tsattn_view *v_cache,
                       const tsattn_view *k_scale, const tsattn_view *v_scale, const void *cos,
                       const void *sin, int64_t pos, void *stream) {
  int rc;
  if ((rc = check_view(k, "key rows")) || (rc = check_view(v, "value rows")) ||
      (rc = check_view(k_cache, "key cache")) || (rc = check_view(v_cache, "value cache")))
    return rc;
  if (!k_scale != !v_scale)
    return fail(TSATTN_ERR_INVALID, "an int8 cache needs both key and value scales");
  if ((k_scale && (rc = check_view(k_scale, "key scales"))) ||
      (v_scale && (rc = check_view(v_scale, "value scales"))))
    return rc;
  if (dtype != TSATTN_F32 && dtype != TSATTN_F16 && dtype != TSATTN_BF16)
    return fail(TSATTN_ERR_INVALID, "cache rows must be f32, f16 or bf16 (got dtype %d)", dtype);
  if (batch <= 0 || heads <= 0 || len <= 0 || dim <= 0 || dim % 2 || pos < 0)
    return fail(TSATTN_ERR_INVALID, "append needs positive sizes, an even head dim and a nonnegative position");
  if (dim > 512) return fail(TSATTN_ERR_UNSUPPORTED, "head dims above 512 are not supported");
  if (rotary_dim < 0 || rotary_dim % 2 || rotary_dim > dim || (rotary_dim && (!cos || !sin)))
    return fail(TSATTN_ERR_INVALID, "RoPE requires a positive even rotary dimension and valid positions/base");
  tsattn::View ks, vs;
  if (k_scale) ks = tsattn::make_view(k_scale), vs = tsattn::make_view(v_scale);
  return hip_status(tsattn::launch_rope_append(dtype, batch, heads, len, dim, rotary_dim,
                                               tsattn::make_view(k), tsattn::make_view(v),
                                               tsattn::make_view(k_cache), tsattn::make_view(v_cache),
                                               k_scale ? &ks : nullptr, v_scale ? &vs : nullptr,
                                               cos, sin, pos, static_cast<hipStream_t>(stream)),
                    "RoPE append launch");
}

int tsattn_qkv_rope_append(int32_t dtype, int32_t batch, int32_t len, int32_t embed, int32_t heads_q,
                           int32_t heads_kv, int32_t dim, const tsattn_view *x, const void *wq,
                           const void *wk, const void *wv, const void *bq, const void *bk,
                           const void *bv, const tsattn_view *q_out, const tsattn_view *k_cache,
                           const tsattn_view *v_cache, const tsattn_view *k_scale,
                           const tsattn_view *v_scale, const void *cos, const void *sin, int64_t pos,
                           void *stream) {
  int rc;
  if ((rc = check_view(x, "input rows")) || (rc = check_view(q_out, "query output")) ||
      (rc = check_view(k_cache, "key cache")) ||
      (rc = check_view(v_cache, "value cache")))
    return rc;
  if (!k_scale != !v_scale)
    return fail(TSATTN_ERR_INVALID, "an int8 cache needs both key and value scales");
  if ((k_scale && (rc = check_view(k_scale, "key scales"))) ||
      (v_scale && (rc = check_view(v_scale, "value scales"))))
    return rc;
  if (dtype != TSATTN_F16 && dtype != TSATTN_BF16)
    return fail(TSATTN_ERR_INVALID, "the fused projection takes f16 or bf16 rows (got dtype %d)", dtype);
  if (batch <= 0 || len <= 0 || embed <= 0 || heads_q <= 0 || heads_kv <= 0 || pos < 0)
    return fail(TSATTN_ERR_INVALID, "projection needs positive sizes and a nonnegative position");
  if (heads_q % heads_kv)
    return fail(TSATTN_ERR_INVALID, "query heads must divide into KV groups");
  if (dim != 64 && dim != 128)
    return fail(TSATTN_ERR_UNSUPPORTED, "the fused projection supports head dims 64 and 128");
  if (embed % 16) return fail(TSATTN_ERR_UNSUPPORTED, "the fused projection needs embed % 16 == 0");
  if (!wq || !wk || !wv) return fail(TSATTN_ERR_INVALID, "the weights must be non-NULL");
  if (!cos != !sin) return fail(TSATTN_ERR_INVALID, "RoPE needs both cos and sin tables");
  const tsattn::View vx = tsattn::make_view(x);
  const uintptr_t al = reinterpret_cast<uintptr_t>(vx.data) | reinterpret_cast<uintptr_t>(wq) |
                       reinterpret_cast<uintptr_t>(wk) | reinterpret_cast<uintptr_t>(wv);
  if (al % 16 || vx.s0 % 8 || vx.s2 % 8 || vx.s0 < 0 || vx.s2 < 0)
    return fail(TSATTN_ERR_INVALID, "x rows and the weights must be 16-byte aligned");
  const int64_t xext = (static_cast<int64_t>(batch) - 1) * vx.s0 + (static_cast<int64_t>(len) - 1) * vx.s2 + embed;
  if (xext * 2 >= (int64_t(1) << 31) ||
      static_cast<int64_t>(heads_q > heads_kv ? heads_q : heads_kv) * dim * embed * 2 >= (int64_t(1) << 31))
    return fail(TSATTN_ERR_UNSUPPORTED, "x or a weight matrix exceeds 2^31 bytes");
  const tsattn::View vq = tsattn::make_view(q_out), vk = tsattn::make_view(k_cache),
                     vv = tsattn::make_view(v_cache);
  // 4-element row pieces: 8-byte stores (16-bit) / 4-byte (int8)
  auto al4 = [](const tsattn::View &v, size_t es) {
    return reinterpret_cast<uintptr_t>(v.data) % (4 * es) == 0 && v.s0 % 4 == 0 && v.s1 % 4 == 0 &&
           v.s2 % 4 == 0;
  };
  const size_t ce = k_scale ? 1 : 2;
  if (!al4(vq, 2) || !al4(vk, ce) || !al4(vv, ce))
    return fail(TSATTN_ERR_INVALID, "query output and cache rows need 4-element aligned strides");
  tsattn::View ks, vs;
  if (k_scale) ks = tsattn::make_view(k_scale), vs = tsattn::make_view(v_scale);
  const void *w[3] = {wq, wk, wv}, *bias[3] = {bq, bk, bv};
  return hip_status(tsattn::launch_qkv_rope_append(dtype, batch, len, embed, heads_q, heads_kv, dim, vx, w,
                                                   bias, vq, vk, vv, k_scale ? &ks : nullptr,
                                                   v_scale ? &vs : nullptr, cos, sin, pos,
                                                   static_cast<hipStream_t>(stream)),
                    "fused projection launch");
}

int tsattn_key_mask_lengths(const uint8_t *mask, int64_t stride_b, int64_t stride_k,
                            int32_t batch, int32_t len_kv, int32_t *kv_len, int32_t *kv_prefix,
                            void *stream) {
  if (!mask || !kv_len) return fail(TSATTN_ERR_INVALID, "mask and kv_len must be non-NULL");
  if (batch <= 0 || len_kv <= 0) return fail(TSATTN_ERR_INVALID, "batch and len_kv must be positive");
  return hip_status(tsattn::launch_key_mask_lengths(mask, stride_b, stride_k, batch, len_kv, kv_len,
                                                    kv_prefix, static_cast<hipStream_t>(stream)),
                    "key mask lengths launch");
}

}  // extern "C"
