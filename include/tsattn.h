/*
 * tsattn.h -- C ABI of libtsattn.so, the MI355X (gfx950) attention kernels
 * behind tensorsmith's `scaled_dot_product_attention(..., backend="hip")`.
 *
 * The reference (KavinP21/custom-ml-library, package `tensorsmith`) computes
 * this path in Python/NumPy and has no FFI for it; each entry point below
 * names the reference code it replaces.  Its user-kernel FFI precedent is
 * `cuda.RawKernel` (src/tensorsmith/cuda.py:129-185): contiguous device
 * buffers plus explicitly typed scalars, launched on the caller's stream.
 *
 * Conventions
 *  - Every pointer is a device pointer owned by the caller; the library keeps
 *    no allocation (apart from the static scratch array of
 *    tsattn_decode_forward_noalloc).  Calls are asynchronous on `stream` (a
 *    hipStream_t, or NULL for the default stream).
 *  - Tensors are strided 4-D views [B, H, S, D] with strides in elements; the
 *    innermost (D) stride must be 1.  Broadcast masks use zero strides.
 *  - Every entry returns a tsattn_status; on failure tsattn_last_error()
 *    describes it (thread-local string, valid until the next call on the
 *    same thread).
 *  - Row log-sum-exp (LSE) buffers are contiguous [B, Hq, Sq], natural log,
 *    float (double for TSATTN_F64); fully masked rows hold -inf.
 */
#ifndef TSATTN_H
#define TSATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TSATTN_ABI_VERSION 8

typedef enum {
  TSATTN_OK = 0,
  TSATTN_ERR_INVALID = 1,     /* contract violation (ValueError / TypeError) */
  TSATTN_ERR_UNSUPPORTED = 2, /* valid request these kernels do not implement */
  TSATTN_ERR_HIP = 3          /* HIP runtime error (RuntimeError) */
} tsattn_status;

typedef enum {
  TSATTN_F32 = 0,
  TSATTN_F16 = 1,
  TSATTN_BF16 = 2,
  TSATTN_F64 = 3,
  TSATTN_BOOL = 4, /* masks only: one byte per element, nonzero = allowed */
  TSATTN_I8 = 5    /* quantised KV cache storage */
} tsattn_dtype;

typedef enum {
  TSATTN_MASK_NONE = 0,
  TSATTN_MASK_BOOL = 1,    /* True = allowed (attention.py:105-107) */
  TSATTN_MASK_ADDITIVE = 2 /* added to the scaled scores */
} tsattn_mask_kind;

/* A strided 4-D view [B, H, S, D]; stride[3] must be 1 for operands. */
typedef struct tsattn_view {
  void *data;
  int64_t stride[4];
} tsattn_view;

/*
 * One attention problem: the arguments of scaled_dot_product_attention
 * (src/tensorsmith/nn/attention.py:16-29) after its validation (:36-62).
 * `kv_len` (device, [batch] int32, nullable) limits the keys of row b to
 * [0, kv_len[b]); `kv_prefix` (device, [batch] int32, nullable) marks rows
 * whose boolean key mask is exactly that prefix, letting kernels skip the
 * per-element mask test (both written by tsattn_key_mask_lengths).
 */
typedef struct tsattn_problem {
  int32_t dtype; /* tsattn_dtype of q, k, v, outputs and gradients */
  int32_t batch, heads_q, heads_kv, len_q, len_kv, dim_qk, dim_v;
  double scale;
  int32_t is_causal;
  int64_t causal_offset; /* key j allowed for query i iff i + offset >= j */
  const int32_t *kv_len;
  const int32_t *kv_prefix;
  int32_t mask_kind;  /* tsattn_mask_kind */
  int32_t mask_dtype; /* TSATTN_BOOL, or the additive mask's float type */
  tsattn_view mask;   /* broadcast to [B, Hq, Sq, Sk] */
  /*
   * Attention dropout (src/tensorsmith/nn/attention.py:140-144): probability
   * p in [0, 1) (0 = none) and the counter-based stream it draws from.
   * Element (b, h, i, j) takes 16-bit word L = ((b Hq + h) Sq + i) Sk16 + j
   * (Sk16 = len_kv rounded up to 16) of a Philox4x32-10 stream: words
   * 16 n .. 16 n + 15 are the outputs of the blocks with 128-bit counters
   * (lo32 t, hi32 t, lo32 key[1], hi32 key[1]) for t = 2 (counter + n) and
   * t + 1 (mod 2^64) under the 64-bit key key[0], four 32-bit outputs per
   * block as little-endian uint16 pairs; it is kept iff word >= round(65536 p);
   * kept probabilities scale by float32(1) / float32(1 - p).  The backward
   * uses the same mask: from `dropout_bits`, or regenerated from the same key
   * and counter.
   */
  double dropout_p;
  uint64_t dropout_key[2];
  uint64_t dropout_counter;
  /*
   * Optional device buffer (tsattn_dropout_bits_bytes) of the keep decisions
   * as bits: word ((b Hq + h) ceil(Sk / 32) + t) round_up(Sq, 4) + i, bit j =
   * element (b, h, i, 32 t + j).  A dropping forward fills it; the backward
   * then reads it instead of drawing the stream again (pass the buffer its
   * forward filled, or NULL: the backward then draws the bits into its
   * workspace first).
   */
  uint32_t *dropout_bits;
} tsattn_problem;

/* ABI version of the loaded library (== TSATTN_ABI_VERSION). */
int tsattn_abi_version(void);

/* Human-readable description of the last failure on this thread. */
const char *tsattn_last_error(void);

/*
 * Kernel-family policy for sdpa forward/backward: 0 = automatic (MFMA kernels
 * where they apply, generic kernels otherwise), 1 = generic kernels only.
 * A diagnostic knob with no counterpart in the reference (it has one
 * algorithm per backend name); tests use it to run both families on the
 * same inputs.
 */
int tsattn_set_kernel_policy(int policy);

/* Kernel family of this thread's last launch: 1 generic, 2 MFMA, 3 decode. */
int tsattn_last_kernel_path(void);

/*
 * Kernel timing probes (diagnostic, no counterpart in the reference; the
 * benchmark uses them to time the dominant kernel on its own stream).
 * While enabled, every kernel launch is bracketed by hipEvents recorded on
 * the launch stream.  tsattn_profile_read(i, ...) synchronises on the
 * recorded events and returns the name, launch count and summed duration
 * (ms) of the i-th distinct kernel (returns -1 past the last one);
 * tsattn_profile_reset clears the totals.
 */
int tsattn_profile_enable(int on);
int tsattn_profile_reset(void);
int tsattn_profile_read(int index, char *name, size_t name_len, long long *launches,
                        double *total_ms);

/*
 * Forward: out = softmax(scale * q k^T + mask) v, with the online-softmax
 * recurrence of the reference's streaming backend and its saved row LSE.
 * Replaces src/tensorsmith/nn/attention.py:175-198 (streaming forward) and,
 * for the same math, :132-145 (dense forward without dropout).
 * `lse` may be NULL (inference, like the `native` early return at :172-173).
 */
int tsattn_sdpa_forward(const tsattn_problem *p, const tsattn_view *q, const tsattn_view *k,
                        const tsattn_view *v, const tsattn_view *out, void *lse, void *stream);

/* Bytes of scratch tsattn_sdpa_backward needs: row deltas and row LSEs (fp32,
 * 2 per query row), the keep bits when dropping without
 * p->dropout_bits, and on the MFMA kernels with a head dim of 128 (q/k or v)
 * room for dS stored once (2 KiB per 32 x 32 tile the causal structure
 * visits); at head dims 64 and 32 the recomputing backward is the faster one
 * and the query sizes no dS. */
size_t tsattn_sdpa_backward_workspace(const tsattn_problem *p);

/*
 * Backward: dq, dk, dv from the saved LSE, recomputing P = exp(S - LSE)
 * blockwise, with delta = rowsum(dout * out).  Replaces
 * src/tensorsmith/nn/attention.py:200-248 (incl. the GQA group sums at
 * :245-247).  Deterministic: no atomics, every element is written once.
 * With the queried workspace the MFMA path stores dS from the dK/dV kernel
 * and forms dQ as one GEMM over it (head dim 128); a smaller workspace that
 * still holds the row values (and keep bits), or head dims 64 and 32, make
 * the dQ kernel recompute S and dP instead.
 */
int tsattn_sdpa_backward(const tsattn_problem *p, const tsattn_view *q, const tsattn_view *k,
                         const tsattn_view *v, const tsattn_view *out, const tsattn_view *dout,
                         const void *lse, const tsattn_view *dq, const tsattn_view *dk,
                         const tsattn_view *dv, void *workspace, size_t workspace_bytes,
                         void *stream);

/*
 * RoPE folded into the attention kernels.  cos / sin: device tables
 * [L, rotary_dim / 2] in the tensor dtype whose row p holds the angles of
 * position p, built as the reference builds its per-call table
 * (src/tensorsmith/nn/attention.py:269-279: float32 angles
 * p * base^(-2i / rotary_dim), NumPy cos / sin, cast to the dtype); query
 * row i sits at position q_pos0 + i, key row j at k_pos0 + j, and the tables
 * must hold those rows.
 */
typedef struct tsattn_rope_desc {
  const void *cos;
  const void *sin;
  int32_t rotary_dim; /* even, 0 < rotary_dim <= dim_qk; later channels pass through */
  int64_t q_pos0;
  int64_t k_pos0;
  /* Optional (NULL: unused), 16-byte aligned [B, Hq, Sq, dim_qk] contiguous
   * rows.  tsattn_sdpa_forward_rope writes the rotated queries there (bits
   * of tsattn_rope on q); tsattn_sdpa_backward_rope given the same buffer
   * reads them instead of rotating and staging the queries itself.  The
   * decode entry points ignore it. */
  void *q_rotated;
} tsattn_rope_desc;

/*
 * rotary_embedding(q, q_pos0) then scaled_dot_product_attention, the step
 * MultiHeadAttention takes (src/tensorsmith/nn/transformer.py:138-149), with
 * the query rotation done in the kernel prologue: `q` holds the unrotated
 * queries, `k` the keys already rotated (tsattn_rope).  Bit-identical to
 * tsattn_rope on q followed by tsattn_sdpa_forward.  Only problems the MFMA
 * kernels take (f16/bf16, dim_qk and dim_v in {64, 128}, 16-byte aligned
 * views); others return TSATTN_ERR_UNSUPPORTED (rotate with tsattn_rope).
 */
int tsattn_sdpa_forward_rope(const tsattn_problem *p, const tsattn_rope_desc *rope,
                             const tsattn_view *q, const tsattn_view *k, const tsattn_view *v,
                             const tsattn_view *out, void *lse, void *stream);

/* Bytes of scratch tsattn_sdpa_backward_rope needs: the row values of
 * tsattn_sdpa_backward plus the rotated query rows the dK/dV kernel reads. */
size_t tsattn_sdpa_backward_rope_workspace(const tsattn_problem *p);

/*
 * Its VJP, with rotary_embedding's VJP (attention.py:289-294) folded in:
 * `q` unrotated, `k` rotated, as in the forward; dq and dk are the gradients
 * of the unrotated queries and keys -- the dQ and dK epilogues round the
 * gradients to the tensor dtype and rotate them back (positions q_pos0 + i,
 * k_pos0 + j), bit-identical to tsattn_sdpa_backward followed by an inverse
 * tsattn_rope on dq and dk.  Workspace: tsattn_sdpa_backward_rope_workspace.
 */
int tsattn_sdpa_backward_rope(const tsattn_problem *p, const tsattn_rope_desc *rope,
                              const tsattn_view *q, const tsattn_view *k, const tsattn_view *v,
                              const tsattn_view *out, const tsattn_view *dout, const void *lse,
                              const tsattn_view *dq, const tsattn_view *dk, const tsattn_view *dv,
                              void *workspace, size_t workspace_bytes, void *stream);

/*
 * The keep mask the attention kernels draw for problem `p` (its dropout
 * fields and sizes): out[b, h, i, j] = 1 if kept, else 0, as a contiguous
 * [B, Hq, Sq, Sk] uint8 array.  The reference's dense backend holds this mask
 * explicitly (attention.py:141-143); this materialises the one the hip
 * kernels regenerate, for inspection and tests.
 */
int tsattn_dropout_keep(const tsattn_problem *p, uint8_t *out, void *stream);

/* Bytes of tsattn_problem.dropout_bits for this problem (B Hq ceil(Sk / 32)
 * round_up(Sq, 4) 32-bit words); no counterpart in the reference, whose
 * dense backend keeps its mask as an array (attention.py:141-143). */
size_t tsattn_dropout_bits_bytes(const tsattn_problem *p);

/* Bytes of scratch tsattn_decode_forward needs for `split_len` keys per split. */
size_t tsattn_decode_workspace(const tsattn_problem *p, int32_t split_len);

/*
 * KV-cache decode: few query rows (len_q * heads_q / heads_kv <= 8 per KV
 * head) against a long cached prefix, split across the cache in chunks of
 * `split_len` keys (0 = choose: 640, halved while the grid is small; an
 * explicit power of two makes concurrent splits share HBM channels and
 * runs ~20% slower), partial (max, sum, acc) merged as in the
 * reference's online softmax (attention.py:185-193).  Replaces the dense
 * path the reference takes for cached decode (MultiHeadAttention.forward,
 * src/tensorsmith/nn/transformer.py:142-154 -> attention.py:132-145).
 * k/v are the cache views [B, Hkv, capacity, D] with len_kv active keys;
 * dtype f16, bf16 or f32 (f32 caches: 32-byte row pieces, every product and
 * sum in fp32), head dims 64 / 128 / 256, 16-byte aligned rows.
 */
int tsattn_decode_forward(const tsattn_problem *p, const tsattn_view *q, const tsattn_view *k,
                          const tsattn_view *v, const tsattn_view *out, int32_t split_len,
                          void *workspace, size_t workspace_bytes, void *stream);

/*
 * Size of the library-owned scratch of tsattn_decode_forward_noalloc: one
 * static device array per GPU, held from the first call on that GPU until the
 * process ends.
 */
#define TSATTN_DECODE_SCRATCH_BYTES (32u << 20)

/*
 * tsattn_decode_forward without a workspace argument and without allocating:
 * the split partials live in the library's static device array of
 * TSATTN_DECODE_SCRATCH_BYTES (32 MiB) on the current GPU.  No counterpart in
 * the reference; it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same inputs, outputs and results as tsattn_decode_forward
 * (bit-identical); problems whose tsattn_decode_workspace exceeds the array
 * return TSATTN_ERR_INVALID.  The first call on a GPU looks up the array's
 * device address (hipGetSymbolAddress).  Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (e.g. on two streams) race --
 * serialise them.
 */
int tsattn_decode_forward_noalloc(const tsattn_problem *p, const tsattn_view *q,
                                  const tsattn_view *k, const tsattn_view *v,
                                  const tsattn_view *out, int32_t split_len, void *stream);

/*
 * KV-cache decode over an int8 cache: k / v are int8 views [B, Hkv, capacity,
 * D] with fp32 row scales k_scale / v_scale [B, Hkv, capacity, 1] -- the
 * reference's quantised KVCache format (src/tensorsmith/nn/cache.py:48-52,
 * :73-77).  The rows are dequantised inside the kernel (x = q * scale), where
 * the reference dequantises the whole prefix eagerly in KVCache.get
 * (cache.py:88-99) before the dense attention.  q / out are f16 or bf16
 * (p->dtype); everything else is as tsattn_decode_forward, whose workspace
 * size query applies unchanged.  A mask is accepted only as key-padding
 * lengths (p->kv_len).
 */
int tsattn_decode_forward_int8(const tsattn_problem *p, const tsattn_view *q, const tsattn_view *k,
                               const tsattn_view *v, const tsattn_view *k_scale,
                               const tsattn_view *v_scale, const tsattn_view *out, int32_t split_len,
                               void *workspace, size_t workspace_bytes, void *stream);

/*
 * KV-cache decode with RoPE folded into the query load: q is the unrotated
 * query (row i at position rope->q_pos0 + i); the cache holds keys rotated
 * when they were appended (tsattn_rope_append), so rope->k_pos0 is not used.
 * Bit-identical to tsattn_rope on q followed by tsattn_decode_forward (or
 * tsattn_decode_forward_int8 when k_scale / v_scale are given: pass both or
 * neither).  Replaces the query half of MultiHeadAttention's rotary step on
 * the cached path (src/tensorsmith/nn/transformer.py:139-141, rotary at
 * src/tensorsmith/nn/attention.py:255-294) ahead of the decode attention.
 * Same table and rotary-dim rules as tsattn_sdpa_forward_rope.
 */
int tsattn_decode_forward_rope(const tsattn_problem *p, const tsattn_rope_desc *rope,
                               const tsattn_view *q, const tsattn_view *k, const tsattn_view *v,
                               const tsattn_view *k_scale, const tsattn_view *v_scale,
                               const tsattn_view *out, int32_t split_len, void *workspace,
                               size_t workspace_bytes, void *stream);

/*
 * KV-cache append into the int8 format (KVCache.append with quantized=True,
 * src/tensorsmith/nn/cache.py:54-86, quantiser at :73-77): every row
 * x = src[b, h, t, 0:dim] (dtype f32 / f16 / bf16, already the cache dtype)
 * is stored as round_half_even(x / s) in dst[b, h, pos + t, :] (int8) with
 * s = max(max|x| / 127, 1e-8) in scale[b, h, pos + t, 0] (fp32), in one
 * pass.  Bit-identical to the reference's NumPy arithmetic.
 */
int tsattn_kv_append_int8(int32_t dtype, int32_t batch, int32_t heads, int32_t len, int32_t dim,
                          const tsattn_view *src, const tsattn_view *dst, const tsattn_view *scale,
                          int64_t pos, void *stream);

/*
 * Interleaved-pair rotary position embedding (rotary_embedding, src/
 * tensorsmith/nn/attention.py:255-296) of x [batch, heads, len, dim] into out
 * (which may be x): channel pair (2i, 2i+1) of row t, i < rotary_dim / 2,
 * rotates by the angle whose cosine / sine are cos[pos0 + t][i] /
 * sin[pos0 + t][i] -- tables of rotary_dim / 2 columns in the tensor dtype,
 * built as the reference builds them (fp32 angles, cast to the dtype).  Each
 * product and sum rounds to the dtype as the reference's array arithmetic
 * does, so results are bit-identical.  inverse != 0 rotates by -angle (the
 * VJP, :289-294).  Channels from rotary_dim on pass through.
 */
int tsattn_rope(int32_t dtype, int32_t batch, int32_t heads, int32_t len, int32_t dim,
                int32_t rotary_dim, const tsattn_view *x, const tsattn_view *out, const void *cos,
                const void *sin, int64_t pos0, int32_t inverse, void *stream);

/*
 * The cached-decode step before attention in one pass: RoPE of the new key
 * rows k (as tsattn_rope, table rows pos .. pos + len - 1; rotary_dim = 0
 * skips it) and the append of k and v at position pos of the caches
 * (MultiHeadAttention.forward, src/tensorsmith/nn/transformer.py:139-143 ->
 * KVCache.append, cache.py:54-86).  k_scale / v_scale NULL: caches in the
 * row dtype; non-NULL: int8 caches with fp32 row scales, quantised exactly as
 * tsattn_kv_append_int8 does.
 */
int tsattn_rope_append(int32_t dtype, int32_t batch, int32_t heads, int32_t len, int32_t dim,
                       int32_t rotary_dim, const tsattn_view *k, const tsattn_view *v,
                       const tsattn_view *k_cache, const tsattn_view *v_cache,
                       const tsattn_view *k_scale, const tsattn_view *v_scale, const void *cos,
                       const void *sin, int64_t pos, void *stream);

/*
 * The cached MultiHeadAttention step before the attention in one kernel:
 * the three input projections (MultiHeadAttention.forward, src/tensorsmith/
 * nn/transformer.py:124-138: q = x Wq^T (+ bq), k = x Wk^T (+ bk),
 * v = x Wv^T (+ bv)), RoPE of q and k at positions pos .. pos + len - 1
 * (:139-141, as tsattn_rope with rotary_dim = dim; cos == NULL skips it) and
 * the append of k and v at position pos of the caches (:142, KVCache.append,
 * cache.py:54-86; k_scale / v_scale non-NULL: int8 caches with fp32 row
 * scales, quantised as tsattn_kv_append_int8).  x: the [batch, len, embed]
 * input as a [batch, 1, len, embed] view (stride[1] unused), rows and row
 * strides 16-byte aligned; wq: [heads_q * dim, embed], wk / wv:
 * [heads_kv * dim, embed], row-major (Linear.weight), 16-byte aligned;
 * bq / bk / bv: NULL or [rows of the matching weight]; q_out: [batch,
 * heads_q, len, dim] (the rotated queries); caches [batch, heads_kv,
 * capacity >= pos + len, dim]; cos / sin as tsattn_rope's tables.  dtype f16
 * or bf16, dim 64 or 128, embed a multiple of 16.  The projections
 * accumulate in fp32 and round to the dtype, then add the bias (when given)
 * in the dtype with one more rounding, as the reference's Linear (matmul,
 * then + bias); the rotation and the int8 rounding are then bit-identical to
 * the reference's on those rows.
 */
int tsattn_qkv_rope_append(int32_t dtype, int32_t batch, int32_t len, int32_t embed, int32_t heads_q,
                           int32_t heads_kv, int32_t dim, const tsattn_view *x, const void *wq,
                           const void *wk, const void *wv, const void *bq, const void *bk,
                           const void *bv, const tsattn_view *q_out, const tsattn_view *k_cache,
                           const tsattn_view *v_cache, const tsattn_view *k_scale,
                           const tsattn_view *v_scale, const void *cos, const void *sin, int64_t pos,
                           void *stream);

/*
 * Boolean key mask [B, K] (strides in bytes-as-elements) -> kv_len[b] = 1 +
 * last allowed key (0 if none) and kv_prefix[b] = 1 iff the allowed keys are
 * exactly [0, kv_len[b]).  Serves the reference's key-padding masks
 * (docs/transformers.md:55, shape [B,1,1,K]).
 */
int tsattn_key_mask_lengths(const uint8_t *mask, int64_t stride_b, int64_t stride_k,
                            int32_t batch, int32_t len_kv, int32_t *kv_len, int32_t *kv_prefix,
                            void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TSATTN_H */
