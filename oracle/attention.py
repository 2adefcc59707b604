"""NumPy restatement of tensorsmith's attention algorithm -- TEST INFRASTRUCTURE.

Follows ``src/tensorsmith/nn/attention.py`` of the reference line for line in
*semantics* (written independently; see the citations on each function):

* validation and dispatch                ``attention.py:36-100``
* block scores with masks / causal       ``attention.py:102-113``
* dense forward                          ``attention.py:132-145``
* streaming (online-softmax) forward     ``attention.py:175-198``
* dense and streaming VJP                ``attention.py:200-248``
* GQA expansion and group reduction      ``attention.py:93-100,245-247``

Half inputs are carried as float32 arrays holding exactly-representable
values (see ``oracle.halfprec``).  Dropout (dense backend, ``:140-144``) is
restated in ``oracle.dropout`` with the hip kernels' counter-based mask.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from .halfprec import compute_dtype, round_to

NEG_INF = -np.inf


def _as_compute(x, dtype: str):
    return np.asarray(x, dtype=compute_dtype(dtype))


def expand_gqa(x, heads_q: int):
    """Repeat each KV head ``heads_q // heads_kv`` times, consecutively.

    Query head ``hq`` reads KV head ``hq // rep`` (``attention.py:93-100``).
    """
    b, hkv, s, d = x.shape
    rep = heads_q // hkv
    if rep == 1:
        return x
    return np.broadcast_to(x[:, :, None], (b, hkv, rep, s, d)).reshape(b, hkv * rep, s, d)


def reduce_gqa(g, heads_kv: int):
    """Sum gradients of the repeated heads back into their KV group (``:245-247``)."""
    b, hq, s, d = g.shape
    rep = hq // heads_kv
    if rep == 1:
        return g
    return g.reshape(b, heads_kv, rep, s, d).sum(axis=2)


@dataclass
class Problem:
    """Everything the score function needs besides the operands."""

    scale: float
    is_causal: bool = False
    causal_offset: int = 0
    mask: np.ndarray | None = None  # broadcast to [B,H,Q,K]
    boolean_mask: bool = False

    def scores(self, qb, kb, qi: int, ki: int):
        """Scaled block scores with masks applied (``attention.py:102-113``).

        Boolean masks keep True entries; float masks are added after scaling;
        causal allows key ``j`` for query ``i`` iff ``i + causal_offset >= j``.
        """
        s = np.matmul(qb, np.swapaxes(kb, -1, -2)) * qb.dtype.type(self.scale)
        nq, nk = qb.shape[2], kb.shape[2]
        if self.mask is not None:
            part = self.mask[:, :, qi : qi + nq, ki : ki + nk]
            if self.boolean_mask:
                s = np.where(part, s, NEG_INF)
            else:
                s = s + part.astype(s.dtype)
        if self.is_causal:
            rows = np.arange(qi, qi + nq)[:, None] + self.causal_offset
            cols = np.arange(ki, ki + nk)[None, :]
            s = np.where(rows >= cols, s, NEG_INF)
        return s.astype(qb.dtype, copy=False)


def _finite_or_zero(x):
    return np.where(np.isfinite(x), x, 0).astype(x.dtype, copy=False)


def dense_forward(q, k, v, prob: Problem):
    """Whole-matrix softmax; returns (out, probabilities) (``attention.py:132-145``)."""
    s = prob.scores(q, k, 0, 0)
    m = _finite_or_zero(np.max(s, axis=-1, keepdims=True))
    e = np.exp(s - m)
    total = np.sum(e, axis=-1, keepdims=True)
    p = e / np.where(total > 0, total, 1).astype(e.dtype)
    return np.matmul(p, v), p


def streaming_forward(q, k, v, prob: Problem, block_size: int):
    """Online softmax over key blocks; returns (out, lse[...,1]) (``:175-198``).

    Per query block keeps running max ``m``, denominator ``l`` and weighted
    accumulator; each key block rescales the old state by ``exp(m - m')``.
    Fully masked rows end with ``l == 0``: output 0 and LSE ``-inf``.
    """
    ct = q.dtype
    qlen, klen = q.shape[2], k.shape[2]
    out_blocks, lse_blocks = [], []
    for qi in range(0, qlen, block_size):
        qb = q[:, :, qi : qi + block_size]
        rows = qb.shape[:3] + (1,)
        m = np.full(rows, NEG_INF, dtype=ct)
        l = np.zeros(rows, dtype=ct)
        acc = np.zeros(qb.shape[:3] + (v.shape[-1],), dtype=ct)
        for ki in range(0, klen, block_size):
            s = prob.scores(qb, k[:, :, ki : ki + block_size], qi, ki)
            m_new = np.maximum(m, np.max(s, axis=-1, keepdims=True))
            base = _finite_or_zero(m_new)
            corr = np.exp(m - base)
            p = np.exp(s - base)
            acc = acc * corr + np.matmul(p, v[:, :, ki : ki + block_size])
            l = l * corr + np.sum(p, axis=-1, keepdims=True)
            m = m_new
        safe_l = np.where(l > 0, l, 1).astype(ct)
        out_blocks.append(acc / safe_l)
        lse_blocks.append(np.where(l > 0, m + np.log(safe_l), NEG_INF).astype(ct))
    return np.concatenate(out_blocks, axis=2), np.concatenate(lse_blocks, axis=2)


def dense_backward(q, k, v, p, g, scale: float):
    """Closed-form VJP from saved probabilities (``attention.py:211-219``)."""
    dv = np.matmul(np.swapaxes(p, -1, -2), g)
    dp = np.matmul(g, np.swapaxes(v, -1, -2))
    ds = p * (dp - np.sum(dp * p, axis=-1, keepdims=True)) * p.dtype.type(scale)
    return np.matmul(ds, k), np.matmul(np.swapaxes(ds, -1, -2), q), dv


def streaming_backward(q, k, v, out, lse, g, prob: Problem, block_size: int):
    """Blockwise VJP recomputing P = exp(S - LSE) (``attention.py:220-244``).

    ``delta = rowsum(dO * O)`` uses the compute-dtype output ``out``
    (``:232``); rows with LSE ``-inf`` use 0 so their P is exactly 0 (``:231``).
    """
    ct = q.dtype
    qlen, klen = q.shape[2], k.shape[2]
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    dq_blocks = []
    for qi in range(0, qlen, block_size):
        qb = q[:, :, qi : qi + block_size]
        gb = g[:, :, qi : qi + block_size]
        lb = _finite_or_zero(lse[:, :, qi : qi + block_size])
        delta = np.sum(gb * out[:, :, qi : qi + block_size], axis=-1, keepdims=True)
        dqb = np.zeros_like(qb)
        for ki in range(0, klen, block_size):
            kb = k[:, :, ki : ki + block_size]
            vb = v[:, :, ki : ki + block_size]
            p = np.exp(prob.scores(qb, kb, qi, ki) - lb)
            ds = p * (np.matmul(gb, np.swapaxes(vb, -1, -2)) - delta) * ct.type(prob.scale)
            dqb = dqb + np.matmul(ds, kb)
            dk[:, :, ki : ki + kb.shape[2]] += np.matmul(np.swapaxes(ds, -1, -2), qb)
            dv[:, :, ki : ki + kb.shape[2]] += np.matmul(np.swapaxes(p, -1, -2), gb)
        dq_blocks.append(dqb)
    return np.concatenate(dq_blocks, axis=2), dk, dv


@dataclass
class SdpaResult:
    """Forward result plus the state the VJP needs.

    ``out`` is in the compute dtype (what the reference's VJP closes over);
    ``out_cast`` is rounded to the input dtype (what the reference returns,
    ``attention.py:250-251``).  ``lse`` is ``[B,H,Q,1]`` for ``streaming``.
    """

    dtype: str
    backend: str
    out: np.ndarray
    out_cast: np.ndarray
    lse: np.ndarray | None
    _state: dict = field(default_factory=dict, repr=False)

    def backward(self, upstream):
        """Return (dq, dk, dv) rounded to the input dtype (``attention.py:248``)."""
        raw = self.backward_compute(upstream)
        return tuple(round_to(x, self.dtype) for x in raw)

    def backward_compute(self, upstream):
        """(dq, dk, dv) in the compute dtype, before the final cast."""
        st = self._state
        g = _as_compute(upstream, self.dtype)
        q, k, v, prob = st["q"], st["k"], st["v"], st["prob"]
        if self.backend == "dense":
            dq, dk, dv = dense_backward(q, k, v, st["p"], g, prob.scale)
        else:
            dq, dk, dv = streaming_backward(q, k, v, self.out, self.lse, g, prob, st["block"])
        hkv = st["heads_kv"]
        return dq, reduce_gqa(dk, hkv), reduce_gqa(dv, hkv)


def sdpa(
    query,
    key,
    value,
    attn_mask=None,
    is_causal: bool = False,
    *,
    dtype: str,
    scale: float | None = None,
    causal_offset: int = 0,
    backend: str = "streaming",
    block_size: int = 64,
    enable_gqa: bool = False,
) -> SdpaResult:
    """Oracle counterpart of ``scaled_dot_product_attention`` (``attention.py:16-252``).

    ``query/key/value`` hold values already representable in ``dtype``.
    ``backend`` is ``"dense"`` or ``"streaming"`` (``"auto"`` follows the
    reference heuristic ``Q*K > 1024**2 -> streaming``, ``attention.py:82``).
    """
    if query.ndim != 4 or key.ndim != 4 or value.ndim != 4:
        raise ValueError("attention expects [batch, heads, sequence, channels]")
    b, hq, qlen, dim = query.shape
    hkv, klen = key.shape[1], key.shape[2]
    if hq != hkv and (not enable_gqa or hq % hkv):
        raise ValueError("grouped-query attention requires enable_gqa and divisible heads")
    mult = 1 / math.sqrt(dim) if scale is None else scale
    if backend == "auto":
        backend = "streaming" if qlen * klen > 1024 * 1024 else "dense"
    if backend not in ("dense", "streaming"):
        raise ValueError("oracle backends are dense and streaming")
    q = _as_compute(query, dtype)
    k = expand_gqa(_as_compute(key, dtype), hq)
    v = expand_gqa(_as_compute(value, dtype), hq)
    mask, boolean = None, False
    if attn_mask is not None:
        boolean = attn_mask.dtype == np.bool_
        mask = np.broadcast_to(attn_mask, (b, hq, qlen, klen))
    prob = Problem(mult, bool(is_causal), int(causal_offset), mask, boolean)
    state = {"q": q, "k": k, "v": v, "prob": prob, "block": block_size, "heads_kv": hkv}
    if backend == "dense":
        out, p = dense_forward(q, k, v, prob)
        state["p"] = p
        lse = None
    else:
        out, lse = streaming_forward(q, k, v, prob, block_size)
    return SdpaResult(dtype, backend, out, round_to(out, dtype), lse, state)


# ---------------------------------------------------------------------------
# Independent float64 brute force (no blocking, explicit masks) used to pin
# the restatement above on tiny shapes.
# ---------------------------------------------------------------------------


def allowed_matrix(b, h, qlen, klen, attn_mask=None, is_causal=False, causal_offset=0):
    """Boolean [B,H,Q,K]: True where the reference's score survives.

    Float masks disallow only ``-inf`` entries.
    """
    allowed = np.ones((b, h, qlen, klen), dtype=bool)
    if attn_mask is not None:
        m = np.broadcast_to(attn_mask, (b, h, qlen, klen))
        allowed &= m if m.dtype == np.bool_ else np.isfinite(m)
    if is_causal:
        allowed &= (np.arange(qlen)[:, None] + causal_offset) >= np.arange(klen)[None, :]
    return allowed


def brute_force_f64(q, k, v, attn_mask=None, is_causal=False, causal_offset=0, scale=None):
    """float64 softmax(scale*QK^T + mask) V with zero rows for fully masked rows.

    Returns (out, lse[B,H,Q], probabilities).  K/V heads are expanded for GQA.
    """
    q = np.asarray(q, np.float64)
    hq = q.shape[1]
    k = expand_gqa(np.asarray(k, np.float64), hq)
    v = expand_gqa(np.asarray(v, np.float64), hq)
    b, _, qlen, dim = q.shape
    klen = k.shape[2]
    mult = 1 / math.sqrt(dim) if scale is None else scale
    s = np.einsum("bhqd,bhkd->bhqk", q, k) * mult
    if attn_mask is not None and np.asarray(attn_mask).dtype != np.bool_:
        s = s + np.broadcast_to(np.asarray(attn_mask, np.float64), s.shape)
    allowed = allowed_matrix(b, hq, qlen, klen, attn_mask, is_causal, causal_offset)
    s = np.where(allowed, s, -np.inf)
    any_row = allowed.any(axis=-1, keepdims=True)
    m = np.where(any_row, np.max(np.where(allowed, s, -np.inf), axis=-1, keepdims=True), 0.0)
    e = np.where(allowed, np.exp(s - m), 0.0)
    total = e.sum(axis=-1, keepdims=True)
    p = np.where(any_row, e / np.where(any_row, total, 1.0), 0.0)
    out = np.einsum("bhqk,bhkd->bhqd", p, v)
    lse = np.where(any_row[..., 0], (m + np.log(np.where(any_row, total, 1.0)))[..., 0], -np.inf)
    return out, lse, p


def key_padding_mask(lengths, klen: int):
    """Boolean [B,1,1,K] key-valid mask (``docs/transformers.md:55`` of the reference)."""
    lengths = np.asarray(lengths)
    return (np.arange(klen)[None, :] < lengths[:, None])[:, None, None, :]


# ---------------------------------------------------------------------------
# int8 KV cache quantiser (``src/tensorsmith/nn/cache.py:73-77,91-98``)
# ---------------------------------------------------------------------------


def quantize_int8(x):
    """Symmetric per-token int8: scale = max(|x|_inf / 127, 1e-8), q = round(x/scale)."""
    x = np.asarray(x, np.float32)
    scale = np.maximum(np.max(np.abs(x), axis=-1, keepdims=True) / np.float32(127), np.float32(1e-8))
    return np.round(x / scale).astype(np.int8), scale.astype(np.float32)


def dequantize_int8(q, scale, dtype: str = "float32"):
    return round_to(q.astype(np.float32) * scale, dtype)
