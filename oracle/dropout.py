"""NumPy restatement of attention dropout on the hip path -- TEST
INFRASTRUCTURE.

The reference drops attention probabilities in its dense backend
(``src/tensorsmith/nn/attention.py:140-144``): keep = uniform >= p, mask =
keep / (1 - p) in the compute dtype, output = (P * mask) V; its VJP
(``:210-217``) uses P * mask for dV and multiplies dP by the mask before
dS = P (dP - rowsum(dP P)) scale.  Its uniforms come from the device's
global stream (``src/tensorsmith/device.py:276-297``), which no parallel
kernel can reproduce; the hip kernels draw them from a counter-based
generator instead, so that the backward (and any recompute) regenerates the
same mask from (key, counter):

* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
  easy as 1, 2, 3", SC'11), pinned in tests against the known-answer vectors
  of its Random123 release; word group n (16 words) of the stream with a
  128-bit key K = K0 + 2^64 K1 and counter c is the two blocks
  Philox4x32-10(t, key K0) and Philox4x32-10(t + 1, key K0), t = 2 (c + n)
  mod 2^64, of the 128-bit counter (lo32 t, hi32 t, lo32 K1, hi32 K1); each
  block's four 32-bit outputs are 8 words, little-endian (``raw_stream``
  packs them as uint64 outputs 4 n .. 4 n + 3);
* element (b, h, i, j) of a [B, H, Sq, Sk] problem takes 16-bit word
  L = ((b H + h) Sq + i) Sk16 + j of the stream viewed as little-endian uint16
  (Sk16 = Sk rounded up to 16): bits 16 (L % 4) .. 16 (L % 4) + 15 of raw
  output L // 4;
* it is kept iff that word >= round(p * 65536) (p resolved to 1/65536), and
  kept probabilities are multiplied by the reference's mask value
  keep.astype(compute dtype) / (1 - p) (``:141-143``): float32(1) /
  float32(1 - p) for half and float32 inputs, 1 / (1 - p) for float64.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module.
"""

from __future__ import annotations

import numpy as np

from .attention import Problem, _as_compute, expand_gqa, reduce_gqa, _finite_or_zero
from .halfprec import round_to

M0, M1 = 0xD2511F53, 0xCD9E8D57  # round multipliers
W0, W1 = 0x9E3779B9, 0xBB67AE85  # key bumps (golden ratio, sqrt(3) - 1)
_M32 = np.uint64(0xFFFFFFFF)
_S32 = np.uint64(32)


def philox4x32(c0, c1, c2, c3, k0: int, k1: int):
    """Philox4x32-10 of 128-bit counters (c0..c3: uint32 values held in
    uint64 arrays) under the 64-bit key (k0, k1)."""
    ka, kb = np.uint64(k0 & 0xFFFFFFFF), np.uint64(k1 & 0xFFFFFFFF)
    for r in range(10):
        if r:
            ka = (ka + np.uint64(W0)) & _M32
            kb = (kb + np.uint64(W1)) & _M32
        p0 = np.uint64(M0) * c0  # < 2^64: exact
        p1 = np.uint64(M1) * c2
        c0, c1, c2, c3 = (p1 >> _S32) ^ c1 ^ ka, p1 & _M32, (p0 >> _S32) ^ c3 ^ kb, p0 & _M32
    return c0, c1, c2, c3


def raw_stream(key: int, counter: int, n: int) -> np.ndarray:
    """First n raw uint64 outputs of the dropout stream: outputs 4 g .. 4 g + 3
    are word group g (block t = 2 (counter + g), then block t + 1; each block
    as (out0 | out1 << 32, out2 | out3 << 32))."""
    groups = (n + 3) // 4
    g = np.arange(groups, dtype=np.uint64)
    k_lo, k_hi = key & 0xFFFFFFFFFFFFFFFF, (key >> 64) & 0xFFFFFFFFFFFFFFFF
    with np.errstate(over="ignore"):
        t = (np.uint64(counter & 0xFFFFFFFFFFFFFFFF) + g) * np.uint64(2)
    outs = []
    for half in (0, 1):
        tt = t | np.uint64(half)
        c = (tt & _M32, tt >> _S32, np.full(groups, k_hi & 0xFFFFFFFF, np.uint64),
             np.full(groups, k_hi >> 32, np.uint64))
        x0, x1, x2, x3 = philox4x32(*c, k_lo & 0xFFFFFFFF, k_lo >> 32)
        outs += [x0 | (x1 << _S32), x2 | (x3 << _S32)]
    return np.stack(outs, axis=1).reshape(-1)[:n]


def threshold(p: float) -> int:
    """16-bit keep threshold: a word w is kept iff w >= threshold(p)."""
    return min(int(round(p * 65536.0)), 65536)


def keep_scale(p: float) -> np.float32:
    return np.float32(1.0) / np.float32(1.0 - p)


def keep_mask(key: int, counter: int, shape, p: float) -> np.ndarray:
    """Boolean keep mask [B, H, Sq, Sk] of the hip kernels' dropout."""
    b, h, sq, sk = shape
    sk16 = (sk + 15) // 16 * 16
    words = raw_stream(key, counter, b * h * sq * sk16 // 4).view("<u2")
    return words.reshape(b, h, sq, sk16)[..., :sk] >= threshold(p)


def sdpa_dropout(query, key, value, attn_mask=None, is_causal=False, *, dtype: str, p: float,
                 rng_key: int, rng_counter: int = 0, scale=None, causal_offset: int = 0,
                 enable_gqa: bool = False):
    """Dense attention with dropout (``attention.py:132-145``) under the
    keep mask above; returns (out in the compute dtype, out rounded to
    ``dtype``, backward(g) -> (dq, dk, dv)) following ``:210-219``."""
    b, hq, sq, d = query.shape
    hkv, sk = key.shape[1], key.shape[2]
    mult = 1 / np.sqrt(d) if scale is None else scale
    q = _as_compute(query, dtype)
    k = expand_gqa(_as_compute(key, dtype), hq)
    v = expand_gqa(_as_compute(value, dtype), hq)
    mask, boolean = None, False
    if attn_mask is not None:
        boolean = attn_mask.dtype == np.bool_
        mask = np.broadcast_to(attn_mask, (b, hq, sq, sk))
    prob = Problem(mult, bool(is_causal), int(causal_offset), mask, boolean)
    ct = q.dtype
    s = prob.scores(q, k, 0, 0)
    m = _finite_or_zero(np.max(s, axis=-1, keepdims=True))
    e = np.exp(s - m)
    total = np.sum(e, axis=-1, keepdims=True)
    probs = e / np.where(total > 0, total, 1).astype(ct)
    # the reference's mask value, literally: keep.astype(compute dtype) / (1 - p)
    drop = keep_mask(rng_key, rng_counter, (b, hq, sq, sk), p).astype(ct) / (1 - p)
    out = np.matmul(probs * drop, v)

    def backward(g):
        g = np.asarray(g, np.float32).astype(ct)
        dv = np.matmul(np.swapaxes(probs * drop, -1, -2), g)
        dp = np.matmul(g, np.swapaxes(v, -1, -2)) * drop
        ds = probs * (dp - np.sum(dp * probs, axis=-1, keepdims=True)) * ct.type(mult)
        dq = np.matmul(ds, k)
        dk = np.matmul(np.swapaxes(ds, -1, -2), q)
        return dq, reduce_gqa(dk, hkv), reduce_gqa(dv, hkv)

    return out, round_to(out, dtype), backward
