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

* Philox4x64-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
  easy as 1, 2, 3", SC'11) -- the generator behind ``numpy.random.Philox``;
  ``raw_stream`` reproduces that bit generator's raw output for the same key
  and counter (pinned in tests against NumPy itself);
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

M0, M1 = 0xD2E7470EE14C6C93, 0xCA5A826395121157  # round multipliers
W0, W1 = 0x9E3779B97F4A7C15, 0xBB67AE8584CAA73B  # key bumps (golden ratio, sqrt(3) - 1)
_M32 = np.uint64(0xFFFFFFFF)
_S32 = np.uint64(32)


def _mulhilo(a, m: int):
    """(high, low) 64-bit halves of the 128-bit products a * m (uint64 a)."""
    al, ah = a & _M32, a >> _S32
    ml, mh = np.uint64(m & 0xFFFFFFFF), np.uint64(m >> 32)
    ll, lh, hl, hh = al * ml, al * mh, ah * ml, ah * mh
    mid = (ll >> _S32) + (lh & _M32) + (hl & _M32)
    lo = (ll & _M32) | ((mid & _M32) << _S32)
    hi = hh + (lh >> _S32) + (hl >> _S32) + (mid >> _S32)
    return hi, lo


def philox4x64(c0, c1, c2, c3, key: int):
    """Philox4x64-10 of counters (c0..c3 uint64 arrays) under a 128-bit key."""
    k0 = np.uint64(key & 0xFFFFFFFFFFFFFFFF)
    k1 = np.uint64((key >> 64) & 0xFFFFFFFFFFFFFFFF)
    with np.errstate(over="ignore"):
        for r in range(10):
            if r:
                k0 = k0 + np.uint64(W0)
                k1 = k1 + np.uint64(W1)
            hi0, lo0 = _mulhilo(c0, M0)
            hi1, lo1 = _mulhilo(c2, M1)
            c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
    return c0, c1, c2, c3


def raw_stream(key: int, counter: int, n: int) -> np.ndarray:
    """First n raw uint64 outputs of a Philox(key, counter) bit generator:
    block b (outputs 4b .. 4b + 3) is Philox4x64-10 of counter + 1 + b."""
    blocks = (n + 3) // 4
    idx = np.arange(blocks, dtype=np.uint64)
    base = counter + 1
    with np.errstate(over="ignore"):
        c0 = np.uint64(base & 0xFFFFFFFFFFFFFFFF) + idx
    carry = (c0 < idx).astype(np.uint64)  # wrap past 2^64
    c1 = np.uint64((base >> 64) & 0xFFFFFFFFFFFFFFFF) + carry
    zero = np.zeros(blocks, dtype=np.uint64)
    out = philox4x64(c0, c1, zero, zero, key)
    return np.stack(out, axis=1).reshape(-1)[:n]


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
