"""ctypes binding of libtsattn.so for tensorsmith itself.

This module is what a tensorsmith maintainer adds as
``src/tensorsmith/_tsattn.py`` to route the reference's own
``scaled_dot_product_attention`` (``src/tensorsmith/nn/attention.py:16-252``)
to the MI355X kernels, next to the device allowlist entry
(``src/tensorsmith/device.py:34-38``) and the backend allowlist entry
(``nn/attention.py:55-56``, ``:78-80``).  It depends only on ctypes, NumPy
and torch-ROCm (the array library of a ``hip`` device) and declares the C ABI
of ``include/tsattn.h`` version 8; ``load()`` refuses any other
version.

The reference calls ``sdpa_hip`` from its dispatch and wraps the result the
way its other backends do (``nn/attention.py:250-252``)::

    out, backward = _tsattn.sdpa_hip(q, k, v, attn_mask, dropout_p, is_causal, scale,
                                      causal_offset, record=recording)
    return Tensor._from_op(out, (query, key, value), backward, "sdpa_hip")

``backward(g) -> (dq, dk, dv)`` returns arrays in the parents' dtypes, as the
VJP closure at ``nn/attention.py:200-248`` does.
"""

from __future__ import annotations

import ctypes
import math
import os
from ctypes import POINTER, c_char_p, c_double, c_int, c_int32, c_int64, c_size_t, c_uint64, c_void_p

import numpy as np
import torch

ABI_VERSION = 8
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP = 0, 1, 2, 3
MASK_NONE, MASK_BOOL, MASK_ADDITIVE = 0, 1, 2
BOOL_CODE = 4
DTYPES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.float64: 3}


class View(ctypes.Structure):
    """tsattn_view: device pointer + four element strides (innermost 1)."""

    _fields_ = [("data", c_void_p), ("stride", c_int64 * 4)]


class Problem(ctypes.Structure):
    """tsattn_problem (160 bytes): every field of include/tsattn.h, in order."""

    _fields_ = [
        ("dtype", c_int32), ("batch", c_int32), ("heads_q", c_int32), ("heads_kv", c_int32),
        ("len_q", c_int32), ("len_kv", c_int32), ("dim_qk", c_int32), ("dim_v", c_int32),
        ("scale", c_double),
        ("is_causal", c_int32),
        ("causal_offset", c_int64),
        ("kv_len", c_void_p), ("kv_prefix", c_void_p),
        ("mask_kind", c_int32), ("mask_dtype", c_int32),
        ("mask", View),
        ("dropout_p", c_double),
        ("dropout_key", c_uint64 * 2),
        ("dropout_counter", c_uint64),
        ("dropout_bits", c_void_p),
    ]


class RopeDesc(ctypes.Structure):
    """tsattn_rope_desc: cos / sin tables, rotary dim, query / key positions,
    optional rotated-query buffer."""

    _fields_ = [("cos", c_void_p), ("sin", c_void_p), ("rotary_dim", c_int32),
                ("q_pos0", c_int64), ("k_pos0", c_int64), ("q_rotated", c_void_p)]


_P, _V = POINTER(Problem), POINTER(View)
_SIGNATURES = {
    "tsattn_abi_version": (c_int, []),
    "tsattn_last_error": (c_char_p, []),
    "tsattn_sdpa_forward": (c_int, [_P, _V, _V, _V, _V, c_void_p, c_void_p]),
    "tsattn_sdpa_backward_workspace": (c_size_t, [_P]),
    "tsattn_sdpa_backward": (c_int, [_P, _V, _V, _V, _V, _V, c_void_p, _V, _V, _V, c_void_p,
                                     c_size_t, c_void_p]),
    "tsattn_dropout_bits_bytes": (c_size_t, [_P]),
    "tsattn_decode_workspace": (c_size_t, [_P, c_int32]),
    "tsattn_decode_forward": (c_int, [_P, _V, _V, _V, _V, c_int32, c_void_p, c_size_t, c_void_p]),
    "tsattn_key_mask_lengths": (c_int, [c_void_p, c_int64, c_int64, c_int32, c_int32, c_void_p,
                                        c_void_p, c_void_p]),
    "tsattn_kv_append_int8": (c_int, [c_int32, c_int32, c_int32, c_int32, c_int32, _V, _V, _V,
                                      c_int64, c_void_p]),
    "tsattn_qkv_rope_append": (c_int, [c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,
                                       _V, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       _V, _V, _V, _V, _V, c_void_p, c_void_p, c_int64, c_void_p]),
}

_lib = None


def library_path() -> str:
    """$TSATTN_LIBRARY, else the in-tree build next to this package."""
    env = os.environ.get("TSATTN_LIBRARY")
    if env:
        return env
    here = os.path.dirname(os.path.abspath(__file__))
    return os.path.join(os.path.dirname(here), "tensorsmith_hip", "_native", "libtsattn.so")


def load(path: str | None = None):
    """Load libtsattn.so once, declare the entry points, check the ABI version."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    lib = ctypes.CDLL(path or library_path())
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    version = lib.tsattn_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"libtsattn.so speaks ABI {version}; this binding needs {ABI_VERSION}")
    if path is None:
        _lib = lib
    return lib


def check(rc: int) -> None:
    """Status -> the exception the reference raises for the same condition
    (``nn/attention.py:36-86``: ValueError / TypeError for contract
    violations)."""
    if rc == OK:
        return
    raw = load().tsattn_last_error()
    msg = raw.decode() if raw else f"libtsattn status {rc}"
    if rc == ERR_INVALID:
        raise TypeError(msg) if ("dtype" in msg or "floating" in msg) else ValueError(msg)
    if rc == ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


def view(t: torch.Tensor) -> View:
    v = View(t.data_ptr())
    for i, s in enumerate(t.stride()):
        v.stride[i] = s
    if t.shape[-1] == 1:
        v.stride[3] = 1
    return v


def _stream(t: torch.Tensor) -> c_void_p:
    return c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def problem(q, k, v, *, is_causal=False, scale=None, causal_offset=0) -> Problem:
    """The sizes, scale and causal fields of one call (``nn/attention.py:58-60``:
    scale defaults to 1 / sqrt(Dqk))."""
    b, hq, sq, d = q.shape
    p = Problem()
    p.dtype = DTYPES[q.dtype]
    p.batch, p.heads_q, p.heads_kv = b, hq, k.shape[1]
    p.len_q, p.len_kv, p.dim_qk, p.dim_v = sq, k.shape[2], d, v.shape[3]
    p.scale = 1 / math.sqrt(d) if scale is None else float(scale)
    p.is_causal = int(bool(is_causal))
    p.causal_offset = int(causal_offset)
    p.mask_kind = MASK_NONE
    return p


def set_mask(p: Problem, mask: torch.Tensor, keep: list) -> None:
    """Broadcast a bool (True = allowed) or additive float mask to
    [B, Hq, Sq, Sk] (``nn/attention.py:64-75``); a bool key-padding mask
    [B, 1, 1, K] also gets per-row lengths so the kernels stop each row there."""
    b, hq, sq, sk = p.batch, p.heads_q, p.len_q, p.len_kv
    m = torch.broadcast_to(mask, (b, hq, sq, sk))
    boolean = m.dtype == torch.bool
    p.mask_kind = MASK_BOOL if boolean else MASK_ADDITIVE
    p.mask_dtype = BOOL_CODE if boolean else DTYPES[m.dtype]
    p.mask = view(m)
    p.mask.stride[3] = m.stride(3)
    keep.append(m)
    if boolean and all(m.stride(d) == 0 or m.shape[d] == 1 for d in (1, 2)):
        lens = torch.empty(2, b, dtype=torch.int32, device=m.device)
        check(load().tsattn_key_mask_lengths(c_void_p(m.data_ptr()), m.stride(0), m.stride(3), b,
                                             sk, c_void_p(lens[0].data_ptr()),
                                             c_void_p(lens[1].data_ptr()), _stream(m)))
        p.kv_len, p.kv_prefix = lens[0].data_ptr(), lens[1].data_ptr()
        keep.append(lens)


def set_dropout(p: Problem, dropout_p: float, key: int | None = None, counter: int = 0) -> int:
    """Attention dropout (``nn/attention.py:140-144``) on the kernels'
    counter-based stream.  ``key`` (128-bit) defaults to a draw from NumPy's
    global state, so ``ts.seed`` reproduces it and a checkpoint that restores
    that state (``nn/checkpoint.py:48,79``) replays the same mask.  Returns
    the key."""
    if key is None:
        key = int.from_bytes(np.random.bytes(16), "little")
    p.dropout_p = float(dropout_p)
    p.dropout_key[0], p.dropout_key[1] = key & (2**64 - 1), key >> 64
    p.dropout_counter = int(counter)
    return key


def sdpa_hip(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, scale=None,
             causal_offset=0, *, record=True, dropout_key=None):
    """Attention of torch-ROCm [B, H, S, D] tensors (any strides, innermost 1)
    through tsattn_sdpa_forward.  Returns ``(out, backward)``; ``backward``
    is None when not recording (the ``native`` early return,
    ``nn/attention.py:172-173``)."""
    q, k, v = (t if t.stride(-1) == 1 else t.contiguous() for t in (query, key, value))
    p = problem(q, k, v, is_causal=is_causal, scale=scale, causal_offset=causal_offset)
    keep: list = []
    if attn_mask is not None:
        set_mask(p, attn_mask, keep)
    if dropout_p:
        set_dropout(p, dropout_p, dropout_key)
    lib = load()
    b, hq, sq, _ = q.shape
    out = torch.empty((b, hq, sq, v.shape[3]), dtype=q.dtype, device=q.device)
    lse = None
    if record:
        lse = torch.empty((b, hq, sq), dtype=torch.float64 if q.dtype == torch.float64
                          else torch.float32, device=q.device)
        if dropout_p:  # the forward writes its keep mask as bits, the backward reads them
            bits = torch.empty(lib.tsattn_dropout_bits_bytes(p), dtype=torch.uint8, device=q.device)
            p.dropout_bits = bits.data_ptr()
            keep.append(bits)
    check(lib.tsattn_sdpa_forward(p, view(q), view(k), view(v), view(out),
                                  None if lse is None else lse.data_ptr(), _stream(q)))
    if not record:
        return out, None

    def backward(g, _keep=keep):
        g = g if g.stride(-1) == 1 else g.contiguous()
        g = g.to(out.dtype)
        dq, dk, dv = (torch.empty(t.shape, dtype=t.dtype, device=t.device) for t in (q, k, v))
        nbytes = lib.tsattn_sdpa_backward_workspace(p)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
        check(lib.tsattn_sdpa_backward(p, view(q), view(k), view(v), view(out), view(g),
                                       lse.data_ptr(), view(dq), view(dk), view(dv),
                                       ws.data_ptr(), nbytes, _stream(q)))
        return dq, dk, dv

    return out, backward


def decode(query, k_cache, v_cache, length, *, is_causal=True, causal_offset=None, scale=None,
           kv_len=None):
    """Cached decode (``MultiHeadAttention.forward`` with a ``KVCache``,
    ``nn/transformer.py:142-154``): ``query`` [B, Hq, Q, D] against the first
    ``length`` rows of the cache arrays [B, Hkv, capacity, D], split across the
    cache.  ``causal_offset`` defaults to ``length - Q`` (the cache already
    holds the new rows); ``kv_len`` (int32 [B], optional) shortens rows."""
    q = query if query.stride(-1) == 1 else query.contiguous()
    kv = k_cache[:, :, :length]
    p = problem(q, kv, v_cache[:, :, :length], is_causal=is_causal, scale=scale,
                causal_offset=length - q.shape[2] if causal_offset is None else causal_offset)
    if kv_len is not None:
        p.kv_len = kv_len.data_ptr()
    lib = load()
    out = torch.empty(q.shape[:3] + (v_cache.shape[3],), dtype=q.dtype, device=q.device)
    nbytes = lib.tsattn_decode_workspace(p, 0)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    check(lib.tsattn_decode_forward(p, view(q), view(k_cache), view(v_cache), view(out), 0,
                                    ws.data_ptr(), nbytes, _stream(q)))
    return out


def append_int8(rows, codes, scales, pos: int) -> None:
    """``KVCache.append`` into the int8 format (``nn/cache.py:73-84``): rows
    [B, H, T, D] in the cache dtype -> codes[:, :, pos:pos+T] and their fp32
    row scales, bit-identical to the reference's quantiser."""
    b, h, t, d = rows.shape
    check(load().tsattn_kv_append_int8(DTYPES[rows.dtype], b, h, t, d, view(rows), view(codes),
                                       view(scales), int(pos), _stream(rows)))


def project_rope_append(x, weights, biases, q_out, k_cache, v_cache, scales, cos, sin, pos: int,
                        heads_q: int, heads_kv: int) -> None:
    """The cached ``MultiHeadAttention`` step before its attention call
    (``nn/transformer.py:124-142``) in one kernel: q / k / v projections of
    ``x`` [B, T, E] (``weights`` / ``biases``: the three ``Linear`` layers'
    arrays, biases may be None), RoPE of q and k at positions pos .. (cos /
    sin: the device tables of ``rotary_embedding``, or None) and the append
    of k and v at ``pos`` (``scales``: (key, value) fp32 scale arrays of an
    int8 cache, or None).  q_out [B, Hq, T, D] receives the rotated queries.
    Raises NotImplementedError outside the kernel's shapes and layouts (f16 /
    bf16, head dim 64 / 128, E % 16 == 0; contiguous weights [heads * D, E]
    and biases [heads * D] of x's dtype; x rows and the weights 16-byte
    aligned): project and append in steps then."""
    b, t, e = x.shape
    d = q_out.shape[-1]
    rows = (heads_q * d, heads_kv * d, heads_kv * d)
    for name, w, n in zip("qkv", weights, rows):
        if w.dtype != x.dtype or not w.is_contiguous() or tuple(w.shape) != (n, e) or w.data_ptr() % 16:
            raise NotImplementedError(f"the fused projection needs w{name} as a contiguous, 16-byte aligned "
                                      f"[{n}, {e}] {x.dtype} array (got {tuple(w.shape)} {w.dtype})")
    if biases is not None:
        for name, bz, n in zip("qkv", biases, rows):
            if bz is not None and (bz.dtype != x.dtype or not bz.is_contiguous() or tuple(bz.shape) != (n,)):
                raise NotImplementedError(f"the fused projection needs b{name} as a contiguous [{n}] "
                                          f"{x.dtype} array (got {tuple(bz.shape)} {bz.dtype})")
    if x.data_ptr() % 16 or x.stride(0) % 8 or x.stride(1) % 8 or x.stride(2) != 1:
        raise NotImplementedError("the fused projection needs x rows 16-byte aligned with unit column stride")
    xv = View(x.data_ptr())
    xv.stride[0], xv.stride[1], xv.stride[2], xv.stride[3] = x.stride(0), 0, x.stride(1), 1
    ptr = lambda a: None if a is None else a.data_ptr()
    bq, bk, bv = biases if biases is not None else (None, None, None)
    ks, vs = (None, None) if scales is None else (ctypes.byref(view(scales[0])), ctypes.byref(view(scales[1])))
    check(load().tsattn_qkv_rope_append(
        DTYPES[x.dtype], b, t, e, heads_q, heads_kv, q_out.shape[-1], ctypes.byref(xv),
        *(w.data_ptr() for w in weights), ptr(bq), ptr(bk), ptr(bv), view(q_out), view(k_cache),
        view(v_cache), ks, vs, ptr(cos), ptr(sin), int(pos), _stream(x)))
