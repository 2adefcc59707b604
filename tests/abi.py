"""Direct C-ABI drivers for the GPU tests (torch tensors in, torch tensors out).

These call ``libtsattn.so`` exactly as a foreign binding would: raw device
pointers, element strides, a ``tsattn_problem`` and the current stream.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import torch

from tensorsmith_hip import _lib

TORCH_DTYPES = {"float32": torch.float32, "float64": torch.float64,
                "float16": torch.float16, "bfloat16": torch.bfloat16}
CODES = {torch.float32: _lib.F32, torch.float64: _lib.F64, torch.float16: _lib.F16,
         torch.bfloat16: _lib.BF16}


def dev_tensor(x: np.ndarray, dtype: str) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda").to(TORCH_DTYPES[dtype])


def host(t: torch.Tensor) -> np.ndarray:
    t = t.detach()
    if t.dtype in (torch.bfloat16, torch.float16):
        t = t.float()
    return t.cpu().numpy()


def view(t: torch.Tensor) -> _lib.View:
    v = _lib.View()
    v.data = t.data_ptr()
    for i, s in enumerate(t.stride()):
        v.stride[i] = s
    return v


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def problem(q, k, v, *, causal=False, offset=0, scale=None, mask=None, kv_len=None,
            kv_prefix=None, dropout=None, dropout_bits=None):
    b, hq, sq, d = q.shape
    p = _lib.Problem()
    p.dtype = CODES[q.dtype]
    p.batch, p.heads_q, p.heads_kv, p.len_q = b, hq, k.shape[1], sq
    p.len_kv, p.dim_qk, p.dim_v = k.shape[2], d, v.shape[3]
    p.scale = 1 / math.sqrt(d) if scale is None else scale
    p.is_causal = int(causal)
    p.causal_offset = offset
    p.kv_len = None if kv_len is None else kv_len.data_ptr()
    p.kv_prefix = None if kv_prefix is None else kv_prefix.data_ptr()
    p.mask_kind = _lib.MASK_NONE
    if dropout is not None:  # (p, 128-bit key, counter)
        p.dropout_p = dropout[0]
        p.dropout_key[0] = dropout[1] & (2**64 - 1)
        p.dropout_key[1] = dropout[1] >> 64
        p.dropout_counter = dropout[2]
    if dropout_bits is not None:  # device buffer of tsattn_dropout_bits_bytes
        p.dropout_bits = dropout_bits.data_ptr()
    if mask is not None:
        m = torch.broadcast_to(mask, (b, hq, sq, k.shape[2]))
        if m.dtype == torch.bool:
            p.mask_kind, p.mask_dtype = _lib.MASK_BOOL, _lib.BOOL
        else:
            p.mask_kind, p.mask_dtype = _lib.MASK_ADDITIVE, CODES[m.dtype]
        p.mask = view(m)
        p._mask_keep = m
    return p


def forward(q, k, v, **kw):
    """(out, lse) through tsattn_sdpa_forward; returns the kernel path used."""
    p = problem(q, k, v, **kw)
    out = torch.empty(q.shape[:3] + (v.shape[3],), dtype=q.dtype, device=q.device)
    lse = torch.empty(q.shape[:3], dtype=torch.float64 if q.dtype == torch.float64 else torch.float32,
                      device=q.device)
    lib = _lib.load()
    _lib.check(lib.tsattn_sdpa_forward(ctypes.byref(p), view(q), view(k), view(v), view(out),
                                       ctypes.c_void_p(lse.data_ptr()), stream()), "forward")
    return out, lse, lib.tsattn_last_kernel_path()


def backward(q, k, v, out, g, lse, ws_bytes=None, **kw):
    """tsattn_sdpa_backward with the queried workspace, or ws_bytes of it."""
    p = problem(q, k, v, **kw)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    lib = _lib.load()
    nbytes = lib.tsattn_sdpa_backward_workspace(ctypes.byref(p)) if ws_bytes is None else ws_bytes
    ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    _lib.check(lib.tsattn_sdpa_backward(
        ctypes.byref(p), view(q), view(k), view(v), view(out), view(g),
        ctypes.c_void_p(lse.data_ptr()), view(dq), view(dk), view(dv),
        ctypes.c_void_p(ws.data_ptr()), nbytes, stream()), "backward")
    return dq, dk, dv, lib.tsattn_last_kernel_path()


def decode(q, k, v, split_len=0, **kw):
    p = problem(q, k, v, **kw)
    out = torch.empty(q.shape[:3] + (v.shape[3],), dtype=q.dtype, device=q.device)
    lib = _lib.load()
    nbytes = lib.tsattn_decode_workspace(ctypes.byref(p), split_len)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    _lib.check(lib.tsattn_decode_forward(ctypes.byref(p), view(q), view(k), view(v), view(out),
                                         split_len, ctypes.c_void_p(ws.data_ptr()), nbytes,
                                         stream()), "decode")
    return out


def decode_rope(q, k, v, desc, ks=None, vs=None, split_len=0, **kw):
    """tsattn_decode_forward_rope: q unrotated, the cache rows rotated; int8
    caches pass their row scales ks / vs (len_kv in kw then)."""
    len_kv = kw.pop("len_kv", None)
    p = problem(q, k, v, **kw)
    if len_kv is not None:
        p.len_kv = len_kv
    out = torch.empty(q.shape[:3] + (v.shape[3],), dtype=q.dtype, device=q.device)
    lib = _lib.load()
    nbytes = lib.tsattn_decode_workspace(ctypes.byref(p), split_len)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    _lib.check(lib.tsattn_decode_forward_rope(
        ctypes.byref(p), ctypes.byref(desc), view(q), view(k), view(v),
        None if ks is None else view(ks), None if vs is None else view(vs), view(out), split_len,
        ctypes.c_void_p(ws.data_ptr()), nbytes, stream()), "decode rope")
    return out


def key_lengths(mask: torch.Tensor):
    """kv_len / kv_prefix of a bool key mask [B, K] via tsattn_key_mask_lengths."""
    b, kl = mask.shape
    out = torch.empty(2, b, dtype=torch.int32, device=mask.device)
    _lib.check(_lib.load().tsattn_key_mask_lengths(
        ctypes.c_void_p(mask.data_ptr()), mask.stride(0), mask.stride(1), b, kl,
        ctypes.c_void_p(out[0].data_ptr()), ctypes.c_void_p(out[1].data_ptr()), stream()),
        "key lengths")
    return out[0], out[1]


class generic_only:
    """Context: force the generic kernel family (tsattn_set_kernel_policy(1))."""

    def __enter__(self):
        _lib.set_kernel_policy(1)

    def __exit__(self, *exc):
        _lib.set_kernel_policy(0)
        return False


def decode_int8(q, k8, v8, kscale, vscale, len_kv, split_len=0, **kw):
    """tsattn_decode_forward_int8 over the first len_kv rows of int8 caches."""
    p = problem(q, k8, v8, **kw)
    p.len_kv = len_kv
    out = torch.empty(q.shape[:3] + (v8.shape[3],), dtype=q.dtype, device=q.device)
    lib = _lib.load()
    nbytes = lib.tsattn_decode_workspace(ctypes.byref(p), split_len)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    _lib.check(lib.tsattn_decode_forward_int8(
        ctypes.byref(p), view(q), view(k8), view(v8), view(kscale), view(vscale), view(out),
        split_len, ctypes.c_void_p(ws.data_ptr()), nbytes, stream()), "int8 decode")
    return out, lib.tsattn_last_kernel_path()


def kv_append_int8(src, codes, scales, pos):
    """tsattn_kv_append_int8: quantise src [B,H,T,D] into codes/scales at pos."""
    b, h, t, d = src.shape
    _lib.check(_lib.load().tsattn_kv_append_int8(
        CODES[src.dtype], b, h, t, d, view(src), view(codes), view(scales), pos, stream()),
        "int8 append")


def rope(x, out, cos, sin, pos0, rotary_dim, inverse=False):
    """tsattn_rope: rotate x [B,H,T,D] into out with table rows pos0 + t."""
    b, h, t, d = x.shape
    _lib.check(_lib.load().tsattn_rope(
        CODES[x.dtype], b, h, t, d, rotary_dim, view(x), view(out),
        ctypes.c_void_p(cos.data_ptr()), ctypes.c_void_p(sin.data_ptr()), pos0, int(inverse),
        stream()), "rope")


def rope_append(k, v, kc, vc, cos, sin, pos, rotary_dim, ks=None, vs=None):
    """tsattn_rope_append: rotate k, write k / v rows into the caches at pos
    (int8 codes + scales when ks / vs are given)."""
    b, h, t, d = k.shape
    scales = tuple(None if s is None else ctypes.byref(view(s)) for s in (ks, vs))
    _lib.check(_lib.load().tsattn_rope_append(
        CODES[k.dtype], b, h, t, d, rotary_dim, view(k), view(v), view(kc), view(vc), *scales,
        ctypes.c_void_p(cos.data_ptr() if cos is not None else 0),
        ctypes.c_void_p(sin.data_ptr() if sin is not None else 0), pos, stream()), "rope append")


def rope_desc(cos, sin, rotary_dim, q_pos0, k_pos0):
    d = _lib.RopeDesc()
    d.cos, d.sin = cos.data_ptr(), sin.data_ptr()
    d.rotary_dim, d.q_pos0, d.k_pos0 = rotary_dim, q_pos0, k_pos0
    return d


def forward_rope(q, k, v, desc, **kw):
    """tsattn_sdpa_forward_rope: q unrotated, k rotated."""
    p = problem(q, k, v, **kw)
    out = torch.empty(q.shape[:3] + (v.shape[3],), dtype=q.dtype, device=q.device)
    lse = torch.empty(q.shape[:3], dtype=torch.float32, device=q.device)
    lib = _lib.load()
    _lib.check(lib.tsattn_sdpa_forward_rope(ctypes.byref(p), ctypes.byref(desc), view(q), view(k),
                                            view(v), view(out), ctypes.c_void_p(lse.data_ptr()),
                                            stream()), "forward rope")
    return out, lse, lib.tsattn_last_kernel_path()


def backward_rope(q, k, v, out, g, lse, desc, ws_bytes=None, **kw):
    """tsattn_sdpa_backward_rope: gradients of the unrotated q and k (with the
    queried workspace, or ws_bytes of it)."""
    p = problem(q, k, v, **kw)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    lib = _lib.load()
    nbytes = lib.tsattn_sdpa_backward_rope_workspace(ctypes.byref(p)) if ws_bytes is None else ws_bytes
    ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    _lib.check(lib.tsattn_sdpa_backward_rope(
        ctypes.byref(p), ctypes.byref(desc), view(q), view(k), view(v), view(out), view(g),
        ctypes.c_void_p(lse.data_ptr()), view(dq), view(dk), view(dv),
        ctypes.c_void_p(ws.data_ptr()), nbytes, stream()), "backward rope")
    return dq, dk, dv


def dropout_bits_buffer(q, k, v, **kw):
    """A device buffer of tsattn_dropout_bits_bytes for the problem, as int32
    words [B, Hq, ceil(Sk / 32), round_up(Sq, 4)]."""
    p = problem(q, k, v, **kw)
    nbytes = _lib.load().tsattn_dropout_bits_bytes(ctypes.byref(p))
    b, hq, sq = q.shape[:3]
    nkt, sqp = -(-k.shape[2] // 32), -(-sq // 4) * 4
    assert nbytes == b * hq * nkt * sqp * 4
    return torch.full((b, hq, nkt, sqp), -1, dtype=torch.int32, device=q.device)


def dropout_keep(q, k, v, **kw):
    """tsattn_dropout_keep: the [B, Hq, Sq, Sk] uint8 keep mask of the problem."""
    p = problem(q, k, v, **kw)
    out = torch.empty((p.batch, p.heads_q, p.len_q, p.len_kv), dtype=torch.uint8, device=q.device)
    _lib.check(_lib.load().tsattn_dropout_keep(ctypes.byref(p), ctypes.c_void_p(out.data_ptr()),
                                               stream()), "dropout keep")
    return out


def qkv_rope_append(x, wq, wk, wv, bias, q_out, kc, vc, scales, cos, sin, pos, heads_q, heads_kv):
    """tsattn_qkv_rope_append: x [B, T, E]; bias = (bq, bk, bv) or None;
    scales = (ks, vs) for int8 caches or None; cos = None skips RoPE."""
    b, t, e = x.shape
    d = q_out.shape[-1]
    bq, bk, bv = bias if bias is not None else (None, None, None)
    ptr = lambda z: ctypes.c_void_p(z.data_ptr()) if z is not None else None
    sc = (view(scales[0]), view(scales[1])) if scales is not None else (None, None)
    _lib.check(_lib.load().tsattn_qkv_rope_append(
        CODES[x.dtype], b, t, e, heads_q, heads_kv, d, view(x.unsqueeze(1)), ptr(wq), ptr(wk), ptr(wv),
        ptr(bq), ptr(bk), ptr(bv), view(q_out), view(kc), view(vc), *sc, ptr(cos), ptr(sin), pos,
        stream()), "fused projection")
