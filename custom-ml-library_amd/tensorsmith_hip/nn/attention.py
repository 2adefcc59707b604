"""``scaled_dot_product_attention`` on hip devices, through ``libtsattn.so``.

Same signature, argument meaning and refusals as the reference
(``src/tensorsmith/nn/attention.py:16-86``), with ``"hip"`` added to the
backend allowlist and chosen by ``auto`` on a hip device (as ``native`` is on
Metal, ``:78-80``).  ``dense`` and ``streaming`` name the same exact math;
on hip both run the HIP kernels (online softmax, saved LSE, recomputing VJP).
Dropout runs in the kernels on ``hip`` / ``dense`` / ``auto`` and is refused on
``streaming`` / ``native`` like the reference (``:83-84``).

Kernel routing (all on the GPU, none on the CPU):

* training / prefill: ``tsattn_sdpa_forward`` + ``tsattn_sdpa_backward``
  (MFMA kernels for f16/bf16 and head dim 64/128, generic kernels otherwise);
* inference with a handful of query rows per KV head (cached decode):
  ``tsattn_decode_forward``, split across the cache.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np

from .. import _lib
from ..device import attention_dropout_key, current_stream
from ..tensor import Tensor, is_grad_enabled

BACKENDS = {"auto", "dense", "streaming", "native", "hip"}
DECODE_MIN_KEYS = 128  # below this the prefill kernel is as fast


def _dtype_code(dtype) -> int:
    name = str(dtype).split(".")[-1]
    codes = {"float32": _lib.F32, "float16": _lib.F16, "bfloat16": _lib.BF16, "float64": _lib.F64}
    if name not in codes:
        raise TypeError("attention inputs must have the same floating-point dtype")
    return codes[name]


def _operand(t):
    """Raw torch tensor with a unit innermost stride (copies only if needed)."""
    return t if t.stride(-1) == 1 or t.shape[-1] == 1 else t.contiguous()


def _view(t) -> _lib.View:
    v = _lib.View()
    v.data = t.data_ptr()
    st = list(t.stride())
    if t.shape[-1] == 1:
        st[-1] = 1
    for i, s in enumerate(st):
        v.stride[i] = s
    return v


def _round256(n: int) -> int:
    return (n + 255) // 256 * 256


def _rows_workspace(prob, fused: bool, dtype) -> int:
    """Smallest backward workspace the C ABI accepts (tsattn.h: the row
    values, then the rotated query rows with RoPE folded in, then the keep
    bits when dropping without the forward's): the kernels then recompute S
    and dP for dQ instead of storing dS."""
    import torch

    rows = prob.batch * prob.heads_q * prob.len_q
    nbytes = 2 * rows * (8 if dtype == torch.float64 else 4)
    if fused:
        nbytes = _round256(nbytes) + rows * prob.dim_qk * 2
    if prob.dropout_p > 0 and not prob.dropout_bits:
        nbytes = _round256(nbytes) + _lib.load().tsattn_dropout_bits_bytes(ctypes.byref(prob))
    return nbytes


def _aligned16(t) -> bool:
    return t.data_ptr() % 16 == 0 and all(s % 8 == 0 for s in t.stride()[:3])


def _problem(b, hq, hkv, sq, sk, dqk, dv, dtype_code, scale, is_causal, offset):
    p = _lib.Problem()
    p.dtype = dtype_code
    p.batch, p.heads_q, p.heads_kv = b, hq, hkv
    p.len_q, p.len_kv, p.dim_qk, p.dim_v = sq, sk, dqk, dv
    p.scale = scale
    p.is_causal = 1 if is_causal else 0
    p.causal_offset = offset
    p.mask_kind = _lib.MASK_NONE
    return p


def scaled_dot_product_attention(
    query: Tensor,
    key: Tensor,
    value: Tensor,
    attn_mask: Tensor | None = None,
    dropout_p: float = 0.0,
    is_causal: bool = False,
    *,
    scale: float | None = None,
    causal_offset: int = 0,
    backend: str = "auto",
    block_size: int = 64,
    enable_gqa: bool = False,
    _rope: tuple | None = None,
) -> Tensor:
    """Attention for [batch, heads, sequence, channels] tensors.

    Boolean masks use True=allowed; floating masks are added to scores. Fully
    masked rows return zero with zero gradients. ``causal_offset`` is the
    absolute position of the first query in a cached key sequence.
    ``block_size`` is accepted for signature compatibility; the kernels use
    their own tiles.

    ``_rope = (q_pos0, k_pos0, base)`` (used by ``MultiHeadAttention``, not
    part of the reference signature): query and key are *unrotated*; the
    result and gradients are those of ``rotary_embedding(query, q_pos0)`` and
    ``rotary_embedding(key, k_pos0)`` fed to this function, bit for bit.  The
    keys are rotated once by the RoPE kernel; the query rotation and both
    inverse rotations of the gradients run inside the MFMA kernels
    (``tsattn_sdpa_forward_rope`` / ``_backward_rope``), with separate RoPE
    kernels where those do not apply.  ``k_pos0 = None``: the keys arrive
    already rotated (a KV cache) and only the query is rotated -- inside the
    decode kernel (``tsattn_decode_forward_rope``) when that runs.  Other
    dtypes than f32 / f16 / bf16 (float64) are rotated by ``rotary_embedding``
    first and then attended as usual.
    """
    if (_rope is not None and getattr(query, "device", None) is not None
            and query.device.type == "hip" and query._data.dtype not in _ROPE_KERNEL_DTYPES()):
        q_pos0, k_pos0, base = _rope
        query = rotary_embedding(query, q_pos0, base)
        if k_pos0 is not None:
            key = rotary_embedding(key, k_pos0, base)
        _rope = None
    # --- the reference's validation, same order and messages (:36-62) ---
    if any(t.ndim != 4 for t in (query, key, value)):
        raise ValueError("attention expects [batch, heads, sequence, channels]")
    if query.device != key.device or query.device != value.device:
        raise ValueError("attention tensors must be on the same device")
    if query.dtype != key.dtype or query.dtype != value.dtype or "float" not in str(query.dtype):
        raise TypeError("attention inputs must have the same floating-point dtype")
    if query.shape[0] != key.shape[0] or key.shape[:3] != value.shape[:3]:
        raise ValueError("attention batch/head dimensions and key/value lengths must agree")
    repetitions = query.shape[1] // key.shape[1] if key.shape[1] else 0
    if query.shape[1] != key.shape[1] and (
        not enable_gqa or not repetitions or query.shape[1] % key.shape[1]
    ):
        raise ValueError(
            "grouped-query attention requires enable_gqa and query heads divisible by KV heads"
        )
    if query.shape[-1] != key.shape[-1] or min(*query.shape, *key.shape, *value.shape) <= 0:
        raise ValueError("query/key head dimensions must match and sequences must be nonempty")
    if not 0 <= dropout_p < 1 or block_size <= 0 or causal_offset < 0:
        raise ValueError("invalid dropout probability, block size, or causal offset")
    if backend not in BACKENDS:
        raise ValueError("attention backend must be auto, dense, streaming, native, or hip")
    b, hq, qlen, dim = query.shape
    hkv, klen, dim_v = key.shape[1], key.shape[2], value.shape[-1]
    multiplier = 1 / math.sqrt(dim) if scale is None else scale
    if not math.isfinite(multiplier):
        raise ValueError("attention scale must be finite")
    if query.device.type != "hip":
        raise RuntimeError(
            "tensorsmith_hip runs attention on hip devices only; move the tensors to 'hip'"
        )
    # the reference drops only in its dense backend, which "auto" selects when
    # dropping (attention.py:77-84); "hip" drops on the kernels as well
    if dropout_p and backend in ("streaming", "native"):
        raise ValueError("attention dropout currently requires the dense backend")
    if backend == "native":
        raise ValueError("native attention requires Metal and equal query/value head dimensions")

    code = _dtype_code(query.dtype)
    q, k, v = (_operand(t._data) for t in (query, key, value))
    import torch

    tdev = q.device
    prob = _problem(b, hq, hkv, qlen, klen, dim, dim_v, code, multiplier, is_causal, causal_offset)
    if dropout_p:
        # a fresh 128-bit Philox key per call from the host stream (ts.seed),
        # recorded / replayed under a checkpoint; the backward reads the keep
        # mask the forward drew from it
        drop_key = attention_dropout_key()
        prob.dropout_p = float(dropout_p)
        prob.dropout_key[0] = drop_key & (2**64 - 1)
        prob.dropout_key[1] = drop_key >> 64
        prob.dropout_counter = 0
    keep = []  # device buffers the launch reads, alive until the call returns

    if attn_mask is not None:
        if not any(name in str(attn_mask.dtype) for name in ("bool", "float")):
            raise TypeError("attention masks must be boolean or floating point")
        if attn_mask.requires_grad or attn_mask.device != query.device:
            raise ValueError("attention masks must be non-differentiable and on the input device")
        try:
            mask = torch.broadcast_to(attn_mask._data, (b, hq, qlen, klen))
        except (ValueError, RuntimeError) as error:
            raise ValueError("attention mask is not broadcastable to [B,H,Q,K]") from error
        boolean = "bool" in str(attn_mask.dtype)
        prob.mask_kind = _lib.MASK_BOOL if boolean else _lib.MASK_ADDITIVE
        prob.mask_dtype = _lib.BOOL if boolean else _dtype_code(attn_mask.dtype)
        prob.mask = _view(mask)
        prob.mask.stride[3] = mask.stride(3)
        keep.append(mask)
        if boolean and all(mask.stride(d) == 0 or mask.shape[d] == 1 for d in (1, 2)):
            # key-padding mask [B,1,1,K]: derive per-row key lengths on device
            lens = torch.empty(2, b, dtype=torch.int32, device=tdev)
            _lib.check(
                _lib.load().tsattn_key_mask_lengths(
                    ctypes.c_void_p(mask.data_ptr()), mask.stride(0), mask.stride(3), b, klen,
                    ctypes.c_void_p(lens[0].data_ptr()), ctypes.c_void_p(lens[1].data_ptr()),
                    ctypes.c_void_p(current_stream(query.device)),
                ),
                "key mask lengths",
            )
            prob.kv_len = lens[0].data_ptr()
            prob.kv_prefix = lens[1].data_ptr()
            keep.append(lens)

    lib = _lib.load()
    stream = ctypes.c_void_p(current_stream(query.device))
    recording = is_grad_enabled() and any(t.requires_grad for t in (query, key, value))
    out = torch.empty((b, hq, qlen, dim_v), dtype=q.dtype, device=tdev)
    rope = None  # (descriptor, tables) when the kernels fold the query rotation in
    if _rope is not None:
        q_pos0, k_pos0, base = _rope
        if (dim % 2 or q_pos0 < 0 or (k_pos0 is not None and k_pos0 < 0) or base <= 0
                or not math.isfinite(base)
                or q.dtype not in (torch.float32, torch.float16, torch.bfloat16)):
            raise ValueError("RoPE requires a positive even rotary dimension and valid positions/base")
        if k_pos0 is not None:
            k = _rope_rows(k, k_pos0, base, dim, False, query.device)
        tables = rope_tables(base, dim, q.dtype, tdev,
                             max(q_pos0 + qlen, 0 if k_pos0 is None else k_pos0 + klen))
        desc = _lib.RopeDesc()
        desc.cos, desc.sin = tables[0].data_ptr(), tables[1].data_ptr()
        desc.rotary_dim, desc.q_pos0, desc.k_pos0 = dim, q_pos0, k_pos0 or 0
        rope = (desc, tables)
    vq, vk, vv, vo = _view(q), _view(k), _view(v), _view(out)

    use_decode = (
        not recording
        and not dropout_p
        and code in (_lib.F16, _lib.BF16, _lib.F32)
        and dim == dim_v
        and dim in (64, 128, 256)
        and repetitions * qlen <= 8
        and klen >= DECODE_MIN_KEYS
        and all(_aligned16(t) for t in (q, k, v))
    )
    if use_decode:
        nbytes = lib.tsattn_decode_workspace(ctypes.byref(prob), 0)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=tdev)
        ws_ptr = ctypes.c_void_p(ws.data_ptr())
        folded = False
        if rope is not None:
            try:  # the query rotation inside the decode kernel
                _lib.check(lib.tsattn_decode_forward_rope(
                    ctypes.byref(prob), ctypes.byref(rope[0]), vq, vk, vv, None, None, vo, 0,
                    ws_ptr, nbytes, stream), "decode forward")
                folded = True
            except NotImplementedError:  # e.g. a rotary dim the kernel does not fold
                q = _rope_rows(q, q_pos0, base, dim, False, query.device)
                vq = _view(q)
        if not folded:
            _lib.check(lib.tsattn_decode_forward(ctypes.byref(prob), vq, vk, vv, vo, 0, ws_ptr,
                                                 nbytes, stream), "decode forward")
        return Tensor._from_op(out, (query, key, value), None, "sdpa_hip")

    lse = None
    if recording:
        lse_dtype = torch.float64 if code == _lib.F64 else torch.float32
        lse = torch.empty((b, hq, qlen), dtype=lse_dtype, device=tdev)
        if dropout_p:
            # the forward writes its keep mask as bits; the backward reads them
            bits = torch.empty(lib.tsattn_dropout_bits_bytes(ctypes.byref(prob)), dtype=torch.uint8,
                               device=tdev)
            prob.dropout_bits = bits.data_ptr()
            keep.append(bits)
    lse_ptr = ctypes.c_void_p(None if lse is None else lse.data_ptr())
    fused = False
    if rope is not None and k_pos0 is None:
        # keys given rotated: their gradient takes no inverse rotation, which the
        # folded backward would apply; rotate the queries on their own
        q = _rope_rows(q, q_pos0, base, dim, False, query.device)
        vq = _view(q)
    elif rope is not None:
        if recording:
            # the forward also stores the rotated queries, which the backward's
            # dK/dV kernel reads (instead of rotating and staging them again)
            q_rot = torch.empty((b, hq, qlen, dim), dtype=q.dtype, device=tdev)
            rope[0].q_rotated = q_rot.data_ptr()
            keep.append(q_rot)
        try:
            _lib.check(lib.tsattn_sdpa_forward_rope(ctypes.byref(prob), ctypes.byref(rope[0]), vq, vk,
                                                    vv, vo, lse_ptr, stream), "attention forward")
            fused = True
        except NotImplementedError:  # not an MFMA problem: rotate the queries separately
            q = _rope_rows(q, q_pos0, base, dim, False, query.device)
            vq = _view(q)
    if not fused:
        _lib.check(lib.tsattn_sdpa_forward(ctypes.byref(prob), vq, vk, vv, vo, lse_ptr, stream),
                   "attention forward")
    if not recording:
        return Tensor._from_op(out, (query, key, value), None, "sdpa_hip")

    def backward(upstream, _keep=keep):  # _keep: mask / length buffers the kernels read
        g = _operand(upstream)
        if (fused or code in (_lib.F16, _lib.BF16)) and (not _aligned16(g) or min(g.stride()[:3]) <= 0):
            # the MFMA kernels (the only ones the folded-RoPE backward has) need
            # 16-byte aligned rows of a real gradient: an expanded one (a sum's
            # VJP) would send the plain backward to the generic kernels
            g = g.contiguous()
        if g.dtype != out.dtype:
            g = g.to(out.dtype)
        dq = torch.empty(q.shape, dtype=q.dtype, device=tdev)
        dk = torch.empty(k.shape, dtype=k.dtype, device=tdev)
        dv = torch.empty(v.shape, dtype=v.dtype, device=tdev)
        nbytes = (lib.tsattn_sdpa_backward_rope_workspace if fused
                  else lib.tsattn_sdpa_backward_workspace)(ctypes.byref(prob))
        try:
            ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=tdev)
        except torch.OutOfMemoryError:
            # no room for the stored-dS region: the row values alone (plus
            # the rotated queries / drawn dropout bits the backward needs),
            # with which the kernels recompute S and dP for dQ instead
            nbytes = _rows_workspace(prob, fused, q.dtype)
            ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=tdev)
        args = (vq, vk, vv, vo, _view(g), ctypes.c_void_p(lse.data_ptr()), _view(dq), _view(dk),
                _view(dv), ctypes.c_void_p(ws.data_ptr()), nbytes,
                ctypes.c_void_p(current_stream(query.device)))
        if fused:  # gradients of the unrotated queries and keys, straight from the kernels
            _lib.check(lib.tsattn_sdpa_backward_rope(ctypes.byref(prob), ctypes.byref(rope[0]), *args),
                       "attention backward")
            return dq, dk, dv
        _lib.check(lib.tsattn_sdpa_backward(ctypes.byref(prob), *args), "attention backward")
        if rope is not None:  # rotary_embedding's VJP on the rotated operands
            dq = _rope_rows(dq, q_pos0, base, dim, True, query.device)
            if k_pos0 is not None:
                dk = _rope_rows(dk, k_pos0, base, dim, True, query.device)
        return dq, dk, dv

    return Tensor._from_op(out, (query, key, value), backward, "sdpa_hip")


def decode_int8_cache(query: Tensor, cache, *, is_causal: bool, causal_offset: int,
                      scale: float | None = None, rope: tuple | None = None) -> Tensor | None:
    """Inference attention of ``query`` [B, Hq, Q, D] against an int8
    ``KVCache``'s active prefix, dequantised inside the decode kernel
    (``tsattn_decode_forward_int8``).  Same result as the reference's
    ``scaled_dot_product_attention(query, *cache.get(), ...)`` (the cache
    dequantised eagerly, ``src/tensorsmith/nn/cache.py:88-99``) up to the
    rounding of the dequantised values to the cache dtype.  ``rope = (q_pos0,
    base)``: ``query`` is unrotated and the kernel rotates it
    (``tsattn_decode_forward_rope``), bit for bit ``rotary_embedding(query,
    q_pos0)``; the cached keys are rotated already.  Returns None when the
    shapes are outside the decode kernel (the caller then goes through
    ``cache.get()``, with ``query`` still unrotated)."""
    q = _operand(query._data)
    b, hq, qlen, dim = q.shape
    code = _dtype_code(q.dtype)
    hkv = cache.num_heads
    if (code not in (_lib.F16, _lib.BF16) or dim not in (64, 128, 256) or cache.value_dim != dim
            or cache.head_dim != dim or hq % hkv or (hq // hkv) * qlen > 8
            or cache.length < DECODE_MIN_KEYS or not _aligned16(q)
            or query.device != cache.device):
        return None
    import torch

    multiplier = 1 / math.sqrt(dim) if scale is None else scale
    prob = _problem(b, hq, hkv, qlen, cache.length, dim, dim, code, multiplier, is_causal,
                    causal_offset)
    keys, values, key_scales, value_scales = cache.storage
    out = torch.empty((b, hq, qlen, dim), dtype=q.dtype, device=q.device)
    lib = _lib.load()
    nbytes = lib.tsattn_decode_workspace(ctypes.byref(prob), 0)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    stream = ctypes.c_void_p(current_stream(query.device))
    args = (_view(keys), _view(values), _view(key_scales), _view(value_scales), _view(out), 0,
            ctypes.c_void_p(ws.data_ptr()), nbytes, stream)
    if rope is not None:
        q_pos0, base = rope
        tables = rope_tables(base, dim, q.dtype, q.device, q_pos0 + qlen)
        desc = _lib.RopeDesc()
        desc.cos, desc.sin = tables[0].data_ptr(), tables[1].data_ptr()
        desc.rotary_dim, desc.q_pos0, desc.k_pos0 = dim, q_pos0, 0
        try:
            _lib.check(lib.tsattn_decode_forward_rope(ctypes.byref(prob), ctypes.byref(desc),
                                                      _view(q), *args), "int8 decode forward")
            return Tensor._from_op(out, (query,), None, "sdpa_hip")
        except NotImplementedError:  # rotate the queries on their own
            q = _rope_rows(q, q_pos0, base, dim, False, query.device)
    _lib.check(lib.tsattn_decode_forward_int8(ctypes.byref(prob), _view(q), *args),
               "int8 decode forward")
    return Tensor._from_op(out, (query,), None, "sdpa_hip")


_ROPE_TABLES: dict = {}


def _ROPE_KERNEL_DTYPES():
    """Dtypes the RoPE kernels and the folded attention kernels take."""
    import torch

    return (torch.float32, torch.float16, torch.bfloat16)


def rope_tables(base: float, dim: int, dtype, dev, length: int):
    """Device (cos, sin) tables [L >= length, dim / 2] in ``dtype`` for
    positions 0 .. L - 1, built as the reference builds its per-call tables
    (``attention.py:269-279``: float32 angles, NumPy cos / sin, cast to the
    tensor dtype); an angle depends only on its absolute position, so one
    table serves every offset.  Grown on demand and kept per (base, dim,
    dtype, device)."""
    import torch

    key = (float(base), int(dim), str(dtype), str(dev))
    have = _ROPE_TABLES.get(key)
    if have is not None and have[0].shape[0] >= length:
        return have
    n = max(length, 2 * (have[0].shape[0] if have is not None else 0), 256)
    freqs = base ** (-(np.arange(0, dim, 2, dtype=np.float32)) / np.float32(dim))
    angles = np.arange(0, n, dtype=np.float32)[:, None] * freqs[None, :]
    made = tuple(torch.from_numpy(np.ascontiguousarray(f(angles))).to(device=dev, dtype=dtype)
                 for f in (np.cos, np.sin))
    _ROPE_TABLES[key] = made
    return made


def _rope_launch(x, out, offset: int, base: float, dim: int, inverse: bool, dev) -> None:
    b, h, t, d = x.shape
    cos, sin = rope_tables(base, dim, x.dtype, x.device, offset + t)
    _lib.check(
        _lib.load().tsattn_rope(
            _dtype_code(x.dtype), b, h, t, d, dim, ctypes.byref(_view(x)), ctypes.byref(_view(out)),
            ctypes.c_void_p(cos.data_ptr()), ctypes.c_void_p(sin.data_ptr()), offset, int(inverse),
            ctypes.c_void_p(current_stream(dev))),
        "RoPE")


def _rope_rows(x, offset: int, base: float, dim: int, inverse: bool, dev):
    """RoPE (or its inverse) of a raw [B, H, T, D] device array into a new one."""
    import torch

    src = x if x.stride(-1) == 1 else x.contiguous()
    out = torch.empty(src.shape, dtype=src.dtype, device=src.device)
    _rope_launch(src, out, offset, base, dim, inverse, dev)
    return out


def rotary_embedding(input: Tensor, offset: int = 0, base: float = 10000.0,
                     rotary_dim: int | None = None) -> Tensor:
    """Interleaved-pair RoPE for [..., sequence, channels] with inverse-rotation VJP.

    Same contract as the reference (``src/tensorsmith/nn/attention.py:255-296``):
    pairs (2i, 2i+1) rotate by angle ``pos * base**(-2i/dim)``, positions start
    at ``offset``, channels past ``rotary_dim`` pass through.  4-D f32 / f16 /
    bf16 inputs on the hip device run one kernel (``tsattn_rope``, bit-identical
    to the reference's array arithmetic), forward and VJP.
    """
    if input.ndim < 2:
        raise ValueError("RoPE requires at least sequence and channel dimensions")
    dim = input.shape[-1] if rotary_dim is None else rotary_dim
    if dim <= 0 or dim % 2 or dim > input.shape[-1] or offset < 0 or base <= 0 or not math.isfinite(base):
        raise ValueError("RoPE requires a positive even rotary dimension and valid positions/base")
    x = input._data
    import torch

    if (input.ndim == 4 and input.shape[-1] % 2 == 0 and input.device.type == "hip"
            and x.dtype in (torch.float32, torch.float16, torch.bfloat16)):
        src = x if x.stride(-1) == 1 else x.contiguous()
        out = torch.empty(src.shape, dtype=src.dtype, device=src.device)
        _rope_launch(src, out, offset, base, dim, False, input.device)

        def backward(g):
            g = g if g.stride(-1) == 1 else g.contiguous()
            dx = torch.empty(g.shape, dtype=g.dtype, device=g.device)
            _rope_launch(g, dx, offset, base, dim, True, input.device)
            return (dx,)

        return Tensor._from_op(out, (input,), backward, "rope")

    seq = input.shape[-2]
    freqs = base ** (-(np.arange(0, dim, 2, dtype=np.float32)) / np.float32(dim))
    angles = np.arange(offset, offset + seq, dtype=np.float32)[:, None] * freqs[None, :]
    cos = np.repeat(np.cos(angles), 2, axis=-1)
    sin = np.repeat(np.sin(angles), 2, axis=-1)
    cos_t = torch.from_numpy(cos).to(device=x.device, dtype=x.dtype)
    sin_t = torch.from_numpy(sin).to(device=x.device, dtype=x.dtype)

    def rotate(raw):
        pairs = raw.reshape(*raw.shape[:-1], dim // 2, 2)
        return torch.stack((-pairs[..., 1], pairs[..., 0]), dim=-1).reshape(raw.shape)

    part = x[..., :dim]
    result = part * cos_t + rotate(part) * sin_t
    if dim < input.shape[-1]:
        result = torch.cat((result, x[..., dim:]), dim=-1)

    def backward(g):
        front = g[..., :dim]
        dx = front * cos_t - rotate(front) * sin_t
        if dim < input.shape[-1]:
            dx = torch.cat((dx, g[..., dim:]), dim=-1)
        return (dx,)

    return Tensor._from_op(result, (input,), backward, "rope")
