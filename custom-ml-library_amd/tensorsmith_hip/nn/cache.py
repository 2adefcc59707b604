"""Preallocated KV cache on a hip device (reference ``src/tensorsmith/nn/cache.py``).

Same API, validation order and storage layout as the reference: keys and
values live in ``[B, H_kv, capacity, D]`` device arrays, ``append`` writes the
slice ``[:, :, length:length+T]`` after checking every shape and the
capacity, ``get`` returns views of the active prefix, and the optional int8
mode stores symmetric per-token/head codes with one fp32 scale each
(``scale = max(max|x| / 127, 1e-8)``, ``q = round(x / scale)``, ``:73-77``),
dequantised on ``get`` (``:91-98``).  The views ``get`` returns feed the decode
kernel directly (no copy: the kernel takes the cache's strides).

On the hip device an int8 append is one fused kernel
(``tsattn_kv_append_int8``: row max, scale, rounding and both writes), and
``MultiHeadAttention`` decodes over the int8 storage itself
(``tsattn_decode_forward_int8`` dequantises inside the kernel) instead of
going through ``get``.
"""

from __future__ import annotations

import math

import numpy as np

import ctypes

from .. import _lib
from ..device import current_stream
from .attention import _view
from ..device import device as parse_device
from ..tensor import Tensor, backend_dtype, is_grad_enabled, to_numpy


class KVCache:
    """Preallocated [B,H,capacity,D] keys/values for autoregressive inference."""

    def __init__(self, batch_size: int, num_heads: int, head_dim: int, max_seq_len: int, *,
                 device=None, dtype="float32", quantized: bool = False, value_dim=None):
        if min(batch_size, num_heads, head_dim, max_seq_len) <= 0:
            raise ValueError("cache dimensions and capacity must be positive")
        self.batch_size, self.num_heads, self.head_dim = batch_size, num_heads, head_dim
        self.value_dim = head_dim if value_dim is None else value_dim
        if self.value_dim <= 0:
            raise ValueError("value_dim must be positive")
        self.max_seq_len = max_seq_len
        self.device = parse_device(device)
        if self.device.type != "hip":
            raise RuntimeError("tensorsmith_hip keeps KV caches on hip devices")
        self.dtype = backend_dtype(dtype, self.device)
        if "float" not in str(self.dtype):
            raise TypeError("cache compute dtype must be floating point")
        self.quantized = quantized
        self.length = 0
        import torch

        dev = self.device.torch
        storage = torch.int8 if quantized else self.dtype
        shape = (batch_size, num_heads, max_seq_len)
        self._keys = torch.zeros(shape + (head_dim,), dtype=storage, device=dev)
        self._values = torch.zeros(shape + (self.value_dim,), dtype=storage, device=dev)
        self._key_scales = torch.ones(shape + (1,), dtype=torch.float32, device=dev) if quantized else None
        self._value_scales = (torch.ones(shape + (1,), dtype=torch.float32, device=dev)
                              if quantized else None)

    def append(self, key: Tensor, value: Tensor) -> tuple[Tensor, Tensor]:
        """Append a chunk after validating all shapes and capacity."""
        self._append(key, value)
        return self.get()

    def _append(self, key: Tensor, value: Tensor) -> None:
        """``append`` without building the returned views."""
        stop = self._check(key, value)
        window = slice(self.length, stop)
        keys, values = key._data.to(self.dtype), value._data.to(self.dtype)
        if self.quantized:
            _append_int8(keys, self._keys, self._key_scales, self.length, self.device)
            _append_int8(values, self._values, self._value_scales, self.length, self.device)
        else:
            self._keys[:, :, window] = keys
            self._values[:, :, window] = values
        self.length = stop

    def _append_rotary(self, key: Tensor, value: Tensor, base: float = 10000.0) -> bool:
        """Rotate ``key`` by RoPE at positions ``length ..`` and append it with
        ``value`` in one kernel (``tsattn_rope_append``).

        Same result as ``rotary_embedding(key, self.length)`` followed by
        ``_append``: the rotation runs in the key dtype, which must be the
        cache dtype here (else False is returned and nothing is written, so
        the caller takes the two-step path).  Needs an even head dim
        <= 512 equal to the value dim.
        """
        import torch

        if (key._data.dtype != self.dtype or value._data.dtype != self.dtype
                or self.dtype not in (torch.float32, torch.float16, torch.bfloat16)
                or self.head_dim % 2 or self.head_dim > 512 or self.value_dim != self.head_dim):
            return False
        stop = self._check(key, value)
        from .attention import rope_tables

        cos, sin = rope_tables(base, self.head_dim, self.dtype, self._keys.device, stop)
        k, v = key._data, value._data
        k = k if k.stride(-1) == 1 else k.contiguous()
        v = v if v.stride(-1) == 1 else v.contiguous()
        b, h, t, d = k.shape
        scales = ((ctypes.byref(_view(self._key_scales)), ctypes.byref(_view(self._value_scales)))
                  if self.quantized else (None, None))
        _lib.check(
            _lib.load().tsattn_rope_append(
                _CODES[str(k.dtype)], b, h, t, d, d, ctypes.byref(_view(k)), ctypes.byref(_view(v)),
                ctypes.byref(_view(self._keys)), ctypes.byref(_view(self._values)), *scales,
                ctypes.c_void_p(cos.data_ptr()), ctypes.c_void_p(sin.data_ptr()), self.length,
                ctypes.c_void_p(current_stream(self.device))),
            "RoPE cache append")
        self.length = stop
        return True

    def _project_append(self, input: Tensor, projections, num_heads: int, rotary: bool,
                        base: float = 10000.0):
        """The cached attention step's q / k / v projections (``projections``:
        the q, k, v ``Linear`` layers), RoPE of q and k at positions
        ``length ..`` and the k / v append, in one kernel
        (``tsattn_qkv_rope_append``).  Returns the rotated queries [B, H, T, D]
        (a device tensor) and advances ``length``; or None, writing nothing,
        when the operands are outside the kernel (16-bit input in the cache
        dtype and the layers' dtype, head dim 64 / 128 equal to the value dim,
        embed a multiple of 16): the caller then projects and appends in steps.
        """
        import torch

        x = input._data
        lin = [(layer.weight._data, None if layer.bias is None else layer.bias._data)
               for layer in projections]
        tensors = [t for pair in lin for t in pair if t is not None]
        if (x.dtype != self.dtype or self.dtype not in (torch.float16, torch.bfloat16)
                or self.head_dim not in (64, 128) or self.value_dim != self.head_dim
                or x.ndim != 3 or x.shape[0] != self.batch_size or x.shape[-1] % 16
                or x.stride(-1) != 1 or x.data_ptr() % 16 or x.stride(0) % 8 or x.stride(1) % 8
                or any(t.dtype != x.dtype or not t.is_contiguous() or t.data_ptr() % 16
                       for t in tensors)
                or lin[0][0].shape[0] != num_heads * self.head_dim
                or any(w.shape[0] != self.num_heads * self.head_dim for w, _ in lin[1:])):
            return None
        b, t, e = x.shape
        stop = self.length + t
        if t == 0 or stop > self.max_seq_len:
            raise ValueError(f"cache capacity {self.max_seq_len} exceeded or empty append")
        q = torch.empty((b, num_heads, t, self.head_dim), dtype=x.dtype, device=x.device)
        cos = sin = None
        if rotary:
            from .attention import rope_tables

            cos, sin = rope_tables(base, self.head_dim, self.dtype, self._keys.device, stop)
        ptr = lambda z: None if z is None else ctypes.c_void_p(z.data_ptr())
        scales = ((ctypes.byref(_view(self._key_scales)), ctypes.byref(_view(self._value_scales)))
                  if self.quantized else (None, None))
        code = _CODES[str(x.dtype)]
        _lib.check(
            _lib.load().tsattn_qkv_rope_append(
                code, b, t, e, num_heads, self.num_heads, self.head_dim, ctypes.byref(_view(x.unsqueeze(1))),
                *(ptr(w) for w, _ in lin), *(ptr(bias) for _, bias in lin), ctypes.byref(_view(q)),
                ctypes.byref(_view(self._keys)), ctypes.byref(_view(self._values)), *scales,
                ptr(cos), ptr(sin), self.length, ctypes.c_void_p(current_stream(self.device))),
            "fused projection, RoPE and cache append")
        self.length = stop
        return q

    def _check(self, key: Tensor, value: Tensor) -> int:
        """Validate an append (reference order, cache.py:54-70); return the new length."""
        if key.device != self.device or value.device != self.device:
            raise ValueError("cache and key/value tensors must be on the same device")
        if is_grad_enabled() and (key.requires_grad or value.requires_grad):
            raise RuntimeError("KVCache is inference-only; use no_grad() for differentiable inputs")
        prefix = (self.batch_size, self.num_heads)
        if key.ndim != 4 or key.shape[:2] != prefix or key.shape[-1] != self.head_dim:
            raise ValueError("key shape does not match cache configuration")
        if value.shape != key.shape[:3] + (self.value_dim,):
            raise ValueError("value shape does not match cache configuration")
        stop = self.length + key.shape[2]
        if key.shape[2] == 0 or stop > self.max_seq_len:
            raise ValueError(f"cache capacity {self.max_seq_len} exceeded or empty append")
        return stop

    def get(self) -> tuple[Tensor, Tensor]:
        keys = self._keys[:, :, : self.length]
        values = self._values[:, :, : self.length]
        if self.quantized:
            keys = (keys.float() * self._key_scales[:, :, : self.length]).to(self.dtype)
            values = (values.float() * self._value_scales[:, :, : self.length]).to(self.dtype)
        return Tensor(keys, device=self.device), Tensor(values, device=self.device)

    def reset(self) -> None:
        """Reuse the allocation; future appends overwrite old entries."""
        self.length = 0

    def truncate(self, length: int) -> None:
        if not 0 <= length <= self.length:
            raise ValueError("truncate length must be between zero and the current length")
        self.length = length

    def reorder(self, indices) -> None:
        """Reorder or duplicate batch rows for fixed-width beam search."""
        host = to_numpy(indices._data if isinstance(indices, Tensor) else indices)
        host = np.asarray(host)
        if host.shape != (self.batch_size,) or host.dtype.kind not in "iu":
            raise ValueError("beam indices must be one integer per cache batch row")
        if (host < 0).any() or (host >= self.batch_size).any():
            raise ValueError("beam index out of range")
        import torch

        order = torch.as_tensor(host.astype(np.int64), device=self._keys.device)
        self._keys, self._values = self._keys[order], self._values[order]
        if self.quantized:
            self._key_scales = self._key_scales[order]
            self._value_scales = self._value_scales[order]

    @property
    def storage(self) -> tuple:
        """Raw persistent arrays."""
        return self._keys, self._values, self._key_scales, self._value_scales

    @property
    def memory_bytes(self) -> int:
        """Allocated persistent payload, excluding temporary dequantised arrays."""
        arrays = [self._keys, self._values]
        if self.quantized:
            arrays += [self._key_scales, self._value_scales]
        return sum(math.prod(a.shape) * a.element_size() for a in arrays)

    def __len__(self):
        return self.length

    def __repr__(self):
        return (f"KVCache(length={self.length}, capacity={self.max_seq_len}, "
                f"quantized={self.quantized}, device='{self.device}')")


_CODES = {"torch.float32": _lib.F32, "torch.float16": _lib.F16, "torch.bfloat16": _lib.BF16}


def _append_int8(rows, codes, scales, pos: int, dev) -> None:
    """Quantise rows [B, H, T, D] (cache dtype) into codes[:, :, pos:pos+T] and
    scales[:, :, pos:pos+T] with the fused append kernel."""
    if rows.stride(-1) != 1:
        rows = rows.contiguous()
    b, h, t, d = rows.shape
    _lib.check(
        _lib.load().tsattn_kv_append_int8(
            _CODES[str(rows.dtype)], b, h, t, d, ctypes.byref(_view(rows)),
            ctypes.byref(_view(codes)), ctypes.byref(_view(scales)), pos,
            ctypes.c_void_p(current_stream(dev))),
        "int8 cache append")
