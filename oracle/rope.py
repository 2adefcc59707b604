"""NumPy restatement of tensorsmith's rotary position embedding -- TEST
INFRASTRUCTURE.

Follows ``rotary_embedding`` (``src/tensorsmith/nn/attention.py:255-296``):
interleaved channel pairs (2i, 2i+1), i < rotary_dim / 2, rotate by the angle
p * base^(-2i / rotary_dim) for row position p = offset + t; the angle table
is built in float32 and its cosines / sines are cast to the tensor dtype
(``:269-279``); the rotation is ``part * cos + rotate(part) * sin`` with
``rotate`` = (-x_{2i+1}, x_{2i}) (``:281-285``), every product and sum rounded
to the tensor dtype as NumPy's array arithmetic rounds it; the VJP rotates by
the negative angle (``:289-294``); channels from rotary_dim on pass through.

Half values are carried as float32 arrays holding exactly-representable
values (``oracle.halfprec``).  Only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg may import this module.
"""

from __future__ import annotations

import numpy as np

from .halfprec import round_to


def tables(length: int, rotary_dim: int, base: float = 10000.0, offset: int = 0):
    """float32 (cos, sin), shape [length, rotary_dim / 2], for positions
    offset .. offset + length - 1 (``attention.py:269-274``)."""
    freqs = base ** (-np.arange(0, rotary_dim, 2).astype(np.float32) / rotary_dim)
    angles = np.arange(offset, offset + length).astype(np.float32)[:, None] * freqs[None, :]
    return np.cos(angles), np.sin(angles)


def rope(x, offset: int = 0, base: float = 10000.0, rotary_dim: int | None = None,
         dtype: str = "float32", inverse: bool = False):
    """RoPE of x [..., S, D] (values already in ``dtype``), rounded per
    operation in ``dtype``; ``inverse`` gives the VJP's rotation.  float64
    inputs stay float64 (the float32 tables cast up, as the reference casts
    them to the input dtype)."""
    x = np.asarray(x, np.float64 if dtype == "float64" else np.float32)
    seq, d = x.shape[-2], x.shape[-1]
    dim = d if rotary_dim is None else rotary_dim
    if dim <= 0 or dim % 2 or dim > d or offset < 0 or base <= 0:
        raise ValueError("RoPE requires a positive even rotary dimension and valid positions/base")
    cos_h, sin_h = tables(seq, dim, base, offset)
    cos = round_to(np.repeat(cos_h, 2, axis=-1), dtype)
    sin = round_to(np.repeat(sin_h, 2, axis=-1), dtype)
    if inverse:
        sin = -sin
    part = x[..., :dim]
    rotated = np.stack((-part[..., 1::2], part[..., 0::2]), axis=-1).reshape(part.shape)
    out = round_to(round_to(part * cos, dtype) + round_to(rotated * sin, dtype), dtype)
    if dim < d:
        out = np.concatenate((out, x[..., dim:]), axis=-1)
    return out
