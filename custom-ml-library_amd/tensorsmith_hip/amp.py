"""Operator-scoped fp16 autocast, the policy of the reference's ``amp.py:17-74``.

Inside ``autocast(device_type, dtype="float16")`` the float32 inputs of
matmul / linear are cast to float16 (float64 untouched); attention then
receives float16 q/k/v, computes in fp32 and returns float16 -- on ``hip``
that is the MFMA path.
"""

from __future__ import annotations

from contextlib import ContextDecorator
from contextvars import ContextVar

import numpy as np

from .device import device as parse_device

_autocast = ContextVar("tensorsmith_hip_autocast", default=None)


class autocast(ContextDecorator):
    """Cast FP32 matmul/linear inputs to FP16 in this context (thread/task local)."""

    def __init__(self, device_type="hip", *, dtype="float16", enabled=True):
        self.device_type = parse_device(device_type).type
        try:
            self.dtype = np.dtype(dtype).name
        except TypeError as error:
            raise ValueError("autocast currently supports dtype='float16' only") from error
        if self.dtype != "float16":
            raise ValueError("autocast currently supports dtype='float16' only")
        self.enabled = bool(enabled)
        self._tokens = []

    def __enter__(self):
        state = dict(_autocast.get() or {})
        state[self.device_type] = (self.enabled, self.dtype)
        self._tokens.append(_autocast.set(state))
        return self

    def __exit__(self, *exc):
        _autocast.reset(self._tokens.pop())
        return False


def is_autocast_enabled(device_type="hip") -> bool:
    entry = (_autocast.get() or {}).get(parse_device(device_type).type)
    return bool(entry and entry[0])


def _cast_inputs(*values):
    """Autocast rule of the reference (``amp.py:61-74``)."""
    tensors = [v for v in values if v is not None]
    if not tensors:
        return values
    dev = tensors[0].device
    entry = (_autocast.get() or {}).get(dev.type)
    if not entry or not entry[0] or any(v.device != dev for v in tensors):
        return values
    names = [str(v.dtype).split(".")[-1] for v in tensors]
    if any(n not in {"float16", "float32"} for n in names):
        return values
    return tuple(
        v.astype(entry[1]) if v is not None and str(v.dtype).split(".")[-1] == "float32" else v
        for v in values
    )
