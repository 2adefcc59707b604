"""Round-to-nearest-even helpers for bf16 / fp16 in NumPy (test infrastructure).

NumPy has no bfloat16 dtype, so bf16 values are carried as float32 arrays
whose every element is exactly representable in bf16.  The reference promotes
half inputs to float32 for compute and casts results back to the input dtype
(``src/tensorsmith/nn/attention.py:63,90-92,248,250-251``); these helpers
perform those casts bit-exactly.  Pinned against ``torch.Tensor.to`` in
``tests/test_oracle.py``.
"""

from __future__ import annotations

import numpy as np

HALF_DTYPES = ("float16", "bfloat16")


def bf16_round(x) -> np.ndarray:
    """float32 -> nearest bf16 value (ties to even), returned as float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = x.view(np.uint32).astype(np.uint64)
    lsb = (bits >> 16) & 1
    rounded = ((bits + 0x7FFF + lsb) & 0xFFFF0000).astype(np.uint32)
    nan = np.isnan(x)
    if nan.any():
        rounded = np.where(nan, (x.view(np.uint32) | 0x00400000) & 0xFFFF0000, rounded)
    return rounded.astype(np.uint32).view(np.float32).reshape(x.shape)


def bf16_bits(x) -> np.ndarray:
    """float32 array of bf16 values -> uint16 storage bits."""
    x = np.ascontiguousarray(bf16_round(x), dtype=np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(bits) -> np.ndarray:
    """uint16 bf16 storage bits -> float32 values."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    return (bits.astype(np.uint32) << 16).view(np.float32)


def round_to(x, dtype: str) -> np.ndarray:
    """Round a float array to ``dtype`` and return it in the compute dtype.

    float16/bfloat16 come back as float32 holding exactly-representable
    values; float32/float64 are plain casts.
    """
    if dtype == "bfloat16":
        return bf16_round(np.asarray(x, dtype=np.float32))
    if dtype == "float16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
    if dtype == "float32":
        return np.asarray(x, dtype=np.float32)
    if dtype == "float64":
        return np.asarray(x, dtype=np.float64)
    raise ValueError(f"unsupported dtype {dtype!r}")


def compute_dtype(dtype: str):
    """The reference computes half inputs in float32 (``attention.py:63``)."""
    return np.float64 if dtype == "float64" else np.float32
