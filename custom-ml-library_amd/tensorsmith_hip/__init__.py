"""tensorsmith_hip -- tensorsmith's attention hot path on MI355X (gfx950).

A ``hip`` backend for the reference's ``scaled_dot_product_attention`` /
``KVCache`` / ``MultiHeadAttention`` API.  Attention runs in the hand-written
HIP kernels of ``libtsattn.so`` (C ABI: ``include/tsattn.h``), loaded through
ctypes; PyTorch-ROCm supplies device memory and streams.
"""

from . import nn
from .amp import autocast
from .device import Device, available_devices, device, is_available, seed, synchronize
from .tensor import Tensor, cat, enable_grad, grad, is_grad_enabled, no_grad, randn, tensor, zeros

__version__ = "0.1.0"

__all__ = [
    "Device", "Tensor", "autocast", "available_devices", "cat", "device", "enable_grad", "grad",
    "is_available", "is_grad_enabled", "nn", "no_grad", "randn", "seed", "synchronize", "tensor",
    "zeros",
]
