"""Tape ops around the attention path, on hip tensors.

Each op is one autograd node with the reference's semantics
(``src/tensorsmith/nn/functional.py`` and ``nn/primitives.py``); the array
math runs as PyTorch-ROCm library calls on the device tensors (GEMMs in
hipBLASLt).  Only attention itself has hand-written HIP kernels.
"""

from __future__ import annotations

import math

from ..amp import _cast_inputs
from ..device import random_uniform
from ..tensor import Tensor, _sum_to_shape, is_torch
from .attention import rotary_embedding, scaled_dot_product_attention

__all__ = [
    "cross_entropy", "dropout", "embedding", "gelu", "layer_norm", "linear", "rms_norm",
    "rotary_embedding", "scaled_dot_product_attention", "silu",
]


def _require_hip(t: Tensor, op: str):
    if not is_torch(t._data):
        raise RuntimeError(f"{op}: tensorsmith_hip computes on hip devices only")


def _compute(raw):
    """Half inputs compute in float32 (reference ``primitives.py:16-18``)."""
    import torch

    return raw.float() if raw.dtype in (torch.float16, torch.bfloat16) else raw


def linear(input: Tensor, weight: Tensor, bias: Tensor | None = None) -> Tensor:
    """x @ W^T + b as one node (reference ``functional.py:63-90``), autocast-aware."""
    input, weight, bias = _cast_inputs(input, weight, bias)
    if input.ndim < 1 or weight.ndim != 2 or input.shape[-1] != weight.shape[1]:
        raise ValueError("linear expects [...,in_features] and [out_features,in_features]")
    parents = (input, weight) if bias is None else (input, weight, bias)
    if any(p.device != input.device for p in parents):
        raise ValueError("linear tensors must be on the same device")
    if bias is not None and bias.shape != (weight.shape[0],):
        raise ValueError("linear bias must have shape [out_features]")
    _require_hip(input, "linear")
    w = weight._data
    x = input._data.reshape(-1, weight.shape[1])
    out = x @ w.t()
    if bias is not None:
        out = out + bias._data.to(out.dtype)
    out = out.reshape(input.shape[:-1] + (weight.shape[0],))

    def backward(g):
        flat = g.reshape(-1, weight.shape[0])
        grads = [(flat @ w).reshape(input.shape).to(input.dtype), (flat.t() @ x).to(weight.dtype)]
        if bias is not None:
            grads.append(flat.sum(0).to(bias.dtype))
        return tuple(grads)

    return Tensor._from_op(out, parents, backward, "linear")


def gelu(input: Tensor) -> Tensor:
    """Tanh-approximate GELU (reference ``primitives.py:21-49``)."""
    _require_hip(input, "gelu")
    import torch

    x = _compute(input._data)
    factor = math.sqrt(2 / math.pi)
    tangent = torch.tanh(factor * (x + 0.044715 * x**3))
    out = (0.5 * x * (1 + tangent)).to(input.dtype)

    def backward(g):
        d = 0.5 * (1 + tangent) + 0.5 * x * (1 - tangent**2) * factor * (1 + 3 * 0.044715 * x**2)
        return ((g * d).to(input.dtype),)

    return Tensor._from_op(out, (input,), backward, "bias_gelu")


def _norm(input: Tensor, weight: Tensor, bias: Tensor | None, eps: float, rms: bool) -> Tensor:
    """Layer / RMS norm over the trailing ``weight.ndim`` dims (reference
    ``primitives.py:67-136``): half inputs compute in float32, the VJP uses
    the saved normalised values and reciprocal std."""
    if eps <= 0 or not math.isfinite(eps):
        raise ValueError("eps must be positive")
    if input.shape[-weight.ndim:] != weight.shape:
        raise ValueError("normalization weight must match the trailing input dimensions")
    if bias is not None and bias.shape != weight.shape:
        raise ValueError("normalization bias and weight must have equal shapes")
    parents = (input, weight) if bias is None else (input, weight, bias)
    if any(p.device != input.device for p in parents):
        raise ValueError("normalization tensors must be on the same device")
    _require_hip(input, "rms_norm" if rms else "layer_norm")
    axes = tuple(range(input.ndim - weight.ndim, input.ndim))
    x = _compute(input._data)
    w = weight._data.to(x.dtype)
    centered = x if rms else x - x.mean(dim=axes, keepdim=True)
    rstd = 1 / (centered.square().mean(dim=axes, keepdim=True) + eps).sqrt()
    normalized = centered * rstd
    out = normalized * w
    if bias is not None:
        out = out + bias._data.to(x.dtype)
    out = out.to(input.dtype)

    def backward(g):
        g = g.to(x.dtype)
        weighted = g * w
        dx = rstd * (weighted - normalized * (weighted * normalized).mean(dim=axes, keepdim=True))
        if not rms:
            dx = dx - rstd * weighted.mean(dim=axes, keepdim=True)
        grads = [dx.to(input.dtype), _sum_to_shape(g * normalized, weight.shape).to(weight.dtype)]
        if bias is not None:
            grads.append(_sum_to_shape(g, bias.shape).to(bias.dtype))
        return tuple(grads)

    return Tensor._from_op(out, parents, backward, "rms_norm" if rms else "layer_norm")


def layer_norm(input: Tensor, weight: Tensor, bias: Tensor | None = None, eps: float = 1e-5) -> Tensor:
    """Layer norm (reference ``primitives.py:134-135``)."""
    return _norm(input, weight, bias, eps, False)


def rms_norm(input: Tensor, weight: Tensor, eps: float = 1e-6) -> Tensor:
    """RMS norm, ``x / sqrt(mean(x^2) + eps) * weight`` (reference ``primitives.py:138-139``)."""
    return _norm(input, weight, None, eps, True)


def silu(input: Tensor) -> Tensor:
    """``x * sigmoid(x)`` in float32 for half inputs (reference ``primitives.py:52-64``)."""
    _require_hip(input, "silu")
    import torch

    x = _compute(input._data)
    sig = torch.sigmoid(x)
    out = (x * sig).to(input.dtype)

    def backward(g):
        return ((g.to(x.dtype) * (sig + x * sig * (1 - sig))).to(input.dtype),)

    return Tensor._from_op(out, (input,), backward, "silu")


def embedding(indices: Tensor, weight: Tensor) -> Tensor:
    """Row gather with scatter-add VJP (reference ``functional.py:130-142``)."""
    if indices.requires_grad:
        raise ValueError("embedding indices cannot require gradients")
    if indices.device != weight.device:
        raise ValueError("indices and embedding weight must be on the same device")
    _require_hip(weight, "embedding")
    idx = indices._data.long()
    out = weight._data[idx]

    def backward(g):
        import torch

        grad = torch.zeros_like(weight._data)
        grad.index_add_(0, idx.reshape(-1), g.reshape(-1, weight.shape[-1]).to(grad.dtype))
        return (grad,)

    return Tensor._from_op(out, (weight,), backward, "embedding")


def dropout(input: Tensor, p: float = 0.5, training: bool = True) -> Tensor:
    """Inverted dropout (reference ``functional.py:121-127``); identity when off."""
    if not 0 <= p < 1:
        raise ValueError("dropout probability must be in [0, 1)")
    if not training or p == 0:
        return input
    _require_hip(input, "dropout")
    mask = (random_uniform(input.shape, input.device) >= p).to(input.dtype) / (1 - p)
    return Tensor._from_op(input._data * mask, (input,), lambda g: (g * mask,), "dropout")


def cross_entropy(input: Tensor, target: Tensor, reduction: str = "mean", *, axis: int = 1,
                  ignore_index: int = -100, label_smoothing: float = 0.0) -> Tensor:
    """Indexed cross-entropy (reference ``functional.py:397-472``)."""
    if input.ndim < 2:
        raise ValueError("cross_entropy expects logits with at least two dimensions")
    if input.device != target.device or "float" not in str(input.dtype):
        raise ValueError("cross_entropy needs floating logits and targets on the same device")
    if not 0 <= label_smoothing <= 1:
        raise ValueError("label_smoothing must be in [0, 1]")
    if reduction not in {"mean", "sum", "none"}:
        raise ValueError("reduction must be 'none', 'mean', or 'sum'")
    if target.requires_grad:
        raise ValueError("class targets cannot require gradients")
    if "int" not in str(target.dtype):
        raise TypeError("class targets must have an integer dtype")
    if not -input.ndim <= axis < input.ndim:
        raise ValueError("class axis is out of range")
    _require_hip(input, "cross_entropy")
    import torch

    axis %= input.ndim
    classes = input.shape[axis]
    expected = input.shape[:axis] + input.shape[axis + 1:]
    labels = target._data
    if tuple(labels.shape) != expected:
        raise ValueError(f"target shape {tuple(labels.shape)} does not match logits shape {input.shape}")
    valid = labels != ignore_index
    if bool((((labels < 0) | (labels >= classes)) & valid).any()):
        raise ValueError("target class index is out of range")
    perm = tuple(i for i in range(input.ndim) if i != axis) + (axis,)
    inverse = tuple(perm.index(i) for i in range(input.ndim))
    logits = _compute(input._data.permute(*perm).reshape(-1, classes))
    index = torch.where(valid, labels, torch.zeros_like(labels)).reshape(-1).long()
    active = valid.reshape(-1)
    log_probs = torch.log_softmax(logits, dim=-1)
    losses = -(1 - label_smoothing) * log_probs.gather(1, index[:, None])[:, 0]
    if label_smoothing:
        losses = losses - label_smoothing * log_probs.mean(dim=-1)
    losses = torch.where(active, losses, torch.zeros_like(losses))
    count = max(int(valid.sum()), 1)
    out = losses.reshape(expected) if reduction == "none" else losses.sum() / (
        count if reduction == "mean" else 1)

    def backward(g):
        grad = log_probs.exp() - label_smoothing / classes
        grad.scatter_add_(1, index[:, None], torch.full_like(grad[:, :1], -(1 - label_smoothing)))
        grad = torch.where(active[:, None], grad, torch.zeros_like(grad))
        grad = grad * (g.reshape(-1, 1) if reduction == "none"
                       else g / (count if reduction == "mean" else 1))
        return (grad.reshape(expected + (classes,)).permute(*inverse).to(input.dtype),)

    return Tensor._from_op(out, (input,), backward, "cross_entropy")
