"""Layers used by the attention path's callers (reference ``nn/layers.py``).

Initialisation follows the reference (``Linear``: U(-1/sqrt(in), 1/sqrt(in))
from the host RNG; ``Embedding``: N(0, 1); ``LayerNorm``: ones / zeros) so
seeded models match parameter for parameter.
"""

from __future__ import annotations

import math
from collections.abc import Sequence

import numpy as np

from ..tensor import Tensor
from . import functional as F
from .module import Module, Parameter


def _uniform(shape, bound, device):
    return Tensor(np.random.uniform(-bound, bound, shape).astype(np.float32), device=device)


class Linear(Module):
    def __init__(self, in_features: int, out_features: int, bias: bool = True, device=None):
        super().__init__()
        self.in_features, self.out_features = in_features, out_features
        bound = 1 / math.sqrt(in_features)
        self.weight = Parameter(_uniform((out_features, in_features), bound, device))
        self.bias = Parameter(_uniform((out_features,), bound, device)) if bias else None

    def forward(self, input: Tensor) -> Tensor:
        return F.linear(input, self.weight, self.bias)


class Embedding(Module):
    def __init__(self, num_embeddings: int, embedding_dim: int, device=None):
        super().__init__()
        self.num_embeddings, self.embedding_dim = num_embeddings, embedding_dim
        values = np.random.normal(0, 1, (num_embeddings, embedding_dim)).astype(np.float32)
        self.weight = Parameter(Tensor(values, device=device))

    def forward(self, indices: Tensor) -> Tensor:
        return F.embedding(indices, self.weight)


class LayerNorm(Module):
    def __init__(self, normalized_shape: int | Sequence[int], eps: float = 1e-5, device=None):
        super().__init__()
        self.normalized_shape = (
            (normalized_shape,) if isinstance(normalized_shape, int) else tuple(normalized_shape))
        self.eps = eps
        self.weight = Parameter(Tensor(np.ones(self.normalized_shape, np.float32), device=device))
        self.bias = Parameter(Tensor(np.zeros(self.normalized_shape, np.float32), device=device))

    def forward(self, input: Tensor) -> Tensor:
        if input.shape[-len(self.normalized_shape):] != self.normalized_shape:
            raise ValueError("input's trailing shape does not match normalized_shape")
        return F.layer_norm(input, self.weight, self.bias, self.eps)


class GELU(Module):
    def forward(self, input: Tensor) -> Tensor:
        return F.gelu(input)


class Dropout(Module):
    def __init__(self, p: float = 0.5):
        super().__init__()
        self.p = p

    def forward(self, input: Tensor) -> Tensor:
        return F.dropout(input, self.p, self.training)
