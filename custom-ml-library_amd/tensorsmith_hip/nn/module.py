"""Module / Parameter registry for the layers around the attention path.

Same names and behaviour as the reference's ``src/tensorsmith/nn/module.py``
(parameters discovered from attributes, ``train``/``eval`` propagate to
sub-modules, ``state_dict`` / ``load_state_dict`` round-trip host arrays), so
``MultiHeadAttention`` and checkpoints written by the reference load here.
Hooks are not provided (not on the attention path).
"""

from __future__ import annotations

from collections import OrderedDict
from collections.abc import Iterator, Mapping
from typing import Any

import numpy as np

from ..device import device as parse_device
from ..tensor import Tensor, to_backend, to_numpy


class Parameter(Tensor):
    """A trainable tensor discovered automatically by :class:`Module`."""

    def __init__(self, data: Any, requires_grad: bool = True, **kwargs: Any) -> None:
        super().__init__(data, requires_grad=requires_grad, **kwargs)


def _walk(value: Any, prefix: str, seen: set[int]):
    if isinstance(value, Parameter):
        if id(value) not in seen:
            seen.add(id(value))
            yield prefix, value
    elif isinstance(value, Module):
        yield from value.named_parameters(prefix, seen)
    elif isinstance(value, (list, tuple)):
        for index, item in enumerate(value):
            yield from _walk(item, f"{prefix}.{index}" if prefix else str(index), seen)


class Module:
    """Base class for stateful neural-network components."""

    def __init__(self) -> None:
        self.training = True

    def forward(self, *args: Any, **kwargs: Any):
        raise NotImplementedError

    def __call__(self, *args: Any, **kwargs: Any):
        return self.forward(*args, **kwargs)

    def named_parameters(self, prefix: str = "", seen: set[int] | None = None):
        seen = set() if seen is None else seen
        for name, value in vars(self).items():
            if name.startswith("_") or name == "training":
                continue
            yield from _walk(value, f"{prefix}.{name}" if prefix else name, seen)

    def parameters(self) -> Iterator[Parameter]:
        for _, p in self.named_parameters():
            yield p

    def modules(self) -> Iterator[Module]:
        yield self
        for value in vars(self).values():
            items = value if isinstance(value, (list, tuple)) else (value,)
            for item in items:
                if isinstance(item, Module):
                    yield from item.modules()

    def train(self, mode: bool = True) -> Module:
        for m in self.modules():
            m.training = mode
        return self

    def eval(self) -> Module:
        return self.train(False)

    def zero_grad(self) -> None:
        for p in self.parameters():
            p.zero_grad()

    def to(self, target=None, dtype=None) -> Module:
        dev = None if target is None else parse_device(target)
        for p in self.parameters():
            p._data = to_backend(p._data, dev or p.device, dtype)
            if dev is not None:
                p.device = dev
        return self

    def state_dict(self) -> OrderedDict[str, np.ndarray]:
        return OrderedDict((name, to_numpy(p._data).copy()) for name, p in self.named_parameters())

    def load_state_dict(self, state: Mapping[str, Any], strict: bool = True) -> None:
        params = dict(self.named_parameters())
        missing = sorted(set(params) - set(state))
        unexpected = sorted(set(state) - set(params))
        if strict and (missing or unexpected):
            raise KeyError(f"state_dict mismatch: missing={missing}, unexpected={unexpected}")
        for name, p in params.items():
            if name not in state:
                continue
            value = np.asarray(state[name])
            if tuple(value.shape) != p.shape:
                raise ValueError(f"shape mismatch for {name}: {value.shape} vs {p.shape}")
            p._data = to_backend(value, p.device, p.dtype)
