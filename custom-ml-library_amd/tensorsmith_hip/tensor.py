"""Tensor and reverse-mode autograd, the contract the attention op plugs into.

Mirrors the reference's node contract and VJP engine:

* ``Tensor._from_op(data, parents, backward, op)`` records a tape node iff
  grad mode is on and any parent requires grad
  (``src/tensorsmith/tensor.py:121-135``);
* ``_run_backward`` topologically sorts the tape, casts each contribution to
  the node's dtype before calling its VJP, sums branch contributions and
  frees the tape unless ``retain_graph`` (``tensor.py:662-724``);
* ``no_grad`` / ``enable_grad`` are ContextVar-scoped (``tensor.py:19-44``).

Host tensors hold NumPy arrays; ``hip`` tensors hold PyTorch-ROCm device
tensors (memory and streams only).  Only the operators the attention path,
its callers and its tests use are provided.
"""

from __future__ import annotations

import math
from collections.abc import Callable, Sequence
from contextlib import ContextDecorator
from contextvars import ContextVar
from typing import Any

import numpy as np

from .device import Device, DeviceLike, require_available
from .device import device as parse_device

_grad_enabled: ContextVar[bool] = ContextVar("tensorsmith_hip_grad_enabled", default=True)


class no_grad(ContextDecorator):
    """Disable graph recording within a block (thread/task local)."""

    def __enter__(self):
        self._token = _grad_enabled.set(False)
        return self

    def __exit__(self, *exc):
        _grad_enabled.reset(self._token)
        return False


class enable_grad(ContextDecorator):
    def __enter__(self):
        self._token = _grad_enabled.set(True)
        return self

    def __exit__(self, *exc):
        _grad_enabled.reset(self._token)
        return False


def is_grad_enabled() -> bool:
    return _grad_enabled.get()


# ---------------------------------------------------------------------------
# Raw-array helpers: NumPy on cpu, torch on hip.
# ---------------------------------------------------------------------------

_TORCH_DTYPES = {
    "float32": "float32", "float": "float32", "float16": "float16", "half": "float16",
    "bfloat16": "bfloat16", "float64": "float64", "double": "float64", "int64": "int64",
    "long": "int64", "int32": "int32", "int8": "int8", "uint8": "uint8", "bool": "bool",
}


def _torch():
    import torch

    return torch


def is_torch(x) -> bool:
    return type(x).__module__.startswith("torch")


def dtype_name(dtype) -> str:
    """Portable name ('float32', 'bfloat16', ...) of a NumPy/torch dtype or string."""
    if dtype is None:
        return ""
    text = str(dtype).split(".")[-1]
    return _TORCH_DTYPES.get(text, text)


def backend_dtype(dtype, dev: Device):
    if dtype is None:
        return None
    name = dtype_name(dtype)
    if dev.type == "hip":
        return getattr(_torch(), name)
    if name == "bfloat16":
        raise TypeError("bfloat16 host arrays are not supported; use a hip device")
    return np.dtype(name)


def is_float_dtype(dtype) -> bool:
    return "float" in str(dtype)


def to_backend(data, dev: Device, dtype=None):
    """Raw array of ``data`` on ``dev`` (copying across devices only)."""
    if isinstance(data, Tensor):
        data = data._data
    if dev.type == "hip":
        torch = _torch()
        require_available(dev)
        tdt = backend_dtype(dtype, dev)
        if is_torch(data):
            return data.to(device=dev.torch, dtype=tdt or data.dtype)
        host = np.asarray(data)
        if tdt is None and host.dtype == np.float64 and not isinstance(data, np.ndarray):
            tdt = torch.float32
        out = torch.from_numpy(np.ascontiguousarray(host)).to(dev.torch)
        return out if tdt is None else out.to(tdt)
    if is_torch(data):
        data = to_numpy(data)
    return np.asarray(data, dtype=backend_dtype(dtype, dev))


def to_numpy(data) -> np.ndarray:
    if isinstance(data, np.ndarray):
        return data
    if is_torch(data):
        torch = _torch()
        t = data.detach()
        if t.dtype == torch.bfloat16:
            t = t.float()  # NumPy has no bfloat16: values are exact in float32
        return t.cpu().numpy()
    return np.asarray(data)


def _cast(x, dtype):
    if is_torch(x):
        return x.to(dtype)
    return x.astype(dtype)


def _sum(x, axis=None, keepdims=False):
    if is_torch(x):
        if axis is None:
            r = x.sum()
            return r.reshape([1] * x.ndim) if keepdims else r
        return x.sum(dim=axis, keepdim=keepdims)
    return np.sum(x, axis=axis, keepdims=keepdims)


def _sum_to_shape(grad, shape):
    """Reverse broadcasting by summing broadcast dimensions."""
    while grad.ndim > len(shape):
        grad = _sum(grad, 0)
    axes = tuple(i for i, (g, s) in enumerate(zip(grad.shape, shape)) if s == 1 and g != 1)
    if axes:
        grad = _sum(grad, axes, keepdims=True)
    return grad


def _permute(x, axes):
    return x.permute(*axes) if is_torch(x) else np.transpose(x, axes)


def _ones_like(x):
    return _torch().ones_like(x) if is_torch(x) else np.ones_like(x)


def _zeros_like(x):
    return _torch().zeros_like(x) if is_torch(x) else np.zeros_like(x)


def _raw(value, like):
    """A Python scalar / Tensor operand as a raw array compatible with ``like``."""
    if isinstance(value, Tensor):
        return value._data
    if is_torch(like):
        return value  # torch promotes Python scalars without changing dtype
    return np.asarray(value, dtype=like.dtype) if isinstance(value, (int, float)) else value


Backward = Callable[[Any], tuple[Any | None, ...]]


class Tensor:
    """An n-dimensional array that can participate in a dynamic autograd graph."""

    __array_priority__ = 1000

    def __init__(self, data: Any, *, requires_grad: bool = False, device: DeviceLike = None,
                 dtype: Any = None, _copy: bool = False) -> None:
        if isinstance(data, Tensor):
            target = data.device if device is None else parse_device(device)
            raw = to_backend(data._data, target, dtype)
            if _copy or raw is data._data:
                raw = raw.clone() if is_torch(raw) else raw.copy()
        else:
            target = parse_device(device)
            if dtype is None and not hasattr(data, "dtype"):
                kind = np.asarray(data).dtype.kind
                dtype = "float32" if kind == "f" else ("int64" if kind in "iu" else None)
            raw = to_backend(data, target, dtype)
        if requires_grad and not is_float_dtype(raw.dtype):
            raise TypeError("only floating-point tensors can require gradients")
        self._data = raw
        self.requires_grad = bool(requires_grad)
        self.device = target
        self._grad = None
        self._parents: tuple[Tensor, ...] = ()
        self._backward: Backward | None = None
        self._op = ""
        self._graph_freed = False

    @classmethod
    def _from_op(cls, data: Any, parents: tuple[Tensor, ...], backward: Backward, op: str) -> Tensor:
        obj = cls.__new__(cls)
        obj._data = data
        obj.device = parents[0].device
        obj.requires_grad = is_grad_enabled() and any(p.requires_grad for p in parents)
        obj._grad = None
        obj._parents = parents if obj.requires_grad else ()
        obj._backward = backward if obj.requires_grad else None
        obj._op = op if obj.requires_grad else ""
        obj._graph_freed = False
        return obj

    # -- properties --------------------------------------------------------
    @property
    def shape(self) -> tuple[int, ...]:
        return tuple(self._data.shape)

    @property
    def ndim(self) -> int:
        return len(self._data.shape)

    @property
    def dtype(self):
        return self._data.dtype

    @property
    def size(self) -> int:
        return int(math.prod(self.shape))

    @property
    def grad(self) -> Tensor | None:
        return None if self._grad is None else Tensor(self._grad, device=self.device)

    @grad.setter
    def grad(self, value) -> None:
        self._grad = None if value is None else to_backend(value, self.device)

    def numpy(self) -> np.ndarray:
        return to_numpy(self._data)

    def item(self):
        return self.numpy().item()

    def __len__(self) -> int:
        return self.shape[0]

    def __repr__(self) -> str:
        suffix = f", device='{self.device}'" if self.device.type != "cpu" else ""
        return f"Tensor(shape={self.shape}, dtype={dtype_name(self.dtype)}{suffix})"

    # -- autograd -----------------------------------------------------------
    def backward(self, gradient=None, retain_graph: bool = False) -> None:
        if not self.requires_grad:
            raise RuntimeError("backward() called on a tensor that does not require grad")
        if gradient is None:
            if self.size != 1:
                raise RuntimeError("backward() needs a gradient for a non-scalar output")
            seed = _ones_like(self._data)
        else:
            seed = to_backend(gradient, self.device)
            if tuple(seed.shape) != self.shape:
                raise ValueError("upstream gradient shape mismatch")
        _run_backward(self, seed, retain_graph=retain_graph, accumulate=True)

    def zero_grad(self) -> None:
        self._grad = None

    def detach(self) -> Tensor:
        return Tensor(self._data, device=self.device)

    def requires_grad_(self, flag: bool = True) -> Tensor:
        if flag and not is_float_dtype(self.dtype):
            raise TypeError("only floating-point tensors can require gradients")
        self.requires_grad = flag
        return self

    # -- elementwise ---------------------------------------------------------
    def astype(self, dtype) -> Tensor:
        target = backend_dtype(dtype, self.device)
        source = self.dtype
        data = _cast(self._data, target)
        return Tensor._from_op(data, (self,), lambda g: (_cast(g, source),), "astype")

    def to(self, device=None, dtype=None) -> Tensor:
        if device is not None and parse_device(device) != self.device:
            return Tensor(self, device=device, dtype=dtype)
        return self if dtype is None else self.astype(dtype)

    def _binary(self, other, fn, vjp, op):
        other_t = other if isinstance(other, Tensor) else None
        a, b = self._data, _raw(other, self._data)
        out = fn(a, b)
        parents = (self,) if other_t is None else (self, other_t)

        def backward(g):
            ga, gb = vjp(g, a, b)
            ga = _sum_to_shape(ga, a.shape)
            if other_t is None:
                return (ga,)
            return ga, _sum_to_shape(gb, tuple(b.shape))

        return Tensor._from_op(out, parents, backward, op)

    def __add__(self, other):
        return self._binary(other, lambda a, b: a + b, lambda g, a, b: (g, g), "add")

    __radd__ = __add__

    def __sub__(self, other):
        return self._binary(other, lambda a, b: a - b, lambda g, a, b: (g, -g), "sub")

    def __rsub__(self, other):
        return (-self) + other

    def __mul__(self, other):
        return self._binary(other, lambda a, b: a * b, lambda g, a, b: (g * b, g * a), "mul")

    __rmul__ = __mul__

    def __truediv__(self, other):
        return self._binary(other, lambda a, b: a / b,
                            lambda g, a, b: (g / b, -g * a / (b * b)), "div")

    def __neg__(self):
        return Tensor._from_op(-self._data, (self,), lambda g: (-g,), "neg")

    def __pow__(self, exponent: float):
        if isinstance(exponent, Tensor):
            raise TypeError("only scalar exponents are supported")
        x = self._data
        out = x**exponent
        return Tensor._from_op(out, (self,), lambda g: (g * exponent * x ** (exponent - 1),), "pow")

    # -- reductions / shape --------------------------------------------------
    def sum(self, axis=None, keepdims: bool = False) -> Tensor:
        x = self._data
        out = _sum(x, axis, keepdims)
        shape = x.shape

        def backward(g):
            if axis is not None and not keepdims:
                axes = (axis,) if isinstance(axis, int) else tuple(axis)
                axes = sorted(a % len(shape) for a in axes)
                for a in axes:
                    g = g.unsqueeze(a) if is_torch(g) else np.expand_dims(g, a)
            elif axis is None and not keepdims:
                g = g.reshape([1] * len(shape))
            return (g * _ones_like(x),)

        return Tensor._from_op(out, (self,), backward, "sum")

    def mean(self, axis=None, keepdims: bool = False) -> Tensor:
        count = self.size if axis is None else math.prod(
            self.shape[a] for a in ((axis,) if isinstance(axis, int) else axis))
        return self.sum(axis, keepdims) * (1.0 / count)

    def reshape(self, *shape) -> Tensor:
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        source = self.shape
        out = self._data.reshape(shape)
        return Tensor._from_op(out, (self,), lambda g: (g.reshape(source),), "reshape")

    def permute(self, *axes) -> Tensor:
        if len(axes) == 1 and isinstance(axes[0], (tuple, list)):
            axes = tuple(axes[0])
        inverse = tuple(np.argsort(axes))
        out = _permute(self._data, axes)
        return Tensor._from_op(out, (self,), lambda g: (_permute(g, inverse),), "permute")

    def transpose(self, a: int = -2, b: int = -1) -> Tensor:
        axes = list(range(self.ndim))
        axes[a], axes[b] = axes[b], axes[a]
        return self.permute(*axes)

    def unsqueeze(self, dim: int) -> Tensor:
        d = dim if dim >= 0 else dim + self.ndim + 1
        if not 0 <= d <= self.ndim:
            raise ValueError("unsqueeze dimension out of range")
        return self.reshape(*self.shape[:d], 1, *self.shape[d:])

    def contiguous(self) -> Tensor:
        if not is_torch(self._data) or self._data.is_contiguous():
            return self
        return Tensor._from_op(self._data.contiguous(), (self,), lambda g: (g,), "contiguous")

    def __getitem__(self, key) -> Tensor:
        if isinstance(key, Tensor):
            key = key._data
        x = self._data
        out = x[key]

        def backward(g):
            full = _zeros_like(x)
            full[key] = full[key] + g
            return (full,)

        return Tensor._from_op(out, (self,), backward, "getitem")

    def __matmul__(self, other: Tensor) -> Tensor:
        from .amp import _cast_inputs

        a_t, b_t = _cast_inputs(self, other)
        a, b = a_t._data, b_t._data
        out = a @ b

        def backward(g):
            ga = g @ (b.transpose(-1, -2) if is_torch(b) else np.swapaxes(b, -1, -2))
            gb = (a.transpose(-1, -2) if is_torch(a) else np.swapaxes(a, -1, -2)) @ g
            return _sum_to_shape(ga, a.shape), _sum_to_shape(gb, b.shape)

        return Tensor._from_op(out, (a_t, b_t), backward, "matmul")


def _run_backward(root: Tensor, seed, *, retain_graph=False, accumulate=False, requested=()):
    """First-order VJP engine (reference ``tensor.py:662-724``)."""
    topo, visited = [], set()
    stack = [(root, False)]
    while stack:
        node, expanded = stack.pop()
        if expanded:
            topo.append(node)
            continue
        if id(node) in visited:
            continue
        if node._graph_freed:
            raise RuntimeError("autograd tape already freed; use retain_graph=True on the first pass")
        visited.add(id(node))
        stack.append((node, True))
        stack.extend((parent, False) for parent in node._parents)
    requested = set(requested)
    result, pending = {}, {id(root): seed}
    for node in reversed(topo):
        contribution = pending.pop(id(node), None)
        if contribution is None:
            continue
        # contributions arrive in the destination tensor's precision (:689-690)
        if node.requires_grad and contribution.dtype != node.dtype:
            contribution = _cast(contribution, node.dtype)
        if id(node) in requested:
            result[id(node)] = contribution
        if accumulate and node.requires_grad:
            node._grad = contribution if node._grad is None else node._grad + contribution
        if node._backward is not None:
            grads = node._backward(contribution)
            if len(grads) != len(node._parents):
                raise RuntimeError(f"internal error: {node._op} returned wrong number of gradients")
            for parent, pg in zip(node._parents, grads):
                if pg is None or not parent.requires_grad:
                    continue
                key = id(parent)
                pending[key] = pg if key not in pending else pending[key] + pg
    if not retain_graph:
        for node in topo:
            if node._backward is not None:
                node._parents = ()
                node._backward = None
                node._graph_freed = True
    return result


def grad(output: Tensor, inputs: Tensor | Sequence[Tensor], grad_outputs=None, *,
         retain_graph=False, allow_unused=False) -> tuple[Tensor | None, ...]:
    """Gradients of ``output`` w.r.t. ``inputs`` without touching ``.grad``
    (reference ``tensor.py:727-760``)."""
    inputs = (inputs,) if isinstance(inputs, Tensor) else tuple(inputs)
    if not output.requires_grad or any(not x.requires_grad for x in inputs):
        raise RuntimeError("output and requested inputs must require gradients")
    seed = _ones_like(output._data) if grad_outputs is None else to_backend(grad_outputs, output.device)
    values = _run_backward(output, seed, retain_graph=retain_graph, requested=(id(x) for x in inputs))
    if not allow_unused and any(id(x) not in values for x in inputs):
        raise RuntimeError("a requested input is not used by the output")
    return tuple(Tensor(values[id(x)], device=x.device) if id(x) in values else None for x in inputs)


# ---------------------------------------------------------------------------
# Creation helpers
# ---------------------------------------------------------------------------


def tensor(data, *, requires_grad=False, device=None, dtype=None) -> Tensor:
    return Tensor(data, requires_grad=requires_grad, device=device, dtype=dtype)


def zeros(*shape, device=None, dtype="float32", requires_grad=False) -> Tensor:
    if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
        shape = tuple(shape[0])
    dev = parse_device(device)
    if dev.type == "hip":
        raw = _torch().zeros(shape, dtype=backend_dtype(dtype, dev), device=dev.torch)
    else:
        raw = np.zeros(shape, dtype=backend_dtype(dtype, dev))
    return Tensor(raw, device=dev, requires_grad=requires_grad)


def randn(*shape, device=None, dtype="float32", requires_grad=False) -> Tensor:
    """N(0,1) drawn from the host RNG (``ts.seed``), then moved to ``device``."""
    if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
        shape = tuple(shape[0])
    host = np.random.standard_normal(shape).astype(np.float32)
    return Tensor(host, device=device, dtype=dtype, requires_grad=requires_grad)


def cat(tensors: Sequence[Tensor], dim: int = 0) -> Tensor:
    tensors = list(tensors)
    raws = [t._data for t in tensors]
    if is_torch(raws[0]):
        out = _torch().cat(raws, dim=dim)
    else:
        out = np.concatenate(raws, axis=dim)
    sizes = [r.shape[dim] for r in raws]

    def backward(g):
        parts, start = [], 0
        for n in sizes:
            index = [slice(None)] * g.ndim
            index[dim] = slice(start, start + n)
            parts.append(g[tuple(index)])
            start += n
        return tuple(parts)

    return Tensor._from_op(out, tuple(tensors), backward, "cat")
