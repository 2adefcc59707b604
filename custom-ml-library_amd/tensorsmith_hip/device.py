"""Devices: ``cpu`` (host arrays) and ``hip`` / ``hip:N`` (an MI355X).

Mirrors the reference's device layer (``src/tensorsmith/device.py:26-62,
117-129,306-314``) with ``hip`` added to the allowed device types.  Host
tensors hold NumPy arrays; ``hip`` tensors hold PyTorch-ROCm device tensors,
which serve only as device memory and stream plumbing -- attention runs in
the HIP kernels of ``libtsattn.so``.
"""

from __future__ import annotations

from contextvars import ContextVar
from dataclasses import dataclass
from functools import cache

import numpy as np


@dataclass(frozen=True)
class Device:
    """A compute device, ``cpu`` or ``hip:N``."""

    type: str = "cpu"
    index: int | None = None

    def __post_init__(self) -> None:
        kind = self.type.lower()
        if kind not in {"cpu", "hip"}:
            raise ValueError(f"unknown device {self.type!r}; expected cpu or hip")
        if kind == "cpu" and self.index is not None:
            raise ValueError("cpu does not accept a device index")
        if kind == "hip" and self.index is not None and self.index < 0:
            raise ValueError("HIP device index must be non-negative")
        if kind == "hip" and self.index is None:
            object.__setattr__(self, "index", 0)
        object.__setattr__(self, "type", kind)

    def __str__(self) -> str:
        return f"hip:{self.index}" if self.type == "hip" else "cpu"

    @property
    def torch(self):
        """The torch.device backing this device (hip:N -> ROCm 'cuda:N')."""
        import torch

        return torch.device("cpu") if self.type == "cpu" else torch.device("cuda", self.index)


DeviceLike = str | Device | None


def device(value: DeviceLike = None) -> Device:
    if value is None:
        return Device("cpu")
    if isinstance(value, Device):
        return value
    value = value.lower().strip()
    if value.startswith("hip:"):
        return Device("hip", int(value.split(":", 1)[1]))
    return Device(value)


@cache
def _is_available(dev: Device) -> bool:
    if dev.type == "cpu":
        return True
    try:
        import torch
    except ImportError:
        return False
    return bool(torch.cuda.is_available() and torch.cuda.device_count() > (dev.index or 0))


def is_available(value: DeviceLike) -> bool:
    return _is_available(device(value))


def require_available(value: DeviceLike) -> Device:
    dev = device(value)
    if is_available(dev):
        return dev
    raise RuntimeError(f"device {dev} is unavailable; an MI355X with PyTorch-ROCm is required")


def available_devices() -> list[Device]:
    result = [Device("cpu")]
    if is_available("hip"):
        import torch

        result.extend(Device("hip", i) for i in range(torch.cuda.device_count()))
    return result


def synchronize(value: DeviceLike = "hip") -> None:
    dev = device(value)
    if dev.type == "hip":
        import torch

        torch.cuda.synchronize(dev.torch)


def seed(value: int) -> None:
    """Seed host-side initialisation and the device generator."""
    np.random.seed(value)
    try:
        import torch

        torch.manual_seed(value)
    except ImportError:
        pass


# Random draws made inside a checkpointed function are recorded on this tape
# and replayed by its recomputation (the reference's ``_random_tape``,
# ``src/tensorsmith/device.py:23,276-297``).  An entry is (kind, shape,
# device, state): a uniform draw keeps the generator state it started from
# (a few bytes, not the drawn array), an attention-dropout key keeps the key.
_random_tape: ContextVar[dict | None] = ContextVar("tensorsmith_hip_random_tape", default=None)


def _replay_entry(kind: str, shape, dev):
    tape = _random_tape.get()
    if tape is None or tape["mode"] != "replay":
        return None
    position = tape["position"]
    if position >= len(tape["draws"]):
        raise RuntimeError("checkpoint recomputation changed the number of random draws")
    entry = tape["draws"][position]
    if entry[0] != kind or entry[1] != shape or entry[2] != dev:
        raise RuntimeError("checkpoint recomputation changed a random draw's shape/device")
    tape["position"] += 1
    return entry


def _record(entry) -> None:
    tape = _random_tape.get()
    if tape is not None and tape["mode"] == "record":
        tape["draws"].append(entry)


def _generator_state(dev: Device):
    import torch

    return torch.cuda.get_rng_state(dev.torch) if dev.type == "hip" else torch.get_rng_state()


def _set_generator_state(dev: Device, state) -> None:
    import torch

    if dev.type == "hip":
        torch.cuda.set_rng_state(state, dev.torch)
    else:
        torch.set_rng_state(state)


def random_uniform(shape, value: DeviceLike = "hip"):
    """Uniform [0, 1) float32 draws from the device generator (the reference's
    ``device.random_uniform``, ``src/tensorsmith/device.py:276-297``).  Under a
    checkpoint the recomputation redraws from the recorded generator state,
    so it sees the same values, and the generator is left where it was."""
    import torch

    dev, shape = device(value), tuple(shape)

    def draw():
        return torch.rand(shape, dtype=torch.float32, device=dev.torch)

    entry = _replay_entry("uniform", shape, dev)
    if entry is not None:
        current = _generator_state(dev)
        _set_generator_state(dev, entry[3])
        try:
            return draw()
        finally:
            _set_generator_state(dev, current)
    _record(("uniform", shape, dev, _generator_state(dev)))
    return draw()


def attention_dropout_key() -> int:
    """A 128-bit Philox key for one attention-dropout call, drawn from NumPy's
    global state (``ts.seed`` reproduces it).  A checkpoint's recomputation
    gets the recorded key back, so the kernels regenerate the same keep mask."""
    drawn = int.from_bytes(np.random.bytes(16), "little")
    entry = _replay_entry("attention_key", None, None)
    if entry is not None:
        return entry[3]
    _record(("attention_key", None, None, drawn))
    return drawn


def current_stream(dev: Device) -> int:
    """Raw hipStream_t of torch's current stream on ``dev`` (0 = default)."""
    import torch

    return torch.cuda.current_stream(dev.torch).cuda_stream
