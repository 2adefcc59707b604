"""ctypes binding of ``libtsattn.so`` (C ABI declared in ``include/tsattn.h``).

The library is loaded lazily on first use and the load fails loudly: there is
no CPU fallback for the attention path.  Status codes map onto the
exceptions the reference raises for the same conditions
(``src/tensorsmith/nn/attention.py:36-86``): contract violations become
``ValueError`` (``TypeError`` for dtype problems), unsupported requests
``NotImplementedError`` and HIP failures ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import POINTER, c_char_p, c_double, c_int, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_native" / "libtsattn.so"
ABI_VERSION = 8

OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP = 0, 1, 2, 3
F32, F16, BF16, F64, BOOL, I8 = 0, 1, 2, 3, 4, 5
MASK_NONE, MASK_BOOL, MASK_ADDITIVE = 0, 1, 2
PATH_GENERIC, PATH_MFMA, PATH_DECODE = 1, 2, 3


class View(ctypes.Structure):
    """``tsattn_view``: data pointer + 4 element strides."""

    _fields_ = [("data", c_void_p), ("stride", c_int64 * 4)]


class Problem(ctypes.Structure):
    """``tsattn_problem``: shapes, scale, causal flags, lengths and mask."""

    _fields_ = [
        ("dtype", c_int32),
        ("batch", c_int32),
        ("heads_q", c_int32),
        ("heads_kv", c_int32),
        ("len_q", c_int32),
        ("len_kv", c_int32),
        ("dim_qk", c_int32),
        ("dim_v", c_int32),
        ("scale", c_double),
        ("is_causal", c_int32),
        ("causal_offset", c_int64),
        ("kv_len", c_void_p),
        ("kv_prefix", c_void_p),
        ("mask_kind", c_int32),
        ("mask_dtype", c_int32),
        ("mask", View),
        ("dropout_p", c_double),
        ("dropout_key", ctypes.c_uint64 * 2),
        ("dropout_counter", ctypes.c_uint64),
        ("dropout_bits", ctypes.c_void_p),
    ]


class RopeDesc(ctypes.Structure):
    """``tsattn_rope_desc``: cos / sin tables, rotary dim, query / key positions,
    optional rotated-query buffer."""

    _fields_ = [
        ("cos", c_void_p),
        ("sin", c_void_p),
        ("rotary_dim", c_int32),
        ("q_pos0", c_int64),
        ("k_pos0", c_int64),
        ("q_rotated", c_void_p),
    ]


_PV = POINTER(View)
_PP = POINTER(Problem)
_PR = POINTER(RopeDesc)

# name -> (restype, argtypes); exactly the symbols include/tsattn.h declares
SIGNATURES = {
    "tsattn_abi_version": (c_int, []),
    "tsattn_last_error": (c_char_p, []),
    "tsattn_set_kernel_policy": (c_int, [c_int]),
    "tsattn_last_kernel_path": (c_int, []),
    "tsattn_sdpa_forward": (c_int, [_PP, _PV, _PV, _PV, _PV, c_void_p, c_void_p]),
    "tsattn_sdpa_backward_workspace": (c_size_t, [_PP]),
    "tsattn_sdpa_backward": (
        c_int,
        [_PP, _PV, _PV, _PV, _PV, _PV, c_void_p, _PV, _PV, _PV, c_void_p, c_size_t, c_void_p],
    ),
    "tsattn_sdpa_forward_rope": (c_int, [_PP, _PR, _PV, _PV, _PV, _PV, c_void_p, c_void_p]),
    "tsattn_sdpa_backward_rope_workspace": (c_size_t, [_PP]),
    "tsattn_dropout_keep": (c_int, [_PP, c_void_p, c_void_p]),
    "tsattn_dropout_bits_bytes": (c_size_t, [_PP]),
    "tsattn_sdpa_backward_rope": (
        c_int,
        [_PP, _PR, _PV, _PV, _PV, _PV, _PV, c_void_p, _PV, _PV, _PV, c_void_p, c_size_t,
         c_void_p],
    ),
    "tsattn_decode_workspace": (c_size_t, [_PP, c_int32]),
    "tsattn_decode_forward": (
        c_int,
        [_PP, _PV, _PV, _PV, _PV, c_int32, c_void_p, c_size_t, c_void_p],
    ),
    "tsattn_decode_forward_noalloc": (c_int, [_PP, _PV, _PV, _PV, _PV, c_int32, c_void_p]),
    "tsattn_decode_forward_int8": (
        c_int,
        [_PP, _PV, _PV, _PV, _PV, _PV, _PV, c_int32, c_void_p, c_size_t, c_void_p],
    ),
    "tsattn_decode_forward_rope": (
        c_int,
        [_PP, _PR, _PV, _PV, _PV, _PV, _PV, _PV, c_int32, c_void_p, c_size_t, c_void_p],
    ),
    "tsattn_kv_append_int8": (
        c_int,
        [c_int32, c_int32, c_int32, c_int32, c_int32, _PV, _PV, _PV, c_int64, c_void_p],
    ),
    "tsattn_rope": (
        c_int,
        [c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, _PV, _PV, c_void_p, c_void_p,
         c_int64, c_int32, c_void_p],
    ),
    "tsattn_rope_append": (
        c_int,
        [c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, _PV, _PV, _PV, _PV, _PV, _PV,
         c_void_p, c_void_p, c_int64, c_void_p],
    ),
    "tsattn_qkv_rope_append": (
        c_int,
        [c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, _PV, c_void_p,
         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, _PV, _PV, _PV, _PV, _PV, c_void_p,
         c_void_p, c_int64, c_void_p],
    ),
    "tsattn_key_mask_lengths": (
        c_int,
        [c_void_p, c_int64, c_int64, c_int32, c_int32, c_void_p, c_void_p, c_void_p],
    ),
    "tsattn_profile_enable": (c_int, [c_int]),
    "tsattn_profile_reset": (c_int, []),
    "tsattn_profile_read": (
        c_int,
        [c_int, ctypes.c_char_p, c_size_t, POINTER(ctypes.c_longlong), POINTER(c_double)],
    ),
}

_lock = threading.Lock()
_lib = None


def load(path: Path | str | None = None):
    """Load (once) and return the library; raises if it is missing or stale."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        target = Path(path) if path is not None else LIB_PATH
        if not target.exists():
            raise RuntimeError(
                f"{target} is not built; run __graft_entry__.build() "
                "(hipcc --offload-arch=gfx950). tensorsmith_hip has no CPU fallback."
            )
        lib = ctypes.CDLL(str(target))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        version = lib.tsattn_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"libtsattn ABI {version} != expected {ABI_VERSION}; rebuild")
        if path is None:
            _lib = lib
        return lib


def last_error() -> str:
    raw = load().tsattn_last_error()
    return raw.decode() if raw else ""


def check(status: int, what: str) -> None:
    if status == OK:
        return
    msg = last_error() or what
    if status == ERR_INVALID:
        if "dtype" in msg or "floating" in msg:
            raise TypeError(msg)
        raise ValueError(msg)
    if status == ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(f"{what}: {msg}")


def set_kernel_policy(policy: int) -> None:
    check(load().tsattn_set_kernel_policy(policy), "set kernel policy")


def last_kernel_path() -> int:
    return load().tsattn_last_kernel_path()


def profile_enable(on: bool) -> None:
    """Bracket every kernel launch with hipEvents on its stream (diagnostic)."""
    load().tsattn_profile_enable(1 if on else 0)


def profile_reset() -> None:
    load().tsattn_profile_reset()


def profile_read() -> dict[str, tuple[int, float]]:
    """{kernel name: (launches, summed ms)} of the probed launches so far."""
    lib = load()
    out = {}
    buf = ctypes.create_string_buffer(64)
    n, ms = ctypes.c_longlong(), c_double()
    i = 0
    while lib.tsattn_profile_read(i, buf, 64, ctypes.byref(n), ctypes.byref(ms)) == OK:
        out[buf.value.decode()] = (int(n.value), float(ms.value))
        i += 1
    return out
