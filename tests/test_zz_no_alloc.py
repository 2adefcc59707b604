"""tsattn_decode_forward_noalloc through the C ABI (needs an MI355X).

The allocation-free decode entry point keeps its split partials in the
library's static per-GPU scratch array instead of a caller workspace.  Its
output must equal tsattn_decode_forward's bit for bit (same kernels, same
split), on two calls in a row -- the second with a smaller problem, so a
stale partial left in the shared array by the first call would show -- and a
problem whose partials exceed the array is refused before any launch.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("no GPU", allow_module_level=True)

import abi  # noqa: E402
from tensorsmith_hip import _lib  # noqa: E402

SCRATCH = 32 << 20


def say(msg):
    print(msg, flush=True)


def decode_pair(b, hq, hkv, sq, length, d, dtype, seed, kv_len=None):
    """(workspace output, no-alloc output) for one problem."""
    gen = torch.Generator(device="cuda").manual_seed(seed)
    tdt = abi.TORCH_DTYPES[dtype]
    q = torch.randn((b, hq, sq, d), generator=gen, device="cuda").to(tdt)
    k = torch.randn((b, hkv, length, d), generator=gen, device="cuda").to(tdt)
    v = torch.randn((b, hkv, length, d), generator=gen, device="cuda").to(tdt)
    lens = None if kv_len is None else torch.tensor(kv_len, dtype=torch.int32, device="cuda")
    p = abi.problem(q, k, v, causal=True, offset=length - sq, kv_len=lens)
    lib = _lib.load()
    nbytes = lib.tsattn_decode_workspace(ctypes.byref(p), 0)
    assert 0 < nbytes <= SCRATCH
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    out_ws = torch.empty((b, hq, sq, d), dtype=tdt, device="cuda")
    out_na = torch.full_like(out_ws, float("nan"))
    _lib.check(lib.tsattn_decode_forward(ctypes.byref(p), abi.view(q), abi.view(k), abi.view(v),
                                         abi.view(out_ws), 0, ctypes.c_void_p(ws.data_ptr()),
                                         nbytes, abi.stream()), "decode")
    _lib.check(lib.tsattn_decode_forward_noalloc(ctypes.byref(p), abi.view(q), abi.view(k),
                                                 abi.view(v), abi.view(out_na), 0, abi.stream()),
               "decode noalloc")
    assert lib.tsattn_last_kernel_path() == _lib.PATH_DECODE
    torch.cuda.synchronize()
    return out_ws, out_na


def test_noalloc_decode_matches_workspace_decode_twice():
    # first call: B64 H32 D128 fp16, 4000 keys (~8 MB of partials)
    say("noalloc decode: call 1, B64 H32 S4000 D128 fp16")
    a, b = decode_pair(64, 32, 32, 1, 4000, 128, "float16", 1)
    assert torch.isfinite(b).all()
    assert torch.equal(a, b)
    # second call, smaller (GQA, 2 query rows, ragged lengths): fewer splits and
    # rows, so slots the first call filled are not read
    say("noalloc decode: call 2, B3 Hq8 Hkv2 Sq2 S700 D64 bf16, ragged")
    a, b = decode_pair(3, 8, 2, 2, 700, 64, "bfloat16", 2, kv_len=[700, 129, 333])
    assert torch.isfinite(b).all()
    assert torch.equal(a, b)


def test_noalloc_decode_refuses_problems_beyond_its_scratch():
    q = torch.zeros((64, 32, 8, 256), dtype=torch.float16, device="cuda")
    kv = torch.zeros((64, 32, 1, 256), dtype=torch.float16, device="cuda")
    p = abi.problem(q, kv, kv)
    p.len_kv = 1 << 20  # 1M keys: far more partials than the array holds
    lib = _lib.load()
    need = lib.tsattn_decode_workspace(ctypes.byref(p), 0)
    assert need > SCRATCH
    rc = lib.tsattn_decode_forward_noalloc(ctypes.byref(p), abi.view(q), abi.view(kv),
                                           abi.view(kv), abi.view(q), 0, abi.stream())
    assert rc == _lib.ERR_INVALID and "scratch" in _lib.last_error()
