"""The four attention workloads at full size (needs an MI355X).

Heads and batch rows are independent, so a sample of (batch, head) pairs (and,
for the 32k prefill, of query-row blocks) checked against the oracle is a
parity check at the real shape; every output is also checked finite.
Tolerances as in test_gpu_parity.py (bf16: rel-L2 1e-2 / 2e-2, max-abs
2e-2 * max|ref|; fp16: 2e-3 / 5e-3, 5e-3 * max|ref|; LSE 1e-3).
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("no GPU", allow_module_level=True)

import abi  # noqa: E402
import tensorsmith_hip as ts  # noqa: E402
from oracle import attention as A  # noqa: E402
from tensorsmith_hip import _lib  # noqa: E402
from test_gpu_parity import check_half, check_lse, say  # noqa: E402


def draw(gen, shape, scale, dtype):
    x = torch.randn(shape, generator=gen, device="cuda", dtype=torch.float32)
    return (x * scale).to(dtype)


def host(t):
    return t.float().cpu().numpy()


def test_causal_fwd_bwd_bf16_b16h16s2048d128():
    gen = torch.Generator(device="cuda").manual_seed(42)
    shape = (16, 16, 2048, 128)
    q, k, v = (draw(gen, shape, 0.5, torch.bfloat16) for _ in range(3))
    g = draw(gen, shape, 1.0, torch.bfloat16)
    say("full-size bf16 causal fwd+bwd")
    out, lse, path = abi.forward(q, k, v, causal=True)
    assert path == _lib.PATH_MFMA
    dq, dk, dv, _ = abi.backward(q, k, v, out, g, lse, causal=True)
    torch.cuda.synchronize()
    for t in (out, lse, dq, dk, dv):
        assert torch.isfinite(t).all()
    for b, h in ((0, 0), (7, 3), (15, 15)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        ref = A.sdpa(host(q[sl]), host(k[sl]), host(v[sl]), None, True, dtype="bfloat16",
                     backend="streaming")
        check_half(host(out[sl]), ref.out, "bfloat16", "o", f"O b{b}h{h}")
        check_lse(host(lse[sl]), ref.lse, f"LSE b{b}h{h}")
        for got, want, n in zip((dq, dk, dv), ref.backward_compute(host(g[sl])), ("dQ", "dK", "dV")):
            check_half(host(got[sl]), want, "bfloat16", "g", f"{n} b{b}h{h}")


def test_decode_f16_b64h32d128_ragged_lengths():
    gen = torch.Generator(device="cuda").manual_seed(42)
    B, H, D, cap = 64, 32, 128, 8192
    q = torch.randn((B, H, 1, D), generator=gen, device="cuda").half()
    k = torch.randn((B, H, cap, D), generator=gen, device="cuda", dtype=torch.float16)
    v = torch.randn((B, H, cap, D), generator=gen, device="cuda", dtype=torch.float16)
    lengths = torch.randint(512, 8193, (B,), generator=gen, device="cuda")
    mask = (torch.arange(cap, device="cuda")[None, :] < lengths[:, None])[:, None, None, :]
    say("full-size fp16 decode")
    with ts.no_grad():
        out = ts.nn.scaled_dot_product_attention(*(ts.Tensor(t, device="hip") for t in (q, k, v)),
                                                 ts.Tensor(mask, device="hip"))
    assert _lib.last_kernel_path() == _lib.PATH_DECODE
    got = out.numpy()
    assert np.isfinite(got).all()
    lens = lengths.cpu().numpy()
    for b, h in ((0, 0), (1, 31), (17, 5), (63, 16), (int(np.argmin(lens)), 7),
                 (int(np.argmax(lens)), 9)):
        L = int(lens[b])
        ref = A.sdpa(host(q[b:b + 1, h:h + 1]), host(k[b:b + 1, h:h + 1, :L]),
                     host(v[b:b + 1, h:h + 1, :L]), None, False, dtype="float16", backend="dense")
        check_half(got[b:b + 1, h:h + 1], ref.out, "float16", "o", f"decode b{b}h{h} len{L}")


def test_padded_prefill_bf16_b2h32s32768d128():
    gen = torch.Generator(device="cuda").manual_seed(42)
    B, H, S, D = 2, 32, 32768, 128
    q, k, v = (draw(gen, (B, H, S, D), 0.5, torch.bfloat16) for _ in range(3))
    lengths = torch.randint(16384, 32769, (B,), generator=gen, device="cuda")
    keymask = torch.arange(S, device="cuda")[None, :] < lengths[:, None]
    say("full-size bf16 32k key-padded prefill")
    with ts.no_grad():
        out = ts.nn.scaled_dot_product_attention(
            *(ts.Tensor(t, device="hip") for t in (q, k, v)),
            ts.Tensor(keymask[:, None, None, :], device="hip"), is_causal=True)
    assert _lib.last_kernel_path() == _lib.PATH_MFMA
    assert torch.isfinite(out._data).all()
    lens = lengths.cpu().numpy()
    kmh = keymask.cpu().numpy()
    for b, h in ((0, 0), (1, 31)):
        L = int(lens[b])
        kh, vh = host(k[b:b + 1, h:h + 1]), host(v[b:b + 1, h:h + 1])
        for r0 in (0, L - 64, S - 64):
            ref = A.sdpa(host(q[b:b + 1, h:h + 1, r0:r0 + 64]), kh, vh, kmh[b][None, None, None],
                         True, dtype="bfloat16", causal_offset=r0, backend="streaming")
            check_half(host(out._data[b:b + 1, h:h + 1, r0:r0 + 64]), ref.out, "bfloat16", "o",
                       f"prefill b{b}h{h} rows {r0}..{r0 + 63} (len {L})")
