"""The reference-side ctypes binding (tensorsmith_binding/_tsattn.py) on the GPU.

This is the module a tensorsmith maintainer copies next to the reference's
attention dispatch (src/tensorsmith/nn/attention.py:87, :250-252).  Checked
here, through that module alone:

* a causal bf16 forward + backward at B16 H16 S2048 D128 gives the same bits
  as the C-ABI drivers of the parity suite (same kernels, same problem), and
  sampled heads meet the bf16 bounds against the oracle (relative L2 1e-2 for
  O, 2e-2 for gradients; max-abs 2e-2 * max|ref|; LSE 1e-3);
* a dropout forward + backward (p = 0.2, explicit key) meets the same bounds
  against the oracle's dense dropout attention under that key's mask, and
  the binding's default key (drawn from NumPy's state) is replayed exactly
  after np.random.seed -- what a checkpoint's state restore relies on;
* decode over a 16-bit cache and the int8 append match the oracle (fp16
  bounds 2e-3; the int8 quantiser bit for bit).
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("no GPU", allow_module_level=True)

import abi  # noqa: E402
from oracle import attention as A  # noqa: E402
from oracle import dropout as DR  # noqa: E402
from oracle.inputs import attention_inputs  # noqa: E402
from tensorsmith_binding import _tsattn as B  # noqa: E402
from test_gpu_parity import check_half, check_lse, say  # noqa: E402


def host(t):
    return t.detach().float().cpu().numpy()


def test_binding_loads_abi():
    lib = B.load()
    assert lib.tsattn_abi_version() == B.ABI_VERSION == 8
    assert B.Problem.dropout_bits.offset == 152


def test_binding_causal_fwd_bwd_bf16_b16h16s2048d128():
    gen = torch.Generator(device="cuda").manual_seed(7)
    shape = (16, 16, 2048, 128)
    q, k, v, g = ((torch.randn(shape, generator=gen, device="cuda") * s).to(torch.bfloat16)
                  for s in (0.5, 0.5, 0.5, 1.0))
    say("binding: bf16 causal fwd+bwd B16 H16 S2048 D128")
    out, backward = B.sdpa_hip(q, k, v, None, 0.0, True, None, 0, record=True)
    dq, dk, dv = backward(g)
    ref_out, ref_lse, _ = abi.forward(q, k, v, causal=True)
    rdq, rdk, rdv, _ = abi.backward(q, k, v, ref_out, g, ref_lse, causal=True)
    torch.cuda.synchronize()
    for got, want, name in ((out, ref_out, "O"), (dq, rdq, "dQ"), (dk, rdk, "dK"), (dv, rdv, "dV")):
        assert torch.equal(got, want), f"{name} differs from the C-ABI driver"
    for b, h in ((0, 5), (11, 14)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        ref = A.sdpa(host(q[sl]), host(k[sl]), host(v[sl]), None, True, dtype="bfloat16",
                     backend="streaming")
        check_half(host(out[sl]), ref.out, "bfloat16", "o", f"O b{b}h{h}")
        check_lse(host(ref_lse[sl]), ref.lse, f"LSE b{b}h{h}")
        for got, want, n in zip((dq, dk, dv), ref.backward_compute(host(g[sl])), ("dQ", "dK", "dV")):
            check_half(host(got[sl]), want, "bfloat16", "g", f"{n} b{b}h{h}")


def test_binding_dropout_fwd_bwd_matches_oracle():
    dtype, b, h, sq, d, p = "bfloat16", 2, 4, 256, 128, 0.2
    inp = attention_inputs(b, h, sq, d, dtype, value_scale=0.5, seed=77)
    key = 0x0123_4567_89AB_CDEF_FEDC_BA98_7654_3210
    say("binding: bf16 causal dropout fwd+bwd")
    out_c, _, back = DR.sdpa_dropout(inp.q, inp.k, inp.v, None, True, dtype=dtype, p=p,
                                     rng_key=key, rng_counter=0)
    q, k, v, g = (abi.dev_tensor(x, dtype) for x in (inp.q, inp.k, inp.v, inp.do))
    out, backward = B.sdpa_hip(q, k, v, None, p, True, None, 0, dropout_key=key)
    dq, dk, dv = backward(g)
    torch.cuda.synchronize()
    check_half(host(out), out_c, dtype, "o", "O")
    for got, want, name in zip((dq, dk, dv), back(inp.do), ("dQ", "dK", "dV")):
        check_half(host(got), want, dtype, "g", name)
    # default keys come from NumPy's global state: reseeding replays them
    np.random.seed(3)
    out1, _ = B.sdpa_hip(q, k, v, None, p, True, None, 0, record=False)
    out2, _ = B.sdpa_hip(q, k, v, None, p, True, None, 0, record=False)
    np.random.seed(3)
    out3, _ = B.sdpa_hip(q, k, v, None, p, True, None, 0, record=False)
    assert torch.equal(out1, out3) and not torch.equal(out1, out2)


def test_binding_decode_and_int8_append():
    dtype, b, hkv, hq, cap, length, d = "float16", 3, 2, 4, 512, 300, 128
    gen = np.random.default_rng(5)
    kc = torch.zeros((b, hkv, cap, d), dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    kh = gen.standard_normal((b, hkv, length, d)).astype(np.float32)
    vh = gen.standard_normal((b, hkv, length, d)).astype(np.float32)
    kc[:, :, :length] = abi.dev_tensor(kh, dtype)
    vc[:, :, :length] = abi.dev_tensor(vh, dtype)
    qh = gen.standard_normal((b, hq, 1, d)).astype(np.float32)
    q = abi.dev_tensor(qh, dtype)
    say("binding: fp16 decode")
    out = B.decode(q, kc, vc, length)
    torch.cuda.synchronize()
    ref = A.sdpa(host(q), host(kc[:, :, :length]), host(vc[:, :, :length]), None, True,
                 dtype=dtype, causal_offset=length - 1, backend="dense", enable_gqa=True)
    check_half(host(out), ref.out, dtype, "o", "decode O")
    say("binding: int8 append")
    codes = torch.zeros((b, hkv, cap, d), dtype=torch.int8, device="cuda")
    scales = torch.zeros((b, hkv, cap, 1), dtype=torch.float32, device="cuda")
    B.append_int8(kc[:, :, :length], codes, scales, 16)
    torch.cuda.synchronize()
    want_codes, want_scales = A.quantize_int8(host(kc[:, :, :length]))
    np.testing.assert_array_equal(codes[:, :, 16:16 + length].cpu().numpy(), want_codes)
    np.testing.assert_array_equal(scales[:, :, 16:16 + length].cpu().numpy(), want_scales)


@pytest.mark.parametrize("quantized", [False, True])
def test_binding_project_rope_append(quantized):
    """The cached step before the attention through the binding gives the
    same bits as the C-ABI driver of the parity suite (test_gpu_qkv.py checks
    that driver against the oracle)."""
    say(f"binding: fused projection + RoPE + append, int8 cache={quantized}")
    gen = torch.Generator(device="cuda").manual_seed(5)
    b, t, e, hq, hkv, d, cap, pos = 2, 3, 256, 4, 2, 128, 16, 5
    x = torch.randn((b, t, e), generator=gen, device="cuda").half()
    ws = [(torch.randn((h * d, e), generator=gen, device="cuda") / 16).half() for h in (hq, hkv, hkv)]
    bs = [(torch.randn(h * d, generator=gen, device="cuda") / 10).half() for h in (hq, hkv, hkv)]
    ang = torch.arange(pos + t, device="cuda", dtype=torch.float32)[:, None] * torch.exp(
        -torch.arange(0, d, 2, device="cuda", dtype=torch.float32) / d * np.log(10000.0))
    cos, sin = ang.cos().half(), ang.sin().half()
    outs = []
    for drive in ("abi", "binding"):
        q = torch.zeros((b, hq, t, d), dtype=torch.float16, device="cuda")
        cdt = torch.int8 if quantized else torch.float16
        kc, vc = (torch.zeros((b, hkv, cap, d), dtype=cdt, device="cuda") for _ in range(2))
        sc = tuple(torch.ones((b, hkv, cap, 1), device="cuda") for _ in range(2)) if quantized else None
        if drive == "abi":
            abi.qkv_rope_append(x, *ws, bs, q, kc, vc, sc, cos, sin, pos, hq, hkv)
        else:
            B.project_rope_append(x, ws, bs, q, kc, vc, sc, cos, sin, pos, hq, hkv)
        torch.cuda.synchronize()
        outs.append([q, kc, vc] + list(sc or ()))
    for got, want in zip(outs[1], outs[0]):
        assert torch.equal(got, want)
    assert outs[0][1][:, :, pos:pos + t].abs().sum() > 0


def test_binding_project_rope_append_refuses_other_layouts():
    """Weights and biases reach the C entry point as bare pointers, so the
    binding refuses, before any launch, what the kernel cannot read as
    [heads * D, E] rows of x's dtype: a transposed weight view, a bias of
    another dtype, a weight of the wrong shape."""
    b, t, e, hq, hkv, d = 1, 1, 64, 2, 1, 64
    x = torch.zeros((b, t, e), dtype=torch.float16, device="cuda")
    ws = [torch.zeros((h * d, e), dtype=torch.float16, device="cuda") for h in (hq, hkv, hkv)]
    q = torch.zeros((b, hq, t, d), dtype=torch.float16, device="cuda")
    kc, vc = (torch.zeros((b, hkv, 4, d), dtype=torch.float16, device="cuda") for _ in range(2))
    transposed = torch.zeros((e, hkv * d), dtype=torch.float16, device="cuda").t()
    assert transposed.shape == ws[1].shape and not transposed.is_contiguous()
    fp32_bias = [None, torch.zeros(hkv * d, device="cuda"), None]
    for weights, biases in (([ws[0], transposed, ws[2]], None),
                            (ws, fp32_bias),
                            ([ws[0], ws[1], ws[1][:, :32]], None)):
        with pytest.raises(NotImplementedError):
            B.project_rope_append(x, weights, biases, q, kc, vc, None, None, None, 0, hq, hkv)
