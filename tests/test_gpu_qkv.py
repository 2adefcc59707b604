"""The cached attention step's projections, RoPE and cache append in one
kernel (tsattn_qkv_rope_append; needs an MI355X).

* Projections q / k / v = x W^T (+ b) against the oracle's fp32 products of
  the same rounded inputs, rounded to the dtype (the reference's Linear,
  src/tensorsmith/nn/layers.py:30-31), at the fp16 / bf16 output bounds of
  the parity tests (relative L2 <= 2e-3 / 1e-2, max-abs <= 5e-3 / 2e-2 of
  max|ref|).
* RoPE bit-exact: the kernel's rotated rows equal oracle/rope.py applied to
  the kernel's own unrotated projections (a run with no tables).
* int8 caches bit-exact: codes and scales equal the reference quantiser
  (cache.py:73-77) on the kernel's own 16-bit rows.
* Cache rows outside [pos, pos + len) untouched; GQA, bias, embed widths
  that split unevenly over the waves (E 64: one 64-column chunk, so one
  wave of the 16-bit kernel and seven of the int8 one have none), one and
  several new rows.
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("no GPU", allow_module_level=True)

import abi  # noqa: E402
from conftest import rel_l2  # noqa: E402
from oracle import attention as A  # noqa: E402
from oracle import rope as R  # noqa: E402
from oracle.halfprec import round_to  # noqa: E402
from tensorsmith_hip import _lib  # noqa: E402

BOUND = {"bfloat16": (1e-2, 2e-2), "float16": (2e-3, 5e-3)}


def say(msg):
    print(msg, flush=True)


def _check(got, ref, dtype, name):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = rel_l2(got, ref)
    mx = np.abs(got - ref).max() / (np.abs(ref).max() or 1.0)
    say(f"  {name}: rel_l2={err:.2e} max_abs/max|ref|={mx:.2e}")
    assert err <= BOUND[dtype][0] and mx <= BOUND[dtype][1], name


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("d,e,t,bias", [(64, 208, 1, False), (128, 256, 5, True), (64, 512, 3, True),
                                        (128, 96, 1, False), (128, 64, 2, True), (64, 64, 1, False)])
def test_fused_projection_rope_append(dtype, d, e, t, bias):
    say(f"qkv rope append {dtype} D{d} E{e} T{t} bias={bias}")
    rng = np.random.default_rng(d + e + t)
    b, hq, hkv, pos, cap = 3, 4, 2, 7, 16
    x = round_to(rng.standard_normal((b, t, e)).astype(np.float32), dtype)
    ws = [round_to((rng.standard_normal((h * d, e)) / np.sqrt(e)).astype(np.float32), dtype)
          for h in (hq, hkv, hkv)]
    bs = ([round_to(rng.standard_normal(h * d).astype(np.float32) * 0.1, dtype) for h in (hq, hkv, hkv)]
          if bias else None)
    dev = lambda a: abi.dev_tensor(a, dtype)
    # x as a strided view (every other position of a longer sequence)
    xw = np.zeros((b, 2 * t, e), np.float32)
    xw[:, ::2] = x
    xd, wd = dev(xw)[:, ::2], [dev(w) for w in ws]
    bd = [dev(z) for z in bs] if bias else None
    cos_h, sin_h = R.tables(pos + t, d)
    cos, sin = dev(round_to(cos_h, dtype)), dev(round_to(sin_h, dtype))
    tdt = xd.dtype

    def run(rope=True, int8=False):
        q = torch.zeros((b, hq, t, d), dtype=tdt, device="cuda")
        if int8:
            kc = torch.zeros((b, hkv, cap, d), dtype=torch.int8, device="cuda")
            vc = torch.zeros_like(kc)
            sc = (torch.ones((b, hkv, cap, 1), dtype=torch.float32, device="cuda"),
                  torch.ones((b, hkv, cap, 1), dtype=torch.float32, device="cuda"))
        else:
            kc = torch.zeros((b, hkv, cap, d), dtype=tdt, device="cuda")
            vc = torch.zeros_like(kc)
            sc = None
        abi.qkv_rope_append(xd, *wd, bd, q, kc, vc, sc, cos if rope else None, sin if rope else None,
                            pos, hq, hkv)
        torch.cuda.synchronize()
        return q, kc, vc, sc

    # oracle projections as the reference's Linear (functional.py:75-77): the
    # product of the rounded operands rounded to the dtype, then + bias
    # rounded again
    heads = lambda y, h: y.reshape(b, t, h, d).transpose(0, 2, 1, 3)
    proj = []
    for i, (w, h) in enumerate(zip(ws, (hq, hkv, hkv))):
        y = round_to((x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32), dtype)
        if bias:
            y = round_to(y.astype(np.float32) + bs[i].astype(np.float32), dtype)
        proj.append(heads(y, h))

    q0, k0, v0, _ = run(rope=False)
    q1, k1, v1, _ = run(rope=True)
    q_pl, k_pl = abi.host(q0), abi.host(k0)[:, :, pos:pos + t]
    _check(q_pl, proj[0], dtype, "q projection")
    _check(k_pl, proj[1], dtype, "k projection")
    _check(abi.host(v0)[:, :, pos:pos + t], proj[2], dtype, "v projection")
    # RoPE bit-exact on the kernel's own projections
    np.testing.assert_array_equal(abi.host(q1), R.rope(q_pl, pos, dtype=dtype))
    np.testing.assert_array_equal(abi.host(k1)[:, :, pos:pos + t], R.rope(k_pl, pos, dtype=dtype))
    np.testing.assert_array_equal(abi.host(v1), abi.host(v0))
    for c in (k1, v1):  # rows outside the append untouched
        assert (c[:, :, :pos] == 0).all() and (c[:, :, pos + t:] == 0).all()
    # int8 caches: the reference quantiser on the kernel's 16-bit rows
    q8, k8, v8, (ks, vs) = run(rope=True, int8=True)
    assert torch.equal(q8, q1)
    for codes, scales, rows in ((k8, ks, k1), (v8, vs, v1)):
        want_q, want_s = A.quantize_int8(abi.host(rows)[:, :, pos:pos + t])
        np.testing.assert_array_equal(abi.host(codes)[:, :, pos:pos + t], want_q)
        np.testing.assert_array_equal(abi.host(scales)[:, :, pos:pos + t], want_s)
        assert (codes[:, :, :pos] == 0).all() and (codes[:, :, pos + t:] == 0).all()
        assert (scales[:, :, :pos] == 1).all() and (scales[:, :, pos + t:] == 1).all()


def test_fused_projection_rejects_bad_arguments():
    x = torch.zeros((1, 1, 64), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((64, 64), dtype=torch.bfloat16, device="cuda")
    q = torch.zeros((1, 1, 1, 64), dtype=torch.bfloat16, device="cuda")
    kc = torch.zeros((1, 1, 4, 64), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(NotImplementedError):  # head dim 32
        abi.qkv_rope_append(x, w, w, w, None, q[..., :32], kc[..., :32], kc[..., :32], None,
                            None, None, 0, 2, 1)
    with pytest.raises(ValueError):  # 3 query heads over 2 KV heads
        abi.qkv_rope_append(x, w, w, w, None, q, kc, kc, None, None, None, 0, 3, 2)


@pytest.mark.parametrize("dtype,quantized", [("bfloat16", False), ("float16", True)])
def test_cached_attention_module_runs_the_fused_kernel(dtype, quantized):
    """MultiHeadAttention with a cache (GQA, RoPE): a prompt then single-token
    steps through the fused projection kernel agree with the same steps taken
    as separate projections, RoPE and append (the fused path switched off),
    at the dtype's output bound; the fused kernel's probe fires once per step."""
    import tensorsmith_hip as ts
    from unittest.mock import patch
    from tensorsmith_hip import nn

    say(f"MHA cached steps through the fused kernel {dtype} quantized={quantized}")
    ts.seed(5)
    mha = nn.MultiHeadAttention(256, 4, num_kv_heads=2, device="hip").eval()
    mha.to(dtype=dtype)
    x = ts.tensor(np.random.default_rng(5).standard_normal((2, 40, 256)).astype(np.float32) * 0.5,
                  device="hip", dtype=dtype)

    def run(fused: bool):
        cache = mha.new_cache(2, 64, dtype=dtype, quantized=quantized)
        outs = []
        _lib.profile_enable(True)
        _lib.profile_reset()
        with ts.no_grad():
            if fused:
                outs.append(mha(x[:, :36], cache=cache))
                for t in range(36, 40):
                    outs.append(mha(x[:, t:t + 1], cache=cache))
            else:
                with patch.object(nn.KVCache, "_project_append", lambda *a, **k: None):
                    outs.append(mha(x[:, :36], cache=cache))
                    for t in range(36, 40):
                        outs.append(mha(x[:, t:t + 1], cache=cache))
        probes = _lib.profile_read()
        _lib.profile_enable(False)
        return np.concatenate([o.numpy().astype(np.float32) for o in outs], axis=1), probes

    got, probes = run(True)
    want, probes_ref = run(False)
    name = "qkv_rope_append_int8" if quantized else "qkv_rope_append"
    assert probes[name][0] == 5 and name not in probes_ref
    l2, mx = BOUND[dtype]
    assert rel_l2(got, want) <= l2
    assert np.abs(got - want).max() <= mx * np.abs(want).max()
