"""fp32 attention on the matrix cores (v_mfma_f32_32x32x2_f32) against the oracle.

The fp32 kernels compute every product and sum in fp32, as the reference's
fp32 path does (``attention.py:63``).  They are held to the reference's
cross-backend fp32 bound ``rtol=1e-4, atol=3e-5`` (``tests/test_transformer.py:92``)
against the oracle's streaming attention, on O, the LSE, dQ, dK and dV.
Head dims 32 / 64 / 128 with equal value dim, no mask or a [B,1,1,K] boolean
key mask, no dropout and no fused rotation take these kernels; the rest stays
on the generic kernels (checked below).
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover - CPU containers
    pytest.skip("no GPU", allow_module_level=True)

import abi  # noqa: E402
from oracle import attention as A  # noqa: E402
from oracle.inputs import attention_inputs  # noqa: E402
from tensorsmith_hip import _lib  # noqa: E402

TOL = dict(rtol=1e-4, atol=3e-5)
DT = "float32"


def expected_probes(b, hq, hkv, sq, sk, d):
    """The kernels a problem runs: at head dims <= 64 a problem with fewer
    128-row (128-key) blocks than the device has CUs runs the split form of
    the forward / dQ (dK/dV) kernel, 32 rows (keys) per workgroup."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sq_split = d <= 64 and -(-sq // 128) * hq * b < cus
    sk_split = d <= 64 and -(-sk // 128) * hkv * b < cus
    sfx = lambda on: "_split" if on else ""
    return ("fwd_mfma_f32" + sfx(sq_split), "bwd_rows_f32", "bwd_dq_mfma_f32" + sfx(sq_split),
            "bwd_dkdv_mfma_f32" + sfx(sk_split))


def say(msg):
    print(msg, flush=True)


F32_CASES = [
    # (B, Hq, Hkv, Sq, Sk, D, causal, offset)
    (8, 4, 4, 256, 256, 64, True, 0),     # the reference's CPU-runnable benchmark shape
    (1, 3, 3, 300, 300, 128, True, 0),
    (2, 2, 2, 200, 333, 64, True, 133),
    (1, 2, 2, 77, 190, 128, False, 0),
    (1, 4, 2, 160, 160, 64, True, 0),     # GQA
    (2, 2, 1, 65, 257, 128, True, 192),   # GQA + offset + ragged
    (1, 1, 1, 1, 300, 128, True, 299),    # one query row
    (2, 2, 2, 200, 333, 32, True, 133),
    (1, 4, 2, 160, 160, 32, True, 0),     # GQA
    (2, 3, 3, 77, 190, 32, False, 0),
    (1, 2, 2, 513, 513, 128, True, 0),    # several key blocks per query block and back
    # enough 128-row blocks for the one-block-per-wave kernels at D = 64 / 32
    (4, 16, 16, 512, 512, 64, True, 0),
    (4, 16, 8, 520, 520, 32, True, 0),    # GQA, ragged: split dK/dV, whole dQ
    (2, 32, 32, 600, 600, 64, False, 0),
    (2, 16, 16, 64, 1100, 64, True, 1036),  # split dQ, whole dK/dV
]


def _check(name, out, lse, grads, ref, do):
    np.testing.assert_allclose(abi.host(out), ref.out_cast, **TOL, err_msg=f"{name} out")
    want = ref.lse[..., 0]
    got = abi.host(lse)
    np.testing.assert_array_equal(np.isneginf(got), np.isneginf(want), err_msg=f"{name} lse")
    live = np.isfinite(want)
    np.testing.assert_allclose(got[live], want[live], **TOL, err_msg=f"{name} lse")
    for g, w, key in zip(grads, ref.backward(do), ("dq", "dk", "dv")):
        h = abi.host(g)
        err = np.abs(h - w).max()
        say(f"  {name} {key}: max-abs {err:.2e}")
        np.testing.assert_allclose(h, w, **TOL, err_msg=f"{name} {key}")


@pytest.mark.parametrize("case", F32_CASES, ids=lambda c: "x".join(map(str, c)))
def test_f32_mfma_forward_backward(case):
    b, hq, hkv, sq, sk, d, causal, off = case
    name = "x".join(map(str, case))
    say(f"f32 mfma {name}")
    inp = attention_inputs(b, hq, sq, d, DT, heads_kv=hkv, seq_k=sk, seed=17)
    ref = A.sdpa(inp.q, inp.k, inp.v, None, causal, dtype=DT, causal_offset=off,
                 backend="streaming", enable_gqa=hkv != hq)
    q, k, v, g = (abi.dev_tensor(x, DT) for x in (inp.q, inp.k, inp.v, inp.do))
    _lib.profile_enable(True)
    _lib.profile_reset()
    try:
        out, lse, path = abi.forward(q, k, v, causal=causal, offset=off)
        dq, dk, dv, bpath = abi.backward(q, k, v, out, g, lse, causal=causal, offset=off)
        torch.cuda.synchronize()
        probes = _lib.profile_read()
    finally:
        _lib.profile_enable(False)
    assert path == _lib.PATH_MFMA and bpath == _lib.PATH_MFMA
    want = expected_probes(b, hq, hkv, sq, sk, d)
    assert all(p in probes for p in want), (want, sorted(probes))
    _check(name, out, lse, (dq, dk, dv), ref, inp.do)


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("prefix", [True, False, "empty"])
def test_f32_mfma_key_padding_mask(prefix, d):
    b, h, s = 3, 2, 200
    inp = attention_inputs(b, h, s, d, DT, seed=9)
    lengths = np.array([200, 131, 0 if prefix == "empty" else 64])
    keymask = np.arange(s)[None, :] < lengths[:, None]
    if prefix is False:
        keymask[1, 17] = False  # a hole inside the valid prefix
        keymask[2, 150] = True  # an allowed key past the padding
    # "empty": batch 2 sees no key at all (O = 0, LSE = -inf, zero gradients)
    say(f"f32 key mask prefix={prefix} d={d}")
    ref = A.sdpa(inp.q, inp.k, inp.v, keymask[:, None, None, :], True, dtype=DT,
                 backend="streaming")
    q, k, v, g = (abi.dev_tensor(x, DT) for x in (inp.q, inp.k, inp.v, inp.do))
    km = torch.from_numpy(keymask).cuda()
    kv_len, kv_prefix = abi.key_lengths(km)
    m4 = km[:, None, None, :]
    kw = dict(causal=True, mask=m4, kv_len=kv_len, kv_prefix=kv_prefix)
    out, lse, path = abi.forward(q, k, v, **kw)
    dq, dk, dv, bpath = abi.backward(q, k, v, out, g, lse, **kw)
    torch.cuda.synchronize()
    assert path == _lib.PATH_MFMA and bpath == _lib.PATH_MFMA
    _check(f"keymask prefix={prefix}", out, lse, (dq, dk, dv), ref, inp.do)


def test_f32_mfma_agrees_with_generic():
    """Same inputs through both fp32 kernel families: they agree to the fp32
    bound with each other, as each does with the oracle."""
    inp = attention_inputs(2, 4, 190, 64, DT, heads_kv=2, seed=5)
    q, k, v, g = (abi.dev_tensor(x, DT) for x in (inp.q, inp.k, inp.v, inp.do))
    out_m, lse_m, path = abi.forward(q, k, v, causal=True)
    assert path == _lib.PATH_MFMA
    grads_m = abi.backward(q, k, v, out_m, g, lse_m, causal=True)[:3]
    with abi.generic_only():
        out_g, lse_g, path = abi.forward(q, k, v, causal=True)
        assert path == _lib.PATH_GENERIC
        grads_g = abi.backward(q, k, v, out_m, g, lse_m, causal=True)[:3]
    torch.cuda.synchronize()
    np.testing.assert_allclose(abi.host(out_m), abi.host(out_g), **TOL)
    np.testing.assert_allclose(abi.host(lse_m), abi.host(lse_g), **TOL)
    for a_, b_, n in zip(grads_m, grads_g, ("dq", "dk", "dv")):
        np.testing.assert_allclose(abi.host(a_), abi.host(b_), **TOL, err_msg=n)


def test_f32_outside_the_mfma_kernels_runs_generic():
    """Head dim 48, a float mask or unequal value dim leave the fp32 MFMA
    kernels; they still meet the bound on the generic ones."""
    rng = np.random.default_rng(2)
    for name, d, dv_, fmask in (("d48", 48, 48, False), ("float mask", 64, 64, True),
                                ("dv differs", 64, 32, False)):
        inp = attention_inputs(1, 2, 96, d, DT, dim_v=dv_, seed=3)
        mask = (rng.standard_normal((96, 96)) * 1.5).astype(np.float32) if fmask else None
        ref = A.sdpa(inp.q, inp.k, inp.v, mask, True, dtype=DT, backend="streaming")
        q, k, v, g = (abi.dev_tensor(x, DT) for x in (inp.q, inp.k, inp.v, inp.do))
        m = None if mask is None else torch.from_numpy(mask).cuda()
        out, lse, path = abi.forward(q, k, v, causal=True, mask=m)
        dq, dk, dv, bpath = abi.backward(q, k, v, out, g, lse, causal=True, mask=m)
        torch.cuda.synchronize()
        assert path == _lib.PATH_GENERIC and bpath == _lib.PATH_GENERIC, name
        _check(name, out, lse, (dq, dk, dv), ref, inp.do)
