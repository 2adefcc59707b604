"""HIP kernels vs the oracle, through the C ABI (needs an MI355X).

Tolerances (stated here, enforced below):

* fp32 / fp64 (generic kernels; the fp32 MFMA kernels are held to the same
  bound in ``test_gpu_f32.py``): the reference's cross-backend bound
  ``rtol=1e-4, atol=3e-5`` for fp32 (``tests/test_transformer.py:92``);
  ``1e-10`` relative for fp64.
* bf16: relative-L2 <= 1e-2 (O) / 2e-2 (dQ, dK, dV); max-abs <= 2e-2 * max|ref|;
  LSE max-abs <= 1e-3.
* fp16: relative-L2 <= 2e-3 (O) / 5e-3 (grads); max-abs <= 5e-3 * max|ref|;
  LSE max-abs <= 1e-3.

The reference values are the oracle's fp32 math on the same rounded inputs
(what the reference does for half inputs, ``attention.py:63,90-92``).
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover - CPU containers
    pytest.skip("no GPU", allow_module_level=True)

import abi  # noqa: E402
from conftest import golden_kwargs, rel_l2  # noqa: E402
from oracle import attention as A  # noqa: E402
from oracle.halfprec import round_to  # noqa: E402
from oracle.inputs import attention_inputs  # noqa: E402
from tensorsmith_hip import _lib  # noqa: E402

TOL = {
    "bfloat16": dict(o=1e-2, g=2e-2, mx=2e-2),
    "float16": dict(o=2e-3, g=5e-3, mx=5e-3),
}


def say(msg):
    print(msg, flush=True)


def check_half(got, ref, dtype, kind, name):
    t = TOL[dtype]
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = rel_l2(got, ref)
    scale = np.abs(ref).max() or 1.0
    mx = np.abs(got - ref).max() / scale
    floor = rel_l2(round_to(ref.astype(np.float32), dtype), ref)
    say(f"  {name}: rel_l2={err:.2e} (rounding floor {floor:.1e}) max_abs/max|ref|={mx:.2e}")
    assert np.isfinite(got).all(), name
    assert err <= t[kind], f"{name}: rel_l2 {err:.3e} > {t[kind]}"
    assert mx <= t["mx"], f"{name}: max-abs {mx:.3e} > {t['mx']}"


def check_lse(got, ref_lse, name):
    ref = ref_lse[..., 0] if ref_lse.ndim == 4 else ref_lse
    np.testing.assert_array_equal(np.isneginf(got), np.isneginf(ref), err_msg=name)
    live = np.isfinite(ref)
    if live.any():
        err = np.abs(got[live] - ref[live]).max()
        say(f"  {name}: lse max-abs={err:.2e}")
        assert err <= 1e-3, name


# ---------------------------------------------------------------------------
# Generic kernels (fp64 / fp32) against the torch-written golden fixtures
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", ["float64", "float32"])
def test_golden_fixtures_generic(golden, dtype):
    for name, case in golden.items():
        kw, mask = golden_kwargs(case)
        say(f"golden {name} {dtype}")
        q, k, v, g = (abi.dev_tensor(case[x], dtype) for x in ("q", "k", "v", "g"))
        m = None
        if mask is not None:
            m = torch.from_numpy(mask).cuda()
            if m.dtype != torch.bool:
                m = m.to(abi.TORCH_DTYPES[dtype])
        args = dict(causal=kw["is_causal"], offset=kw["causal_offset"], scale=kw.get("scale"),
                    mask=m)
        with abi.generic_only():
            out, lse, path = abi.forward(q, k, v, **args)
            assert path == _lib.PATH_GENERIC
            dq, dk, dv, _ = abi.backward(q, k, v, out, g, lse, **args)
        torch.cuda.synchronize()
        tol = dict(rtol=1e-10, atol=1e-12) if dtype == "float64" else dict(rtol=1e-4, atol=3e-5)
        np.testing.assert_allclose(abi.host(out), case["out"], **tol, err_msg=f"{name} out")
        lse_h = abi.host(lse)
        np.testing.assert_array_equal(np.isneginf(lse_h), np.isneginf(case["lse"]))
        live = np.isfinite(case["lse"])
        np.testing.assert_allclose(lse_h[live], case["lse"][live], **tol)
        for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
            np.testing.assert_allclose(abi.host(got), case[key], **tol, err_msg=f"{name} {key}")


# ---------------------------------------------------------------------------
# MFMA kernels (bf16 / fp16, D = 64 / 128) against the oracle
# ---------------------------------------------------------------------------

MFMA_CASES = [
    # (B, Hq, Hkv, Sq, Sk, D, causal, offset)
    (2, 2, 2, 128, 128, 128, True, 0),
    (1, 3, 3, 300, 300, 128, True, 0),
    (2, 2, 2, 200, 333, 64, True, 133),
    (1, 2, 2, 77, 190, 128, False, 0),
    (1, 4, 2, 160, 160, 64, True, 0),     # GQA
    (2, 2, 1, 65, 257, 128, True, 192),  # GQA + offset + ragged
    (1, 1, 1, 1, 300, 128, True, 299),    # one query row (decode shape through prefill)
    # head dim 32 (the reference's default TransformerConfig: dim 128, 4 heads)
    (2, 2, 2, 200, 333, 32, True, 133),
    (1, 4, 2, 160, 160, 32, True, 0),     # GQA
    (2, 3, 3, 77, 190, 32, False, 0),
]


def _oracle(inp, dtype, causal, offset, mask=None, gqa=False):
    return A.sdpa(inp.q, inp.k, inp.v, mask, causal, dtype=dtype, causal_offset=offset,
                  backend="streaming", enable_gqa=gqa)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("case", MFMA_CASES, ids=lambda c: "x".join(map(str, c)))
def test_mfma_forward_backward(dtype, case):
    b, hq, hkv, sq, sk, d, causal, off = case
    say(f"mfma {dtype} {case}")
    inp = attention_inputs(b, hq, sq, d, dtype, heads_kv=hkv, seq_k=sk, value_scale=0.5, seed=11)
    ref = _oracle(inp, dtype, causal, off, gqa=hkv != hq)
    q, k, v, g = (abi.dev_tensor(x, dtype) for x in (inp.q, inp.k, inp.v, inp.do))
    out, lse, path = abi.forward(q, k, v, causal=causal, offset=off)
    assert path == _lib.PATH_MFMA
    dq, dk, dv, bpath = abi.backward(q, k, v, out, g, lse, causal=causal, offset=off)
    assert bpath == _lib.PATH_MFMA
    torch.cuda.synchronize()
    check_half(abi.host(out), ref.out, dtype, "o", "O")
    check_lse(abi.host(lse), ref.lse, "LSE")
    # the oracle's VJP uses its own fp32 O; the kernels use the returned (rounded) O
    rdq, rdk, rdv = ref.backward_compute(inp.do)
    check_half(abi.host(dq), rdq, dtype, "g", "dQ")
    check_half(abi.host(dk), rdk, dtype, "g", "dK")
    check_half(abi.host(dv), rdv, dtype, "g", "dV")


@pytest.mark.parametrize("case", MFMA_CASES, ids=lambda c: "x".join(map(str, c)))
def test_mfma_backward_both_dq_paths(case):
    """With a 128-wide head the queried workspace holds dS for the one-GEMM
    dQ (row values, dK/dV storing dS, then dQ = scale dS K); a workspace of
    the row values alone runs the dQ kernel that recomputes S and dP, as does
    any workspace at head dims 64 and 32 (the query sizes none there: the
    recomputing backward is the faster one).  Both meet the bounds."""
    b, hq, hkv, sq, sk, d, causal, off = case
    dtype = "bfloat16"
    say(f"mfma backward dQ paths {case}")
    inp = attention_inputs(b, hq, sq, d, dtype, heads_kv=hkv, seq_k=sk, value_scale=0.5, seed=13)
    ref = _oracle(inp, dtype, causal, off, gqa=hkv != hq)
    q, k, v, g = (abi.dev_tensor(x, dtype) for x in (inp.q, inp.k, inp.v, inp.do))
    out, lse, _ = abi.forward(q, k, v, causal=causal, offset=off)
    rdq, rdk, rdv = ref.backward_compute(inp.do)
    rows_bytes = 2 * b * hq * sq * 4
    stored = d == 128
    for ws, dq_probe in ((None, "bwd_dq_ds" if stored else "bwd_dq_mfma"), (rows_bytes, "bwd_dq_mfma")):
        _lib.profile_enable(True)
        _lib.profile_reset()
        dq, dk, dv, bpath = abi.backward(q, k, v, out, g, lse, ws_bytes=ws, causal=causal, offset=off)
        torch.cuda.synchronize()
        probes = _lib.profile_read()
        _lib.profile_enable(False)
        assert bpath == _lib.PATH_MFMA
        assert dq_probe in probes and (ws is None and stored) == ("bwd_rows" in probes), sorted(probes)
        for got, want, n in ((dq, rdq, "dQ"), (dk, rdk, "dK"), (dv, rdv, "dV")):
            check_half(abi.host(got), want, dtype, "g", f"{n} ({dq_probe})")


GENERIC_LAYOUT_CASES = [
    # (name, dtype, B, Hq, Hkv, Sq, Sk, Dqk, Dv, causal, offset, mask, misaligned view)
    # K / V rows on 16-byte boundaries (16-byte row loads), GQA, a last wave
    # whose four query rows run past Sq
    ("f32-gqa-d36x20-rows77", "float32", 2, 4, 2, 77, 130, 36, 20, True, 0, None, False),
    # rows not 16-byte aligned (element loads), an additive mask
    ("f32-d33x17-floatmask", "float32", 1, 2, 2, 70, 90, 33, 17, False, 0, "float", False),
    # views whose base is one element past a 16-byte boundary
    ("f32-d64-misaligned-view", "float32", 1, 2, 2, 100, 100, 64, 64, True, 0, None, True),
    # a Q / dO chunk too large for LDS (the unstaged dK/dV kernel), causal offset
    ("f64-d256-unstaged-boolmask", "float64", 1, 1, 1, 80, 96, 256, 256, True, 16, "bool", False),
]


def _misaligned(t):
    """The same values in a view whose rows start one element past the
    allocation's 16-byte boundaries."""
    pad = torch.zeros(*t.shape[:-1], t.shape[-1] + 1, dtype=t.dtype, device=t.device)
    pad[..., 1:] = t
    return pad[..., 1:]


@pytest.mark.parametrize("case", GENERIC_LAYOUT_CASES, ids=lambda c: c[0])
def test_generic_kernel_layouts_match_oracle(case):
    """The generic kernels' load and staging variants (16-byte or element row
    loads, four query rows per wave with a ragged last wave, the LDS-staged or
    unstaged dK/dV kernel) against the oracle's streaming attention, at the
    fp32 / fp64 bounds above."""
    name, dtype, b, hq, hkv, sq, sk, dqk, dv, causal, off, mkind, mis = case
    say(f"generic layout {name}")
    inp = attention_inputs(b, hq, sq, dqk, dtype, heads_kv=hkv, seq_k=sk, dim_v=dv, seed=13)
    rng = np.random.default_rng(3)
    mask = None
    if mkind == "bool":
        mask = rng.random((sq, sk)) > 0.25
    elif mkind == "float":
        mask = (rng.standard_normal((sq, sk)) * 1.5).astype(np.float32)
    ref = A.sdpa(inp.q, inp.k, inp.v, mask, causal, dtype=dtype, causal_offset=off,
                 backend="streaming", enable_gqa=hkv != hq)
    rdq, rdk, rdv = ref.backward(inp.do)
    q, k, v, g = (abi.dev_tensor(x, dtype) for x in (inp.q, inp.k, inp.v, inp.do))
    if mis:
        q, k, v, g = (_misaligned(t) for t in (q, k, v, g))
    m = None if mask is None else torch.from_numpy(mask).cuda()
    args = dict(causal=causal, offset=off, mask=m)
    with abi.generic_only():
        out, lse, path = abi.forward(q, k, v, **args)
        assert path == _lib.PATH_GENERIC
        dq, dk, dv_, _ = abi.backward(q, k, v, out, g, lse, **args)
    torch.cuda.synchronize()
    tol = dict(rtol=1e-10, atol=1e-12) if dtype == "float64" else dict(rtol=1e-4, atol=3e-5)
    np.testing.assert_allclose(abi.host(out), ref.out_cast, **tol, err_msg=f"{name} out")
    want_lse = ref.lse[..., 0]
    got_lse = abi.host(lse)
    np.testing.assert_array_equal(np.isneginf(got_lse), np.isneginf(want_lse))
    live = np.isfinite(want_lse)
    np.testing.assert_allclose(got_lse[live], want_lse[live], **tol, err_msg=f"{name} lse")
    for got, want, key in ((dq, rdq, "dq"), (dk, rdk, "dk"), (dv_, rdv, "dv")):
        np.testing.assert_allclose(abi.host(got), want, **tol, err_msg=f"{name} {key}")


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_mfma_agrees_with_generic_on_same_inputs(dtype):
    inp = attention_inputs(2, 2, 190, 128, dtype, value_scale=0.5, seed=5)
    q, k, v, g = (abi.dev_tensor(x, dtype) for x in (inp.q, inp.k, inp.v, inp.do))
    say(f"mfma vs generic {dtype}")
    out_m, lse_m, _ = abi.forward(q, k, v, causal=True)
    dq_m, dk_m, dv_m, _ = abi.backward(q, k, v, out_m, g, lse_m, causal=True)
    with abi.generic_only():
        out_g, lse_g, path = abi.forward(q, k, v, causal=True)
        assert path == _lib.PATH_GENERIC
        dq_g, dk_g, dv_g, _ = abi.backward(q, k, v, out_m, g, lse_m, causal=True)
    torch.cuda.synchronize()
    check_half(abi.host(out_m), abi.host(out_g), dtype, "o", "O mfma/generic")
    check_lse(abi.host(lse_m), abi.host(lse_g), "LSE mfma/generic")
    for a_, b_, n in ((dq_m, dq_g, "dQ"), (dk_m, dk_g, "dK"), (dv_m, dv_g, "dV")):
        check_half(abi.host(a_), abi.host(b_), dtype, "g", n + " mfma/generic")


@pytest.mark.parametrize("prefix", [True, False])
def test_mfma_key_padding_mask(prefix):
    dtype = "bfloat16"
    b, h, s, d = 3, 2, 200, 128
    inp = attention_inputs(b, h, s, d, dtype, value_scale=0.5, seed=9)
    lengths = np.array([200, 131, 64])
    keymask = np.arange(s)[None, :] < lengths[:, None]
    if not prefix:
        keymask[1, 17] = False  # a hole inside the valid prefix
        keymask[2, 150] = True  # an allowed key past the padding
    mask4 = keymask[:, None, None, :]
    say(f"key mask prefix={prefix}")
    ref = A.sdpa(inp.q, inp.k, inp.v, mask4, True, dtype=dtype, backend="streaming")
    q, k, v, g = (abi.dev_tensor(x, dtype) for x in (inp.q, inp.k, inp.v, inp.do))
    km = torch.from_numpy(keymask).cuda()
    kv_len, kv_prefix = abi.key_lengths(km)
    torch.cuda.synchronize()
    last = np.array([np.nonzero(r)[0].max() + 1 for r in keymask])
    np.testing.assert_array_equal(kv_len.cpu().numpy(), last)
    np.testing.assert_array_equal(kv_prefix.cpu().numpy(),
                                  [int(r[:l].all()) for r, l in zip(keymask, last)])
    m4 = km[:, None, None, :]
    out, lse, path = abi.forward(q, k, v, causal=True, mask=m4, kv_len=kv_len, kv_prefix=kv_prefix)
    assert path == _lib.PATH_MFMA
    dq, dk, dv, _ = abi.backward(q, k, v, out, g, lse, causal=True, mask=m4, kv_len=kv_len,
                                 kv_prefix=kv_prefix)
    torch.cuda.synchronize()
    check_half(abi.host(out), ref.out, dtype, "o", "O")
    check_lse(abi.host(lse), ref.lse, "LSE")
    for got, want, n in zip((dq, dk, dv), ref.backward_compute(inp.do), ("dQ", "dK", "dV")):
        check_half(abi.host(got), want, dtype, "g", n)


# General masks on the MFMA kernels: boolean masks of any broadcast shape
# (read per row and key) and additive masks in f32 / f16 / bf16, with causal
# windows, offsets, GQA and fully masked rows (O = 0, LSE = -inf, zero grads).
MASK_CASES = [
    # (id, dtype, B, Hq, Hkv, Sq, Sk, D, causal, offset, mask shape, mask dtype)
    ("bool-qk-causal", "bfloat16", 2, 2, 2, 200, 333, 128, True, 133, (200, 333), "bool"),
    ("bool-b1qk-gqa", "float16", 2, 4, 2, 160, 190, 64, False, 0, (2, 1, 160, 190), "bool"),
    ("bool-1h1k", "bfloat16", 2, 3, 3, 129, 257, 128, False, 0, (1, 3, 1, 257), "bool"),
    ("add-f32-1hqk-causal", "float16", 1, 2, 2, 300, 300, 128, True, 0, (1, 2, 300, 300), "float32"),
    ("add-bf16-qk", "bfloat16", 2, 2, 1, 77, 150, 64, True, 73, (77, 150), "bfloat16"),
    ("add-f16-keybias", "float16", 3, 2, 2, 96, 200, 128, False, 0, (3, 1, 1, 200), "float16"),
    # rows 16-byte aligned, keys contiguous: the 16-byte row-piece reads
    ("bool-qk-rows", "bfloat16", 2, 2, 2, 160, 256, 128, True, 96, (160, 256), "bool"),
    ("add-bf16-rows", "float16", 1, 4, 2, 128, 192, 64, False, 0, (128, 192), "bfloat16"),
    ("bool-qk-d32", "bfloat16", 2, 2, 2, 200, 333, 32, True, 133, (200, 333), "bool"),
    ("add-f32-rows-d32", "float16", 1, 2, 1, 160, 256, 32, False, 0, (1, 2, 160, 256), "float32"),
]


def _mask(rng, shape, mdtype, sq):
    if mdtype == "bool":
        m = rng.random(shape) > 0.3
        if len(shape) >= 2 and shape[-2] == sq:
            m[..., 5, :] = False  # a fully masked query row
        return m
    m = (rng.standard_normal(shape) * 1.5).astype(np.float32)
    m[rng.random(shape) < 0.2] = -np.inf
    if len(shape) >= 2 and shape[-2] == sq:
        m[..., 7, :] = -np.inf  # a fully masked query row
    return round_to(m, mdtype)


@pytest.mark.parametrize("case", MASK_CASES, ids=lambda c: c[0])
def test_mfma_general_masks(case):
    _, dtype, b, hq, hkv, sq, sk, d, causal, off, mshape, mdtype = case
    say(f"mfma general mask {case}")
    inp = attention_inputs(b, hq, sq, d, dtype, heads_kv=hkv, seq_k=sk, value_scale=0.5, seed=21)
    rng = np.random.default_rng(sq + sk)
    mask = _mask(rng, mshape, mdtype, sq)
    ref = _oracle(inp, dtype, causal, off, mask=mask, gqa=hkv != hq)
    q, k, v, g = (abi.dev_tensor(x, dtype) for x in (inp.q, inp.k, inp.v, inp.do))
    tm = (torch.from_numpy(mask).cuda() if mdtype == "bool"
          else abi.dev_tensor(mask, mdtype))
    _lib.profile_enable(True)
    _lib.profile_reset()
    out, lse, path = abi.forward(q, k, v, causal=causal, offset=off, mask=tm)
    assert path == _lib.PATH_MFMA
    dq, dk, dv, bpath = abi.backward(q, k, v, out, g, lse, causal=causal, offset=off, mask=tm)
    assert bpath == _lib.PATH_MFMA
    torch.cuda.synchronize()
    probes = _lib.profile_read()
    _lib.profile_enable(False)
    dq_probe = "bwd_dq_ds_masked" if d == 128 else "bwd_dq_mfma_masked"  # stored dS at D = 128 only
    assert {"fwd_mfma_masked", dq_probe, "bwd_dkdv_mfma_masked"} <= set(probes), sorted(probes)
    check_half(abi.host(out), ref.out, dtype, "o", "O")
    check_lse(abi.host(lse), ref.lse, "LSE")
    rdq, rdk, rdv = ref.backward_compute(inp.do)
    check_half(abi.host(dq), rdq, dtype, "g", "dQ")
    check_half(abi.host(dk), rdk, dtype, "g", "dK")
    check_half(abi.host(dv), rdv, dtype, "g", "dV")
    if mshape[-2] == sq:  # the fully masked row: O = 0, LSE = -inf, dQ = 0
        row = 5 if mdtype == "bool" else 7
        assert (abi.host(out)[:, :, row] == 0).all()
        assert np.isneginf(abi.host(lse)[:, :, row]).all()
        assert (abi.host(dq)[:, :, row] == 0).all()


@pytest.mark.parametrize("case", MASK_CASES, ids=lambda c: c[0])
def test_mfma_general_masks_recomputing_dq(case):
    """A workspace of the row values alone (no room for stored dS) runs the
    masked dQ kernel that recomputes S and dP per key tile, then dK/dV: the
    only backward for a caller that passes a rows-only workspace."""
    _, dtype, b, hq, hkv, sq, sk, d, causal, off, mshape, mdtype = case
    say(f"mfma general mask, recomputing dQ {case}")
    inp = attention_inputs(b, hq, sq, d, dtype, heads_kv=hkv, seq_k=sk, value_scale=0.5, seed=23)
    rng = np.random.default_rng(sq + 2 * sk)
    mask = _mask(rng, mshape, mdtype, sq)
    ref = _oracle(inp, dtype, causal, off, mask=mask, gqa=hkv != hq)
    q, k, v, g = (abi.dev_tensor(x, dtype) for x in (inp.q, inp.k, inp.v, inp.do))
    tm = (torch.from_numpy(mask).cuda() if mdtype == "bool"
          else abi.dev_tensor(mask, mdtype))
    out, lse, _ = abi.forward(q, k, v, causal=causal, offset=off, mask=tm)
    rows_bytes = 2 * b * hq * sq * 4
    _lib.profile_enable(True)
    _lib.profile_reset()
    dq, dk, dv, bpath = abi.backward(q, k, v, out, g, lse, ws_bytes=rows_bytes, causal=causal,
                                     offset=off, mask=tm)
    torch.cuda.synchronize()
    probes = _lib.profile_read()
    _lib.profile_enable(False)
    assert bpath == _lib.PATH_MFMA
    assert {"bwd_dq_mfma_masked", "bwd_dkdv_mfma_masked"} <= set(probes), sorted(probes)
    assert "bwd_dq_ds_masked" not in probes and "bwd_rows" not in probes, sorted(probes)
    rdq, rdk, rdv = ref.backward_compute(inp.do)
    check_half(abi.host(dq), rdq, dtype, "g", "dQ")
    check_half(abi.host(dk), rdk, dtype, "g", "dK")
    check_half(abi.host(dv), rdv, dtype, "g", "dV")
    if mshape[-2] == sq:
        row = 5 if mdtype == "bool" else 7
        assert (abi.host(dq)[:, :, row] == 0).all()


def test_mfma_key_mask_without_lengths_reads_the_mask():
    """A [B,1,1,K] boolean mask passed without kv_len runs the general-mask
    kernels and agrees with the length-reduced path."""
    dtype = "bfloat16"
    inp = attention_inputs(2, 2, 150, 128, dtype, value_scale=0.5, seed=4)
    keymask = np.ones((2, 150), dtype=bool)
    keymask[0, 100:] = False
    keymask[1, [3, 77, 149]] = False
    q, k, v, g = (abi.dev_tensor(x, dtype) for x in (inp.q, inp.k, inp.v, inp.do))
    km = torch.from_numpy(keymask).cuda()
    m4 = km[:, None, None, :]
    out_g, lse_g, _ = abi.forward(q, k, v, causal=True, mask=m4)
    grads_g = abi.backward(q, k, v, out_g, g, lse_g, causal=True, mask=m4)[:3]
    kv_len, kv_prefix = abi.key_lengths(km)
    out_l, lse_l, _ = abi.forward(q, k, v, causal=True, mask=m4, kv_len=kv_len, kv_prefix=kv_prefix)
    grads_l = abi.backward(q, k, v, out_l, g, lse_l, causal=True, mask=m4, kv_len=kv_len,
                           kv_prefix=kv_prefix)[:3]
    torch.cuda.synchronize()
    # same tiles, same arithmetic on every allowed score: identical results
    assert torch.equal(out_g, out_l) and torch.equal(lse_g, lse_l)
    for a_, b_ in zip(grads_g, grads_l):
        assert torch.equal(a_, b_)


# Value head dim != query/key head dim on the MFMA kernels (the reference's
# value_dim, tests/test_transformer.py:44-46): tiles and accumulators sized per
# operand, with GQA, causal offsets and a general mask.
VALUE_DIM_CASES = [
    # (dtype, B, Hq, Hkv, Sq, Sk, Dqk, Dv, causal, offset, masked)
    ("bfloat16", 2, 2, 2, 200, 333, 128, 64, True, 133, False),
    ("float16", 1, 4, 2, 160, 160, 64, 128, True, 0, False),
    ("bfloat16", 2, 2, 1, 77, 190, 128, 64, False, 0, True),
    ("float16", 1, 2, 2, 129, 257, 64, 128, False, 0, True),
]


@pytest.mark.parametrize("case", VALUE_DIM_CASES, ids=lambda c: "-".join(map(str, c)))
def test_mfma_value_dim_differs(case):
    dtype, b, hq, hkv, sq, sk, dqk, dv, causal, off, masked = case
    say(f"mfma Dqk {dqk} Dv {dv} {case}")
    inp = attention_inputs(b, hq, sq, dqk, dtype, heads_kv=hkv, seq_k=sk, dim_v=dv,
                           value_scale=0.5, seed=17)
    mask = np.random.default_rng(3).random((sq, sk)) > 0.2 if masked else None
    ref = _oracle(inp, dtype, causal, off, mask=mask, gqa=hkv != hq)
    q, k, v, g = (abi.dev_tensor(x, dtype) for x in (inp.q, inp.k, inp.v, inp.do))
    kw = dict(causal=causal, offset=off, mask=None if mask is None else torch.from_numpy(mask).cuda())
    out, lse, path = abi.forward(q, k, v, **kw)
    assert path == _lib.PATH_MFMA
    dq, dk, dv_, bpath = abi.backward(q, k, v, out, g, lse, **kw)
    assert bpath == _lib.PATH_MFMA
    torch.cuda.synchronize()
    check_half(abi.host(out), ref.out, dtype, "o", "O")
    check_lse(abi.host(lse), ref.lse, "LSE")
    rdq, rdk, rdv = ref.backward_compute(inp.do)
    check_half(abi.host(dq), rdq, dtype, "g", "dQ")
    check_half(abi.host(dk), rdk, dtype, "g", "dK")
    check_half(abi.host(dv_), rdv, dtype, "g", "dV")


def test_mfma_value_dim_differs_agrees_with_generic():
    dtype = "bfloat16"
    inp = attention_inputs(1, 2, 150, 64, dtype, seq_k=150, dim_v=128, value_scale=0.5, seed=2)
    q, k, v, g = (abi.dev_tensor(x, dtype) for x in (inp.q, inp.k, inp.v, inp.do))
    out_m, lse_m, path = abi.forward(q, k, v, causal=True)
    assert path == _lib.PATH_MFMA
    grads_m = abi.backward(q, k, v, out_m, g, lse_m, causal=True)[:3]
    with abi.generic_only():
        out_g, lse_g, _ = abi.forward(q, k, v, causal=True)
        grads_g = abi.backward(q, k, v, out_m, g, lse_m, causal=True)[:3]
    torch.cuda.synchronize()
    check_half(abi.host(out_m), abi.host(out_g), dtype, "o", "O mfma/generic")
    for a_, b_, n in zip(grads_m, grads_g, ("dQ", "dK", "dV")):
        check_half(abi.host(a_), abi.host(b_), dtype, "g", n + " mfma/generic")


# ---------------------------------------------------------------------------
# Decode kernel
# ---------------------------------------------------------------------------

DECODE_CASES = [
    # (B, Hq, Hkv, Sq, cap, D, lengths)
    (4, 4, 4, 1, 1000, 128, [1000, 517, 3, 880]),
    (2, 8, 2, 1, 700, 64, [700, 129]),      # GQA 4 rows per kv head
    (2, 4, 4, 2, 600, 128, [600, 400]),     # two new tokens (causal)
    (1, 2, 2, 1, 2048, 256, [2048]),
]


def check_decode(got, ref, dtype, name):
    """fp32: the fp32 bound (every product and sum in fp32); 16-bit: check_half."""
    if dtype == "float32":
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=3e-5, err_msg=name)
    else:
        check_half(got, ref, dtype, "o", name)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32"])
@pytest.mark.parametrize("case", DECODE_CASES, ids=lambda c: f"b{c[0]}h{c[1]}kv{c[2]}q{c[3]}d{c[5]}")
def test_decode_matches_oracle(dtype, case):
    b, hq, hkv, sq, cap, d, lengths = case
    say(f"decode {dtype} {case[:6]}")
    inp = attention_inputs(b, hq, sq, d, dtype, heads_kv=hkv, seq_k=cap, with_grad=False, seed=3)
    lengths = np.array(lengths)
    # query rows sit at the end of each sequence: causal offset = len - sq
    q, k, v = (abi.dev_tensor(x, dtype) for x in (inp.q, inp.k, inp.v))
    kv_len = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    offset = int(lengths.max()) - sq
    for split in (0, 64, 256):
        out = abi.decode(q, k, v, split_len=split, causal=True, offset=offset, kv_len=kv_len)
        torch.cuda.synchronize()
        assert _lib.last_kernel_path() == _lib.PATH_DECODE
        got = abi.host(out)
        for bi in range(b):
            ref = A.sdpa(inp.q[bi:bi + 1], inp.k[bi:bi + 1, :, :lengths[bi]],
                         inp.v[bi:bi + 1, :, :lengths[bi]], None, True, dtype=dtype,
                         causal_offset=offset, backend="dense", enable_gqa=hkv != hq)
            check_decode(got[bi:bi + 1], ref.out, dtype, f"b{bi} split{split}")


@pytest.mark.parametrize("dtype", ["float16", "float32"])
def test_decode_with_bool_mask_and_float_mask(dtype):
    inp = attention_inputs(2, 2, 1, 128, dtype, seq_k=300, with_grad=False, seed=4)
    q, k, v = (abi.dev_tensor(x, dtype) for x in (inp.q, inp.k, inp.v))
    rng = np.random.default_rng(0)
    bmask = rng.random((2, 1, 1, 300)) > 0.3
    fmask = (rng.standard_normal((1, 2, 1, 300)) * 0.5).astype(np.float32)
    for mask in (bmask, fmask):
        say(f"decode mask {mask.dtype}")
        out = abi.decode(q, k, v, mask=torch.from_numpy(mask).cuda())
        torch.cuda.synchronize()
        ref = A.sdpa(inp.q, inp.k, inp.v, mask, False, dtype=dtype, backend="dense")
        check_decode(abi.host(out), ref.out, dtype, f"mask {mask.dtype}")


# ---------------------------------------------------------------------------
# Error paths forced from the host (no kernel ever faults)
# ---------------------------------------------------------------------------


def test_abi_rejects_bad_arguments_before_launch():
    q = torch.zeros(1, 2, 4, 8, device="cuda")
    p = abi.problem(q, q, q)
    p.heads_kv = 3  # 2 % 3 != 0
    out = torch.empty_like(q)
    lib = _lib.load()
    rc = lib.tsattn_sdpa_forward(abi.ctypes.byref(p), abi.view(q), abi.view(q), abi.view(q),
                                 abi.view(out), None, abi.stream())
    assert rc == _lib.ERR_INVALID and "divisible" in _lib.last_error()
    p = abi.problem(q, q, q)
    p.scale = float("inf")
    rc = lib.tsattn_sdpa_forward(abi.ctypes.byref(p), abi.view(q), abi.view(q), abi.view(q),
                                 abi.view(out), None, abi.stream())
    assert rc == _lib.ERR_INVALID and "finite" in _lib.last_error()
    bad = abi.view(q)
    bad.stride[3] = 2
    p = abi.problem(q, q, q)
    rc = lib.tsattn_sdpa_forward(abi.ctypes.byref(p), bad, abi.view(q), abi.view(q),
                                 abi.view(out), None, abi.stream())
    assert rc == _lib.ERR_INVALID
