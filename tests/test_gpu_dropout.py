"""Attention dropout on the MFMA kernels (needs an MI355X).

The reference drops probabilities in its dense backend
(src/tensorsmith/nn/attention.py:140-144, VJP :210-217) with uniforms from its
global stream; the hip kernels regenerate a counter-based Philox4x32-10 mask
(oracle/dropout.py states the element mapping and is pinned against the
generator's published known-answer vectors).  Checked here:

* the keep mask the kernels draw (tsattn_dropout_keep) equals the oracle's
  bit for bit -- ragged key lengths (rows padded to 16 words), GQA heads,
  counters that carry past 2^64;
* forward and backward with dropout against the oracle's dense dropout
  attention under that same mask, at the bf16 / fp16 bounds of the parity
  tests (relative L2 1e-2 / 2e-3 for O, 2e-2 / 5e-3 for gradients; max-abs
  2e-2 / 5e-3 of max|ref|), with causal windows, offsets, GQA and a general
  mask;
* the generic kernels (fp32 / fp64 / other head dims) drop with the same
  mask, at the reference's fp32 cross-backend bound (rtol 1e-4, atol 3e-5,
  tests/test_transformer.py:92) and 1e-10 for fp64;
* the keep bits a dropping forward writes for its backward (the MFMA forward
  for every tile it computes, the generic path for all) are that mask
  packed; a backward that gets no bits draws the same ones into its
  workspace, and both give the same gradients bit for bit;
* p at the top of the 16-bit threshold range (threshold 65535, and 65536,
  which keeps nothing) gives the oracle's bits, outputs and gradients;
* the same key and counter reproduce every output bit; another key changes
  them; the mirror drops on backend "hip" / "dense" / "auto" and raises the
  reference's ValueError on "streaming" (tests/test_transformer.py:164-171).
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
from conftest import rel_l2  # noqa: E402
from oracle import dropout as DR  # noqa: E402
from oracle.inputs import attention_inputs  # noqa: E402
from tensorsmith_hip import _lib, nn  # noqa: E402

TOL = {"bfloat16": dict(o=1e-2, g=2e-2, mx=2e-2), "float16": dict(o=2e-3, g=5e-3, mx=5e-3)}


def say(msg):
    print(msg, flush=True)


def check(got, ref, dtype, kind, name):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = rel_l2(got, ref)
    mx = np.abs(got - ref).max() / (np.abs(ref).max() or 1.0)
    say(f"  {name}: rel_l2={err:.2e} max_abs/max|ref|={mx:.2e}")
    assert np.isfinite(got).all(), name
    assert err <= TOL[dtype][kind], f"{name}: rel_l2 {err:.3e}"
    assert mx <= TOL[dtype]["mx"], f"{name}: max-abs {mx:.3e}"


@pytest.mark.parametrize("shape,key,counter,p", [
    ((2, 3, 37, 50), 12345, 0, 0.3),
    ((1, 4, 128, 256), 2**127 + 99, 2**64 - 2, 0.1),
    ((2, 2, 5, 16), 7, 3, 0.9),
])
def test_keep_mask_is_the_oracles(shape, key, counter, p):
    b, h, sq, sk = shape
    q = torch.zeros((b, h, sq, 64), dtype=torch.bfloat16, device="cuda")
    kv = torch.zeros((b, 1, sk, 64), dtype=torch.bfloat16, device="cuda")
    got = abi.dropout_keep(q, kv, kv, dropout=(p, key, counter)).cpu().numpy().astype(bool)
    want = DR.keep_mask(key, counter, shape, p)
    np.testing.assert_array_equal(got, want)


def packed_bits(keep):
    """The tsattn_problem.dropout_bits words of a [B, H, Sq, Sk] keep mask:
    [B, H, ceil(Sk / 32), round_up(Sq, 4)] int32, bit j = key 32 t + j."""
    b, h, sq, sk = keep.shape
    nkt, sqp = -(-sk // 32), -(-sq // 4) * 4
    padded = np.zeros((b, h, sqp, nkt * 32), dtype=np.uint64)
    padded[:, :, :sq, :sk] = keep
    tiles = padded.reshape(b, h, sqp, nkt, 32)
    words = (tiles << np.arange(32, dtype=np.uint64)).sum(axis=-1)
    return words.astype(np.uint32).view(np.int32).transpose(0, 1, 3, 2)


def key_bits_valid(sk):
    """Per key tile, the bits of keys below Sk."""
    nkt = -(-sk // 32)
    valid = np.zeros(nkt, dtype=np.uint64)
    for t in range(nkt):
        n = min(32, sk - 32 * t)
        valid[t] = (1 << n) - 1
    return valid.astype(np.uint32).view(np.int32)


CASES = [
    # (dtype, B, Hq, Hkv, Sq, Sk, D, causal, offset, p, masked); D may be (Dqk, Dv)
    ("bfloat16", 2, 2, 2, 130, 130, 128, True, 0, 0.2, False),
    ("float16", 1, 4, 2, 96, 200, 64, True, 104, 0.5, False),
    ("bfloat16", 2, 2, 1, 77, 150, 128, False, 0, 0.1, True),
    ("float16", 1, 2, 2, 256, 256, 128, False, 0, 0.3, False),
    ("bfloat16", 1, 2, 2, 100, 140, (128, 64), True, 40, 0.25, False),
    ("float16", 2, 2, 1, 130, 170, 32, True, 0, 0.2, True),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(map(str, c)))
def test_dropout_attention_matches_oracle(case):
    dtype, b, hq, hkv, sq, sk, d, causal, off, p, masked = case
    say(f"dropout attention {case}")
    d, dv = d if isinstance(d, tuple) else (d, d)
    inp = attention_inputs(b, hq, sq, d, dtype, heads_kv=hkv, seq_k=sk, dim_v=dv, value_scale=0.5,
                           seed=31)
    key, counter = 0x5EED_0000_0000_0000_1234_5678_9ABC_DEF0, 11
    mask = np.random.default_rng(1).random((sq, sk)) > 0.25 if masked else None
    out_c, ref_out, back = DR.sdpa_dropout(inp.q, inp.k, inp.v, mask, causal, dtype=dtype, p=p,
                                           rng_key=key, rng_counter=counter,
                                           causal_offset=off, enable_gqa=hkv != hq)
    q, k, v, g = (abi.dev_tensor(x, dtype) for x in (inp.q, inp.k, inp.v, inp.do))
    kw = dict(causal=causal, offset=off, dropout=(p, key, counter),
              mask=None if mask is None else torch.from_numpy(mask).cuda())
    bits = abi.dropout_bits_buffer(q, k, v, **kw)
    out, lse, path = abi.forward(q, k, v, dropout_bits=bits, **kw)
    assert path == _lib.PATH_MFMA
    # a forward given no bits buffer (its per-tile bit stores then fall
    # outside an empty range) computes the same output and LSE
    out_nb, lse_nb, _ = abi.forward(q, k, v, **kw)
    assert torch.equal(out_nb, out) and torch.equal(lse_nb, lse)
    dq, dk, dv, _ = abi.backward(q, k, v, out, g, lse, dropout_bits=bits, **kw)
    # without the forward's bits the backward draws them itself: same gradients
    _lib.profile_enable(True)
    _lib.profile_reset()
    grads_drawn = abi.backward(q, k, v, out, g, lse, **kw)[:3]
    torch.cuda.synchronize()
    probes = _lib.profile_read()
    _lib.profile_enable(False)
    assert probes["dropout_bits"][0] == 1
    for a_, b_ in zip((dq, dk, dv), grads_drawn):
        assert torch.equal(a_, b_)
    check(abi.host(out), out_c, dtype, "o", "O")
    for got, want, name in zip((dq, dk, dv), back(inp.do), ("dQ", "dK", "dV")):
        check(abi.host(got), want, dtype, "g", name)
    # the bits the forward wrote: the keep mask packed, on every tile a wave of
    # 32 rows computes (keys below Sk)
    want_bits = packed_bits(abi.dropout_keep(q, k, v, **kw).cpu().numpy())
    got_bits = bits.cpu().numpy()
    valid = key_bits_valid(sk)
    for qw in range(0, sq, 32):
        last = min(qw + 32, sq) - 1
        wlim = min(sk, last + off + 1) if causal else sk
        tiles = -(-wlim // 32) if wlim > 0 else 0
        for t in range(tiles):
            rows = slice(qw, last + 1)
            np.testing.assert_array_equal(got_bits[:, :, t, rows] & valid[t],
                                          want_bits[:, :, t, rows] & valid[t])
    # the same stream again: every bit; another key: different outputs
    out2, lse2, _ = abi.forward(q, k, v, **kw)
    assert torch.equal(out, out2) and torch.equal(lse, lse2)
    kw3 = dict(kw, dropout=(p, key + 1, counter))
    out3, _, _ = abi.forward(q, k, v, **kw3)
    assert not torch.equal(out, out3)


@pytest.mark.parametrize("case", [CASES[0], CASES[2]], ids=lambda c: "-".join(map(str, c)))
def test_dropout_recomputing_dq_matches_oracle(case):
    """Workspaces without room for stored dS run the dropout dQ kernel that
    recomputes S and dP (reading the keep bits with each key tile): the row
    values alone when the forward's bits are passed, the row values plus the
    drawn bits otherwise.  Both match the oracle and give the same gradients."""
    dtype, b, hq, hkv, sq, sk, d, causal, off, p, masked = case
    say(f"dropout, recomputing dQ {case}")
    inp = attention_inputs(b, hq, sq, d, dtype, heads_kv=hkv, seq_k=sk, value_scale=0.5, seed=37)
    key, counter = 0x0DD5_EED0_0000_0000_0000_0000_4242_4242, 5
    mask = np.random.default_rng(2).random((sq, sk)) > 0.25 if masked else None
    _, _, back = DR.sdpa_dropout(inp.q, inp.k, inp.v, mask, causal, dtype=dtype, p=p,
                                 rng_key=key, rng_counter=counter, causal_offset=off,
                                 enable_gqa=hkv != hq)
    q, k, v, g = (abi.dev_tensor(x, dtype) for x in (inp.q, inp.k, inp.v, inp.do))
    kw = dict(causal=causal, offset=off, dropout=(p, key, counter),
              mask=None if mask is None else torch.from_numpy(mask).cuda())
    bits = abi.dropout_bits_buffer(q, k, v, **kw)
    out, lse, _ = abi.forward(q, k, v, dropout_bits=bits, **kw)
    rows_bytes = 2 * b * hq * sq * 4
    with_bits = -(-rows_bytes // 256) * 256 + bits.numel() * 4
    results = []
    for ws, given in ((rows_bytes, bits), (with_bits, None)):
        _lib.profile_enable(True)
        _lib.profile_reset()
        grads = abi.backward(q, k, v, out, g, lse, ws_bytes=ws, dropout_bits=given, **kw)[:3]
        torch.cuda.synchronize()
        probes = _lib.profile_read()
        _lib.profile_enable(False)
        assert {"bwd_dq_mfma_dropout", "bwd_dkdv_mfma_dropout"} <= set(probes), sorted(probes)
        assert "bwd_dq_ds_dropout" not in probes, sorted(probes)
        assert ("dropout_bits" in probes) == (given is None), sorted(probes)
        results.append(grads)
        for got, want, name in zip(grads, back(inp.do), ("dQ", "dK", "dV")):
            check(abi.host(got), want, dtype, "g", name)
    for a_, b_ in zip(*results):
        assert torch.equal(a_, b_)


@pytest.mark.parametrize("p", [0.99999, 0.999995])
def test_dropout_probability_near_one(p):
    """The top of the 16-bit threshold range on the MFMA forward: p = 0.99999
    gives threshold 65535 (a word is kept only when it is 65535), p = 0.999995
    rounds it to 65536, which no word reaches (the kernel then zeroes the
    probabilities and the keep bits without comparing): the written bits equal
    the oracle's mask packed, and O and the gradients match the oracle's."""
    dtype, b, h, s, d = "bfloat16", 1, 2, 256, 128
    say(f"dropout near one: p={p}")
    assert DR.threshold(p) == (65535 if p < 0.999995 else 65536)
    inp = attention_inputs(b, h, s, d, dtype, value_scale=0.5, seed=5)
    key, counter = 99, 0
    keep = DR.keep_mask(key, counter, (b, h, s, s), p)
    q, k, v, g = (abi.dev_tensor(x, dtype) for x in (inp.q, inp.k, inp.v, inp.do))
    kw = dict(causal=False, dropout=(p, key, counter))
    bits = abi.dropout_bits_buffer(q, k, v, **kw)
    out, lse, path = abi.forward(q, k, v, dropout_bits=bits, **kw)
    assert path == _lib.PATH_MFMA
    np.testing.assert_array_equal(bits.cpu().numpy(), packed_bits(keep))
    dq, dk, dv, _ = abi.backward(q, k, v, out, g, lse, dropout_bits=bits, **kw)
    out_c, _, back = DR.sdpa_dropout(inp.q, inp.k, inp.v, None, False, dtype=dtype, p=p,
                                     rng_key=key, rng_counter=counter)
    say(f"  kept elements: {int(keep.sum())}")
    if not keep.any():
        for t in (out, dq, dk, dv):
            assert not t.float().abs().max().item()
    check(abi.host(out), out_c, dtype, "o", "O")
    for got, want, name in zip((dq, dk, dv), back(inp.do), ("dQ", "dK", "dV")):
        check(abi.host(got), want, dtype, "g", name)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_dropout_with_key_padding_lengths(dtype):
    """Dropout with a [B,1,1,K] key-padding mask reduced to kv_len: the
    kernels stop at each row's length (the forward writes bits only up to it)
    and match the oracle under the same boolean mask."""
    b, h, sq, sk, d, p = 3, 2, 96, 200, 128, 0.25
    say(f"dropout + key padding {dtype}")
    inp = attention_inputs(b, h, sq, d, dtype, seq_k=sk, value_scale=0.5, seed=53)
    lens = np.array([200, 37, 129])
    km = np.arange(sk)[None, :] < lens[:, None]  # [B, K] allowed keys
    mask4 = km[:, None, None, :]
    key, counter = 0x1234_5678_9ABC_DEF0, 2
    out_c, _, back = DR.sdpa_dropout(inp.q, inp.k, inp.v, mask4, True, dtype=dtype, p=p,
                                     rng_key=key, rng_counter=counter, causal_offset=sk - sq)
    q, k, v, g = (abi.dev_tensor(x, dtype) for x in (inp.q, inp.k, inp.v, inp.do))
    tmask = torch.from_numpy(km).cuda()
    kv_len, kv_prefix = abi.key_lengths(tmask)
    kw = dict(causal=True, offset=sk - sq, dropout=(p, key, counter),
              mask=tmask[:, None, None, :], kv_len=kv_len, kv_prefix=kv_prefix)
    bits = abi.dropout_bits_buffer(q, k, v, **kw)
    out, lse, path = abi.forward(q, k, v, dropout_bits=bits, **kw)
    assert path == _lib.PATH_MFMA
    grads = abi.backward(q, k, v, out, g, lse, dropout_bits=bits, **kw)[:3]
    grads_drawn = abi.backward(q, k, v, out, g, lse, **kw)[:3]
    torch.cuda.synchronize()
    for a_, b_ in zip(grads, grads_drawn):
        assert torch.equal(a_, b_)
    check(abi.host(out), out_c, dtype, "o", "O")
    for got, want, name in zip(grads, back(inp.do), ("dQ", "dK", "dV")):
        check(abi.host(got), want, dtype, "g", name)
    dk = abi.host(grads[1])
    for bi, n in enumerate(lens):  # keys past a row's length get no gradient
        assert (dk[bi, :, n:] == 0).all()


GENERIC_CASES = [
    # (dtype, B, Hq, Hkv, Sq, Sk, Dqk, Dv, causal, p): generic kernels
    ("float32", 2, 2, 1, 33, 70, 32, 48, True, 0.25),
    ("float64", 1, 2, 2, 20, 40, 16, 16, False, 0.5),
    ("bfloat16", 1, 2, 2, 40, 40, 96, 96, True, 0.2),  # head dim 96: not an MFMA shape
]


@pytest.mark.parametrize("case", GENERIC_CASES, ids=lambda c: "-".join(map(str, c)))
def test_dropout_on_the_generic_kernels(case):
    dtype, b, hq, hkv, sq, sk, d, dv_, causal, p = case
    say(f"generic dropout {case}")
    inp = attention_inputs(b, hq, sq, d, dtype, heads_kv=hkv, seq_k=sk, dim_v=dv_, seed=41)
    key, counter = 2**100 + 17, 2**64 - 1
    out_c, _, back = DR.sdpa_dropout(inp.q, inp.k, inp.v, None, causal, dtype=dtype, p=p,
                                     rng_key=key, rng_counter=counter, enable_gqa=hkv != hq)
    q, k, v, g = (abi.dev_tensor(x, dtype) for x in (inp.q, inp.k, inp.v, inp.do))
    kw = dict(causal=causal, dropout=(p, key, counter))
    bits = abi.dropout_bits_buffer(q, k, v, **kw)
    out, lse, path = abi.forward(q, k, v, dropout_bits=bits, **kw)
    assert path == _lib.PATH_GENERIC
    grads = abi.backward(q, k, v, out, g, lse, **kw)[:3]
    torch.cuda.synchronize()
    # the generic forward writes every word of the bits (padding rows zero)
    np.testing.assert_array_equal(bits.cpu().numpy(),
                                  packed_bits(abi.dropout_keep(q, k, v, **kw).cpu().numpy()))
    if dtype in TOL:
        check(abi.host(out), out_c, dtype, "o", "O")
        for got, want, name in zip(grads, back(inp.do), ("dQ", "dK", "dV")):
            check(abi.host(got), want, dtype, "g", name)
    else:  # the reference's fp32 cross-backend bound / fp64
        tol = dict(rtol=1e-4, atol=3e-5) if dtype == "float32" else dict(rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(abi.host(out), out_c, **tol)
        for got, want in zip(grads, back(inp.do)):
            np.testing.assert_allclose(abi.host(got), want, **tol)


def test_dropout_probability_is_validated():
    q = torch.zeros((1, 1, 8, 32), dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError, match="dropout"):
        abi.forward(q, q, q, dropout=(1.0, 1, 0))
    with pytest.raises(ValueError, match="dropout"):
        abi.forward(q, q, q, dropout=(-0.1, 1, 0))


def test_mirror_dropout_backends_and_gradients():
    ts.seed(8)
    q, k, v = (ts.tensor(np.random.default_rng(i).standard_normal((2, 2, 64, 64)).astype(np.float32),
                         device="hip", dtype="bfloat16", requires_grad=True) for i in range(3))
    _lib.profile_enable(True)
    _lib.profile_reset()
    for backend in ("hip", "dense", "auto"):
        out = nn.scaled_dot_product_attention(q, k, v, dropout_p=0.3, backend=backend)
        out.sum().backward()
    probes = _lib.profile_read()
    _lib.profile_enable(False)
    assert probes["fwd_mfma_dropout"][0] == 3 and probes["bwd_dkdv_mfma_dropout"][0] == 3
    assert "dropout_bits" not in probes  # the backward reads the forward's bits
    assert all(np.isfinite(t.grad.numpy()).all() for t in (q, k, v))
    with pytest.raises(ValueError, match="dense backend"):
        nn.scaled_dot_product_attention(q, k, v, dropout_p=0.1, backend="streaming")
    # seeded: the same host seed gives the same draw
    ts.seed(5)
    a = nn.scaled_dot_product_attention(q, k, v, dropout_p=0.4, backend="hip").numpy()
    ts.seed(5)
    b_ = nn.scaled_dot_product_attention(q, k, v, dropout_p=0.4, backend="hip").numpy()
    np.testing.assert_array_equal(a, b_)
