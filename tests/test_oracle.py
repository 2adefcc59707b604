"""Pin the NumPy oracle before it is trusted to check the HIP kernels (CPU only).

Each check is chosen so a plausible restatement mistake fails it: the golden
fixtures come from torch (not from the oracle), the brute force is an
independent closed form, finite differences pin the VJP without any formula,
and the invariants hold only for the exact math.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import golden_kwargs, rel_l2
from oracle import attention as A
from oracle.halfprec import bf16_bits, bf16_from_bits, bf16_round, round_to
from oracle.inputs import attention_inputs


@pytest.mark.parametrize("backend", ["dense", "streaming"])
@pytest.mark.parametrize("block", [2, 3, 64])
def test_oracle_matches_torch_golden_f64(golden, backend, block):
    for name, case in golden.items():
        kw, mask = golden_kwargs(case)
        r = A.sdpa(case["q"], case["k"], case["v"], mask, dtype="float64",
                   backend=backend, block_size=block, **kw)
        np.testing.assert_allclose(r.out, case["out"], rtol=1e-10, atol=1e-12, err_msg=name)
        if r.lse is not None:
            np.testing.assert_array_equal(np.isinf(r.lse[..., 0]), np.isinf(case["lse"]))
            live = np.isfinite(case["lse"])
            np.testing.assert_allclose(r.lse[..., 0][live], case["lse"][live], rtol=1e-12)
        dq, dk, dv = r.backward(case["g"])
        for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
            np.testing.assert_allclose(got, case[key], rtol=1e-9, atol=1e-11,
                                       err_msg=f"{name}/{key}")


def test_oracle_f32_matches_golden_within_reference_tolerance(golden):
    # the reference's cross-backend bound (tests/test_transformer.py:92)
    for name, case in golden.items():
        kw, mask = golden_kwargs(case)
        if mask is not None and mask.dtype != np.bool_:
            mask = mask.astype(np.float32)
        q, k, v, g = (case[x].astype(np.float32) for x in ("q", "k", "v", "g"))
        r = A.sdpa(q, k, v, mask, dtype="float32", backend="streaming", block_size=2, **kw)
        np.testing.assert_allclose(r.out, case["out"], rtol=1e-4, atol=3e-5, err_msg=name)
        for got, key in zip(r.backward(g), ("dq", "dk", "dv")):
            np.testing.assert_allclose(got, case[key], rtol=1e-4, atol=3e-5, err_msg=name)


def _random_case(rng, b=2, hq=4, hkv=2, sq=9, sk=13, d=6, dv=5):
    q = rng.standard_normal((b, hq, sq, d))
    k = rng.standard_normal((b, hkv, sk, d))
    v = rng.standard_normal((b, hkv, sk, dv))
    g = rng.standard_normal((b, hq, sq, dv))
    return q, k, v, g


@pytest.mark.parametrize("causal,offset", [(False, 0), (True, 0), (True, 4), (True, 20)])
def test_oracle_matches_brute_force(causal, offset):
    rng = np.random.default_rng(3)
    q, k, v, g = _random_case(rng)
    mask = rng.random((2, 1, 9, 13)) > 0.3
    mask[0, 0, 5] = False  # fully masked row
    for m in (None, mask):
        r = A.sdpa(q, k, v, m, causal, dtype="float64", causal_offset=offset,
                   backend="streaming", block_size=4, enable_gqa=True)
        out, lse, _ = A.brute_force_f64(q, k, v, m, causal, offset)
        np.testing.assert_allclose(r.out, out, rtol=1e-11, atol=1e-13)
        np.testing.assert_array_equal(np.isinf(r.lse[..., 0]), np.isinf(lse))


def test_streaming_equals_dense_for_any_block():
    rng = np.random.default_rng(4)
    q, k, v, g = _random_case(rng, hkv=4)
    ref = A.sdpa(q, k, v, None, True, dtype="float64", backend="dense", causal_offset=3)
    want = ref.backward(g)
    for block in (1, 2, 5, 8, 64):
        r = A.sdpa(q, k, v, None, True, dtype="float64", backend="streaming",
                   block_size=block, causal_offset=3)
        np.testing.assert_allclose(r.out, ref.out, rtol=1e-12, atol=1e-14)
        for a, b in zip(r.backward(g), want):
            np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-12)


def test_vjp_central_differences():
    """The reference's own VJP check method (tests/test_transformer.py:13-33)."""
    np.random.seed(19)
    arrays = [np.random.randn(1, 2, 3, 4), np.random.randn(1, 2, 5, 4), np.random.randn(1, 2, 5, 3)]
    upstream = np.random.default_rng(12).normal(size=(1, 2, 3, 3))
    for backend in ("dense", "streaming"):
        def f(q, k, v):
            return A.sdpa(q, k, v, None, True, dtype="float64", causal_offset=2,
                          backend=backend, block_size=2)
        grads = f(*arrays).backward(upstream)
        for index, raw in enumerate(arrays):
            for flat in np.linspace(0, raw.size - 1, min(8, raw.size), dtype=int):
                pos = np.unravel_index(flat, raw.shape)
                orig = raw[pos]
                raw[pos] = orig + 1e-5
                hi = (f(*arrays).out * upstream).sum()
                raw[pos] = orig - 1e-5
                lo = (f(*arrays).out * upstream).sum()
                raw[pos] = orig
                assert abs(grads[index][pos] - (hi - lo) / 2e-5) < 5e-6


def test_vjp_invariants():
    """Shift invariance of softmax gives sum_j dK_j = 0; sum_j P_ij = 1 gives
    sum_j dV_j = sum of upstream rows that attend to anything."""
    rng = np.random.default_rng(5)
    q, k, v, g = _random_case(rng, hkv=4)
    mask = rng.random((2, 1, 9, 13)) > 0.4
    mask[1, 0, 2] = False
    r = A.sdpa(q, k, v, mask, True, dtype="float64", causal_offset=6, backend="streaming",
               block_size=4)
    dq, dk, dv = r.backward(g)
    np.testing.assert_allclose(dk.sum(axis=2), 0, atol=1e-11)
    live = A.allowed_matrix(2, 4, 9, 13, mask, True, 6).any(-1)
    np.testing.assert_allclose(dv.sum(axis=2), (g * live[..., None]).sum(axis=2), atol=1e-11)
    # fully masked rows: zero output and zero dq (tests/test_transformer.py:86-87)
    np.testing.assert_array_equal(r.out[1, :, 2], 0)
    np.testing.assert_array_equal(dq[1, :, 2], 0)


def test_gqa_equals_expanded_mha():
    rng = np.random.default_rng(6)
    q, k, v, g = _random_case(rng, hq=6, hkv=2)
    r = A.sdpa(q, k, v, None, True, dtype="float64", enable_gqa=True, backend="streaming",
               block_size=4)
    ek = np.repeat(k, 3, axis=1)
    ev = np.repeat(v, 3, axis=1)
    e = A.sdpa(q, ek, ev, None, True, dtype="float64", backend="streaming", block_size=4)
    np.testing.assert_allclose(r.out, e.out, rtol=1e-13)
    dq, dk, dv = r.backward(g)
    edq, edk, edv = e.backward(g)
    np.testing.assert_allclose(dq, edq, rtol=1e-12)
    np.testing.assert_allclose(dk, edk.reshape(2, 2, 3, 13, 6).sum(2), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dv, edv.reshape(2, 2, 3, 13, 5).sum(2), rtol=1e-10, atol=1e-12)
    with pytest.raises(ValueError):
        A.sdpa(q, k, v, dtype="float64")


def test_decode_equals_last_row_of_prefill():
    """Cached decode of the last token == last row of the full causal prefill."""
    rng = np.random.default_rng(8)
    q, k, v, _ = _random_case(rng, hq=2, hkv=2, sq=12, sk=12)
    full = A.sdpa(q, k, v, None, True, dtype="float64", backend="dense")
    dec = A.sdpa(q[:, :, -1:], k, v, None, True, dtype="float64", causal_offset=11,
                 backend="streaming", block_size=5)
    np.testing.assert_allclose(dec.out[:, :, 0], full.out[:, :, -1], rtol=1e-12)
    lengths = np.array([12, 7])
    kp = A.key_padding_mask(lengths, 12)
    dec = A.sdpa(q[:, :, -1:], k, v, kp, False, dtype="float64", backend="streaming")
    short = A.sdpa(q[1:, :, -1:], k[1:, :, :7], v[1:, :, :7], None, False, dtype="float64",
                   backend="dense")
    np.testing.assert_allclose(dec.out[1:], short.out, rtol=1e-12)


def test_bf16_and_f16_rounding_match_torch():
    rng = np.random.default_rng(9)
    x = np.concatenate([
        rng.standard_normal(100_000).astype(np.float32) * 3,
        np.array([0.0, -0.0, 1e-40, 3.4e38, -3.4e38, 65504.0, 1.00390625, 1.01171875],
                 np.float32),
    ])
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(bf16_round(x), want)
    bits = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bf16_bits(x), bits)
    np.testing.assert_array_equal(bf16_from_bits(bits), want)
    want16 = torch.from_numpy(x).to(torch.float16).to(torch.float32).numpy()
    np.testing.assert_array_equal(round_to(x, "float16"), want16)


def test_half_inputs_compute_in_f32_and_round_outputs():
    inp = attention_inputs(1, 2, 40, 16, "bfloat16", value_scale=0.5)
    assert np.array_equal(bf16_round(inp.q), inp.q)
    r = A.sdpa(inp.q, inp.k, inp.v, None, True, dtype="bfloat16", backend="streaming")
    assert r.out.dtype == np.float32
    np.testing.assert_array_equal(r.out_cast, bf16_round(r.out))
    ref, _, _ = A.brute_force_f64(inp.q, inp.k, inp.v, None, True)
    assert rel_l2(r.out, ref) < 1e-6


def test_int8_quantiser_closed_form():
    rng = np.random.default_rng(10)
    x = rng.standard_normal((2, 3, 7, 16)).astype(np.float32)
    x[0, 0, 0] = 0  # all-zero token uses the 1e-8 floor
    q, s = A.quantize_int8(x)
    assert q.dtype == np.int8 and s.shape == (2, 3, 7, 1)
    np.testing.assert_allclose(s[..., 0], np.maximum(np.abs(x).max(-1) / 127, 1e-8), rtol=1e-7)
    assert np.abs(q).max() <= 127
    err = np.abs(A.dequantize_int8(q, s) - x)
    assert np.all(err <= s / 2 + 1e-7)
    assert np.all(q[0, 0, 0] == 0)


def test_inputs_recipe_is_seeded_and_ordered():
    a = attention_inputs(2, 2, 8, 4, "float32", length_range=(3, 8))
    rng = np.random.default_rng(42)
    np.testing.assert_array_equal(a.q, rng.standard_normal((2, 2, 8, 4), dtype=np.float32))
    np.testing.assert_array_equal(a.k, rng.standard_normal((2, 2, 8, 4), dtype=np.float32))
    np.testing.assert_array_equal(a.v, rng.standard_normal((2, 2, 8, 4), dtype=np.float32))
    np.testing.assert_array_equal(a.do, rng.standard_normal((2, 2, 8, 4), dtype=np.float32))
    assert np.array_equal(a.lengths, rng.integers(3, 9, size=2))
    assert math.isclose(float(np.std(attention_inputs(1, 1, 64, 64, "float32",
                                                      value_scale=0.5).q)), 0.5, rel_tol=0.1)


# ---------------------------------------------------------------------------
# RoPE oracle (reference attention.py:255-296), pinned by what the
# mathematics fixes rather than by retyping the formula.
# ---------------------------------------------------------------------------
from oracle import rope as R  # noqa: E402


def test_rope_position_zero_is_identity_and_tail_passes_through():
    x = np.random.default_rng(1).standard_normal((2, 3, 5, 16)).astype(np.float32)
    y = R.rope(x, offset=0, rotary_dim=12)
    np.testing.assert_array_equal(y[..., 0, :], x[..., 0, :])  # cos 0 = 1, sin 0 = 0
    np.testing.assert_array_equal(y[..., 12:], x[..., 12:])    # channels past rotary_dim


def test_rope_f32_is_complex_multiplication():
    """(x0 + i x1) * exp(i theta) in float64 on the same float32 cos / sin:
    each component rounds twice (products, then the sum) in float32."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 7, 32)).astype(np.float32)
    y = R.rope(x, offset=11, base=500.0)
    c, s = R.tables(7, 32, 500.0, 11)
    z = (x[..., 0::2].astype(np.float64) + 1j * x[..., 1::2]) * (c.astype(np.float64) + 1j * s)
    np.testing.assert_allclose(y[..., 0::2], z.real, rtol=0, atol=4e-7 * np.abs(x).max())
    np.testing.assert_allclose(y[..., 1::2], z.imag, rtol=0, atol=4e-7 * np.abs(x).max())


def test_rope_f64_is_complex_multiplication():
    """float64 inputs: the float32 cos / sin cast to float64, products and
    sums in float64."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 9, 16))
    y = R.rope(x, offset=5, dtype="float64")
    assert y.dtype == np.float64
    c, s = R.tables(9, 16, 10000.0, 5)
    z = (x[..., 0::2] + 1j * x[..., 1::2]) * (c.astype(np.float64) + 1j * s.astype(np.float64))
    np.testing.assert_allclose(y[..., 0::2], z.real, rtol=0, atol=1e-15 * np.abs(x).max())
    np.testing.assert_allclose(y[..., 1::2], z.imag, rtol=0, atol=1e-15 * np.abs(x).max())


@pytest.mark.parametrize("dtype,tol", [("float32", 1e-6), ("float16", 2e-3), ("bfloat16", 1.6e-2)])
def test_rope_inverse_undoes_rotation_and_keeps_pair_norms(dtype, tol):
    from oracle.halfprec import round_to

    x = round_to(np.random.default_rng(3).standard_normal((3, 9, 64)), dtype)
    y = R.rope(x, offset=100, dtype=dtype)
    back = R.rope(y, offset=100, dtype=dtype, inverse=True)
    np.testing.assert_allclose(back, x, atol=tol * 4, rtol=tol * 4)
    n0 = np.hypot(x[..., 0::2], x[..., 1::2])
    n1 = np.hypot(y[..., 0::2], y[..., 1::2])
    np.testing.assert_allclose(n1, n0, rtol=tol * 2, atol=tol * 2)


def test_rope_rows_depend_only_on_absolute_position():
    x = np.random.default_rng(4).standard_normal((1, 1, 8, 16)).astype(np.float32)
    whole = R.rope(x, offset=3)
    for t in range(8):
        np.testing.assert_array_equal(R.rope(x[..., t:t + 1, :], offset=3 + t), whole[..., t:t + 1, :])


# ---------------------------------------------------------------------------
# Dropout: Philox4x32-10 pinned against the known-answer vectors of its
# Random123 release; the stream layout against those blocks one by one; the
# element mapping against an explicit loop; the attention math against the
# dropout-free oracle (p = 0), finite differences (fixed mask) and the
# reference's mask value formula.
# ---------------------------------------------------------------------------

from oracle import dropout as DR  # noqa: E402

# (counter words, key words) -> output words, Random123's kat_vectors for
# philox4x32 with 10 rounds
PHILOX4X32_KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,want", PHILOX4X32_KAT)
def test_philox4x32_known_answers(ctr, key, want):
    got = DR.philox4x32(*(np.array([c], np.uint64) for c in ctr), *key)
    assert tuple(int(x[0]) for x in got) == want


@pytest.mark.parametrize("key,counter", [(0, 0), (0x0123456789ABCDEF_FEDCBA9876543210, 5),
                                         (2**128 - 1, 2**64 - 3), (987654321, 2**63 + 9)])
def test_stream_is_the_philox_blocks_in_order(key, counter):
    """Group g = blocks t = 2 (counter + g) and t + 1 (mod 2^64), counter
    words (lo t, hi t, lo K1, hi K1), key K0; outputs packed little-endian."""
    raw = DR.raw_stream(key, counter, 41)
    k0, k1 = key & (2**64 - 1), key >> 64
    words = []
    for g in range(11):
        for half in (0, 1):
            t = (2 * (counter + g) + half) % 2**64
            ctr = (t & 0xFFFFFFFF, t >> 32, k1 & 0xFFFFFFFF, k1 >> 32)
            out = DR.philox4x32(*(np.array([c], np.uint64) for c in ctr), k0 & 0xFFFFFFFF, k0 >> 32)
            x = [int(v[0]) for v in out]
            words += [x[0] | x[1] << 32, x[2] | x[3] << 32]
    assert [int(v) for v in raw] == words[:41]


def test_keep_mask_element_mapping():
    key, counter, shape, p = 77, 3, (2, 3, 4, 5), 0.4
    raw = DR.raw_stream(key, counter, 2 * 3 * 4 * 16 // 4)
    got = DR.keep_mask(key, counter, shape, p)
    thr = DR.threshold(p)
    for b in range(2):
        for h in range(3):
            for i in range(4):
                for j in range(5):
                    word_index = ((b * 3 + h) * 4 + i) * 16 + j
                    w = (int(raw[word_index // 4]) >> (16 * (word_index % 4))) & 0xFFFF
                    assert got[b, h, i, j] == (w >= thr)


def test_keep_fraction_and_scale():
    p = 0.3
    keep = DR.keep_mask(5, 0, (4, 8, 64, 200), p)
    n = keep.size
    assert abs(keep.mean() - (1 - p)) < 5 * math.sqrt(p * (1 - p) / n)
    assert DR.threshold(0.0) == 0 and DR.keep_mask(1, 0, (1, 1, 3, 7), 0.0).all()
    # the reference's mask value: keep.astype(float32) / (1 - p) with a Python float
    ref = np.ones(3, np.float32) / (1 - p)
    assert ref.dtype == np.float32 and (ref == DR.keep_scale(p)).all()


def test_dropout_attention_without_dropout_is_the_dense_oracle():
    inp = attention_inputs(2, 2, 9, 8, "float32", seed=3)
    out, _, back = DR.sdpa_dropout(inp.q, inp.k, inp.v, None, True, dtype="float32", p=0.0,
                                   rng_key=9)
    ref = A.sdpa(inp.q, inp.k, inp.v, None, True, dtype="float32", backend="dense")
    np.testing.assert_array_equal(out, ref.out)
    for got, want in zip(back(inp.do), ref.backward(inp.do)):
        np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)


def test_dropout_attention_vjp_matches_finite_differences():
    rng = np.random.default_rng(4)
    q, k, v = (rng.standard_normal((1, 2, 5, 4)) for _ in range(3))
    g = rng.standard_normal((1, 2, 5, 4))
    kw = dict(dtype="float64", p=0.35, rng_key=123, rng_counter=7)
    mask = np.tril(np.ones((5, 5), bool))
    _, _, back = DR.sdpa_dropout(q, k, v, mask, **kw)
    grads = back(g)
    f = lambda q_, k_, v_: float(np.sum(DR.sdpa_dropout(q_, k_, v_, mask, **kw)[0] * g))
    eps = 1e-6
    for which, grad in enumerate(grads):
        args = [q, k, v]
        x = args[which]
        num = np.zeros_like(x)
        for idx in np.ndindex(x.shape):
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            num[idx] = (f(*[xp if i == which else a for i, a in enumerate(args)])
                        - f(*[xm if i == which else a for i, a in enumerate(args)])) / (2 * eps)
        np.testing.assert_allclose(grad, num, rtol=1e-6, atol=1e-8)
    # the mask really drops something and keeps something
    keep = DR.keep_mask(123, 7, (1, 2, 5, 5), 0.35)
    assert 0 < keep.sum() < keep.size
