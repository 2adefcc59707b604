"""Rotary position embedding on the device (needs an MI355X).

* ``tsattn_rope``: bit-exact against the oracle's restatement of the
  reference's rotary_embedding (src/tensorsmith/nn/attention.py:255-296) for
  f32 / f16 / bf16, full and partial rotary dims, odd pair counts past one
  wave (D = 130), position offsets and strided (permuted) sources; the
  inverse rotation is bit-exact against the oracle's VJP rotation.
* The mirror's ``rotary_embedding`` runs that kernel forward and backward
  (timing probe) with the same bits.
* ``tsattn_rope_append``: the new key rows rotated and both K and V written
  into the cache rows at ``pos`` -- bit-exact against oracle rope followed by
  a plain copy (fp caches) or by the oracle's restatement of the reference
  quantiser (cache.py:73-77, int8 caches); rows outside the window untouched.
* Model level: cached TransformerLM decoding through the fused kernel gives
  bit-identical logits and cache contents to the two-step path
  (rotary_embedding, then append), fp16 and int8 caches.
* RoPE folded into the MFMA attention kernels
  (``tsattn_sdpa_forward_rope`` / ``_backward_rope``): O, LSE, dQ, dK, dV
  bit-identical to the unfused chain (tsattn_rope on q and k, attention,
  inverse tsattn_rope on dq and dk) -- partial rotary dims, GQA, causal
  offsets, distinct query / key positions, general masks; problems outside
  the MFMA kernels refuse with ERR_UNSUPPORTED; MultiHeadAttention training
  steps give bit-identical outputs and gradients through the fused path and
  through rotary_embedding + attention.
"""

from __future__ import annotations

from unittest.mock import patch

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("no GPU", allow_module_level=True)

import abi  # noqa: E402
import tensorsmith_hip as ts  # noqa: E402
from oracle import attention as A  # noqa: E402
from oracle import rope as R  # noqa: E402
from oracle.halfprec import round_to  # noqa: E402
from tensorsmith_hip import _lib, nn  # noqa: E402
from tensorsmith_hip.nn.cache import KVCache  # noqa: E402

DTYPES = ["float32", "float16", "bfloat16"]


def say(msg):
    print(msg, flush=True)


def tables(n, rdim, dtype):
    cos, sin = R.tables(n, rdim)
    return abi.dev_tensor(round_to(cos, dtype), dtype), abi.dev_tensor(round_to(sin, dtype), dtype)


def rows(rng, shape, dtype, scale=2.0):
    return round_to(rng.standard_normal(shape).astype(np.float32) * scale, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("dim,rdim", [(64, 64), (130, 130), (256, 96), (6, 4)])
@pytest.mark.parametrize("offset", [0, 37])
@pytest.mark.parametrize("inverse", [False, True])
def test_rope_kernel_is_bit_exact(dtype, dim, rdim, offset, inverse):
    say(f"rope {dtype} D{dim} R{rdim} offset {offset} inverse {inverse}")
    rng = np.random.default_rng(dim + offset)
    b, h, t = 2, 3, 9
    x = rows(rng, (b, t, h, dim), dtype)
    src = abi.dev_tensor(x, dtype).permute(0, 2, 1, 3)  # [B,H,T,D] strided view
    out = torch.full((b, h, t, dim), 7.0, dtype=src.dtype, device="cuda")
    cos, sin = tables(offset + t + 3, rdim, dtype)
    abi.rope(src, out, cos, sin, offset, rdim, inverse)
    want = R.rope(x.transpose(0, 2, 1, 3), offset, rotary_dim=rdim, dtype=dtype, inverse=inverse)
    np.testing.assert_array_equal(abi.host(out), want)


def test_rope_then_inverse_is_the_identity_up_to_rounding():
    rng = np.random.default_rng(3)
    x = rows(rng, (1, 4, 33, 128), "float32")
    src = abi.dev_tensor(x, "float32")
    mid, back = torch.empty_like(src), torch.empty_like(src)
    cos, sin = tables(1000, 128, "float32")
    abi.rope(src, mid, cos, sin, 900, 128)
    abi.rope(mid, back, cos, sin, 900, 128, inverse=True)
    np.testing.assert_allclose(abi.host(back), x, rtol=0, atol=4e-6 * np.abs(x).max())
    assert np.abs(abi.host(mid) - x).max() > 0.1  # it did rotate


@pytest.mark.parametrize("dtype", DTYPES)
def test_mirror_rotary_embedding_runs_the_kernel_forward_and_backward(dtype):
    say(f"rotary_embedding mirror {dtype}")
    rng = np.random.default_rng(11)
    x = rows(rng, (2, 4, 17, 64), dtype)
    g = rows(rng, (2, 4, 17, 64), dtype, 1.0)
    xt = ts.tensor(x, device="hip", dtype=dtype, requires_grad=True)
    _lib.profile_enable(True)
    _lib.profile_reset()
    y = nn.functional.rotary_embedding(xt, 5, rotary_dim=48)
    y.backward(ts.tensor(g, device="hip", dtype=dtype))
    probes = _lib.profile_read()
    _lib.profile_enable(False)
    assert probes["rope"][0] == 2
    np.testing.assert_array_equal(y.numpy().astype(np.float32),
                                  R.rope(x, 5, rotary_dim=48, dtype=dtype))
    np.testing.assert_array_equal(xt.grad.numpy().astype(np.float32),
                                  R.rope(g, 5, rotary_dim=48, dtype=dtype, inverse=True))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("dim,rdim", [(64, 64), (130, 66), (512, 512), (128, 0)])
@pytest.mark.parametrize("quantized", [False, True])
def test_rope_append_is_bit_exact(dtype, dim, rdim, quantized):
    say(f"rope append {dtype} D{dim} R{rdim} int8 {quantized}")
    rng = np.random.default_rng(dim + rdim)
    b, h, t, pos, cap = 2, 3, 5, 6, 16
    k = rows(rng, (b, t, h, dim), dtype)
    v = rows(rng, (b, t, h, dim), dtype)
    k[1, 2] = 0.0  # all-zero rows: scale 1e-8 in an int8 cache
    kd = abi.dev_tensor(k, dtype).permute(0, 2, 1, 3)
    vd = abi.dev_tensor(v, dtype).permute(0, 2, 1, 3)
    cos, sin = tables(cap, rdim, dtype) if rdim else (None, None)
    store = torch.int8 if quantized else kd.dtype
    kc = torch.zeros((b, h, cap, dim), dtype=store, device="cuda")
    vc = torch.zeros((b, h, cap, dim), dtype=store, device="cuda")
    ks = torch.ones((b, h, cap, 1), dtype=torch.float32, device="cuda") if quantized else None
    vs = torch.ones((b, h, cap, 1), dtype=torch.float32, device="cuda") if quantized else None
    abi.rope_append(kd, vd, kc, vc, cos, sin, pos, rdim, ks, vs)
    kr = k.transpose(0, 2, 1, 3)
    vr = v.transpose(0, 2, 1, 3)
    if rdim:
        kr = R.rope(kr, pos, rotary_dim=rdim, dtype=dtype)
    win = slice(pos, pos + t)
    if quantized:
        for cache, scale, want in ((kc, ks, kr), (vc, vs, vr)):
            q, s = A.quantize_int8(want)
            np.testing.assert_array_equal(cache[:, :, win].cpu().numpy(), q)
            np.testing.assert_array_equal(scale[:, :, win].cpu().numpy(), s)
            assert (scale[:, :, :pos] == 1).all() and (scale[:, :, pos + t:] == 1).all()
    else:
        np.testing.assert_array_equal(abi.host(kc[:, :, win]), kr)
        np.testing.assert_array_equal(abi.host(vc[:, :, win]), vr)
    for cache in (kc, vc):
        assert (cache[:, :, :pos] == 0).all() and (cache[:, :, pos + t:] == 0).all()


def test_rope_append_rejects_what_it_cannot_hold():
    x = torch.zeros((1, 1, 1, 514), dtype=torch.float16, device="cuda")
    cos, sin = tables(4, 514, "float16")
    with pytest.raises(Exception, match="512"):
        abi.rope_append(x, x, x, x, cos, sin, 0, 514)
    y = torch.zeros((1, 1, 1, 64), dtype=torch.float16, device="cuda")
    with pytest.raises(Exception, match="rotary"):
        abi.rope_append(y, y, y, y, cos, sin, 0, 63)
    with pytest.raises(Exception, match="rotary"):
        abi.rope(y, y, cos, sin, 0, 66)
    with pytest.raises(Exception, match="both"):
        abi.rope_append(y, y, y, y, cos, sin, 0, 64, ks=torch.ones((1, 1, 1, 1), device="cuda"),
                        vs=None)


@pytest.mark.parametrize("quantized", [False, True])
def test_fused_cached_decode_is_bitwise_the_two_step_path(quantized):
    say(f"LM fused RoPE append int8 {quantized}")
    ts.seed(21)
    cfg = nn.TransformerConfig(61, dim=256, num_heads=4, num_kv_heads=2, num_layers=2,
                               max_seq_len=64)
    model = nn.TransformerLM(cfg, device="hip").eval()
    model.to(dtype="float16")
    tokens = ts.tensor(np.random.default_rng(21).integers(0, 61, (2, 24)), device="hip")
    fused_calls = []
    original = KVCache._append_rotary

    def counting(self, *args, **kw):
        done = original(self, *args, **kw)
        fused_calls.append(done)
        return done

    def run():
        caches = model.new_cache(2, quantized=quantized)
        parts = [model(tokens[:, :20], caches=caches).numpy()]
        for t in range(20, 24):
            parts.append(model(tokens[:, t:t + 1], caches=caches).numpy())
        return np.concatenate(parts, axis=1), [c.storage for c in caches]

    # the fused projection kernel (one launch for projections, RoPE and the
    # append) switched off: this is the path for what it does not take
    with ts.no_grad(), patch.object(KVCache, "_project_append", lambda *a, **k: None):
        with patch.object(KVCache, "_append_rotary", counting):
            got, got_store = run()
        with patch.object(KVCache, "_append_rotary", lambda self, *a, **k: False):
            want, want_store = run()
    assert fused_calls and all(fused_calls)
    np.testing.assert_array_equal(got, want)
    for a, b in zip(got_store, want_store):
        for x, y in zip(a, b):
            if x is not None:
                assert torch.equal(x, y)


FUSED_CASES = [
    # (dtype, B, Hq, Hkv, Sq, Sk, D, R, causal, offset, q_pos0, k_pos0); D may be (Dqk, Dv)
    ("bfloat16", 2, 2, 2, 200, 200, 128, 128, True, 0, 0, 0),
    ("float16", 1, 4, 2, 130, 257, 64, 64, True, 127, 127, 0),
    ("bfloat16", 2, 2, 1, 77, 150, 128, 64, False, 0, 9, 3),
    ("float16", 1, 2, 2, 256, 256, 128, 96, True, 0, 5, 5),
    ("bfloat16", 1, 2, 2, 90, 120, (128, 64), 128, True, 30, 30, 0),
    ("float16", 2, 4, 2, 100, 140, 32, 32, True, 40, 40, 0),  # head dim 32
]


@pytest.mark.parametrize("case", FUSED_CASES, ids=lambda c: "-".join(map(str, c)))
def test_rope_folded_into_attention_is_bitwise_the_unfused_chain(case):
    dtype, b, hq, hkv, sq, sk, d, r, causal, off, qp, kp = case
    say(f"fused rope attention {case}")
    d, dv = d if isinstance(d, tuple) else (d, d)
    rng = np.random.default_rng(sq + d)
    q, k, v, g = (abi.dev_tensor(rows(rng, shape, dtype, 0.7), dtype)
                  for shape in ((b, hq, sq, d), (b, hkv, sk, d), (b, hkv, sk, dv), (b, hq, sq, dv)))
    cos, sin = tables(max(qp + sq, kp + sk) + 1, r, dtype)
    rot = lambda x, pos, inv=False: _rot(x, cos, sin, pos, r, inv)
    k_rot = rot(k, kp)
    kw = dict(causal=causal, offset=off)
    # unfused chain
    out_u, lse_u, _ = abi.forward(rot(q, qp), k_rot, v, **kw)
    dq_r, dk_r, dv_u, _ = abi.backward(rot(q, qp), k_rot, v, out_u, g, lse_u, **kw)
    dq_u, dk_u = rot(dq_r, qp, True), rot(dk_r, kp, True)
    # folded
    desc = abi.rope_desc(cos, sin, r, qp, kp)
    out_f, lse_f, path = abi.forward_rope(q, k_rot, v, desc, **kw)
    assert path == _lib.PATH_MFMA
    dq_f, dk_f, dv_f = abi.backward_rope(q, k_rot, v, out_f, g, lse_f, desc, **kw)
    torch.cuda.synchronize()
    for name, a_, b_ in (("O", out_f, out_u), ("LSE", lse_f, lse_u), ("dQ", dq_f, dq_u),
                         ("dK", dk_f, dk_u), ("dV", dv_f, dv_u)):
        assert torch.equal(a_, b_), name
    # with a rotated-query buffer: the forward stores tsattn_rope(q) there and
    # the backward reads it -- the same bits as without, in the stored-dS
    # pipeline (the queried workspace) and in the recomputing one (a
    # workspace holding only the row values and the staged queries)
    rows_bytes = (2 * b * hq * sq * 4 + 255) // 256 * 256 + b * hq * sq * d * 2
    want = {None: (dq_f, dk_f, dv_f),
            rows_bytes: abi.backward_rope(q, k_rot, v, out_f, g, lse_f, desc, ws_bytes=rows_bytes, **kw)}
    q_rot = torch.full((b, hq, sq, d), 7.0, dtype=q.dtype, device=q.device)
    desc.q_rotated = q_rot.data_ptr()
    out_r, lse_r, _ = abi.forward_rope(q, k_rot, v, desc, **kw)
    torch.cuda.synchronize()
    assert torch.equal(q_rot, rot(q, qp)), "rotated queries"
    assert torch.equal(out_r, out_u) and torch.equal(lse_r, lse_u)
    for ws, grads in want.items():
        got = abi.backward_rope(q, k_rot, v, out_r, g, lse_r, desc, ws_bytes=ws, **kw)
        torch.cuda.synchronize()
        for name, a_, b_ in zip(("dQ", "dK", "dV"), got, grads):
            assert torch.equal(a_, b_), f"{name} with the rotated-query buffer, workspace {ws}"


DECODE_CASES = [
    # (dtype, B, Hq, Hkv, Sq, cached keys L, D, rotary dim, int8 cache)
    ("float16", 4, 8, 2, 1, 700, 128, 128, False),
    ("bfloat16", 2, 4, 4, 2, 300, 64, 32, False),   # two new rows, partial rotary dim
    ("float16", 2, 4, 1, 1, 1000, 256, 128, False),  # D = 256, half of it rotated
    ("bfloat16", 3, 8, 2, 1, 513, 128, 128, True),
    ("float16", 2, 2, 2, 4, 260, 64, 64, True),
    ("bfloat16", 2, 8, 1, 1, 400, 128, 64, False),  # 8 query rows per KV head (the maximum)
    ("float16", 1, 4, 2, 4, 333, 128, 128, True),   # 4 heads x 2 rows per KV head
]


@pytest.mark.parametrize("case", DECODE_CASES, ids=lambda c: "-".join(map(str, c)))
def test_decode_with_folded_rope_is_bitwise_the_two_step_path(case):
    """tsattn_decode_forward_rope == tsattn_rope on q, then the decode kernel."""
    dtype, b, hq, hkv, sq, klen, d, r, q8 = case
    say(f"decode folded rope {case}")
    rng = np.random.default_rng(klen + d)
    q0 = klen - sq  # the new rows' positions: the last sq of the cache
    q = abi.dev_tensor(rows(rng, (b, hq, sq, d), dtype, 0.7), dtype)
    k, v = (abi.dev_tensor(rows(rng, (b, hkv, klen, d), dtype, 0.7), dtype) for _ in range(2))
    cos, sin = tables(klen + 1, r, dtype)
    desc = abi.rope_desc(cos, sin, r, q0, 0)
    q_rot = _rot(q, cos, sin, q0, r, False)
    kw = dict(causal=True, offset=q0)
    if q8:
        codes = [torch.zeros((b, hkv, klen, d), dtype=torch.int8, device="cuda") for _ in range(2)]
        scales = [torch.ones((b, hkv, klen, 1), dtype=torch.float32, device="cuda") for _ in range(2)]
        abi.kv_append_int8(k, codes[0], scales[0], 0)
        abi.kv_append_int8(v, codes[1], scales[1], 0)
        want, path = abi.decode_int8(q_rot, codes[0], codes[1], scales[0], scales[1], klen, **kw)
        got = abi.decode_rope(q, codes[0], codes[1], desc, ks=scales[0], vs=scales[1],
                              len_kv=klen, **kw)
    else:
        want = abi.decode(q_rot, k, v, **kw)
        got = abi.decode_rope(q, k, v, desc, **kw)
    torch.cuda.synchronize()
    assert _lib.load().tsattn_last_kernel_path() == _lib.PATH_DECODE
    assert torch.equal(got, want)


def _rot(x, cos, sin, pos, r, inverse):
    out = torch.empty_like(x)
    abi.rope(x, out, cos, sin, pos, r, inverse)
    return out


def test_rope_folded_with_a_general_mask():
    dtype, b, h, s, d = "bfloat16", 2, 2, 150, 128
    rng = np.random.default_rng(7)
    q, k, v, g = (abi.dev_tensor(rows(rng, (b, h, s, d), dtype, 0.7), dtype) for _ in range(4))
    mask = torch.from_numpy(rng.random((s, s)) > 0.2).cuda()
    cos, sin = tables(s + 1, d, dtype)
    k_rot = _rot(k, cos, sin, 0, d, False)
    out_u, lse_u, _ = abi.forward(_rot(q, cos, sin, 0, d, False), k_rot, v, causal=True, mask=mask)
    grads_u = abi.backward(_rot(q, cos, sin, 0, d, False), k_rot, v, out_u, g, lse_u, causal=True,
                           mask=mask)[:3]
    desc = abi.rope_desc(cos, sin, d, 0, 0)
    out_f, lse_f, _ = abi.forward_rope(q, k_rot, v, desc, causal=True, mask=mask)
    dq_f, dk_f, dv_f = abi.backward_rope(q, k_rot, v, out_f, g, lse_f, desc, causal=True, mask=mask)
    torch.cuda.synchronize()
    assert torch.equal(out_f, out_u) and torch.equal(lse_f, lse_u)
    assert torch.equal(dq_f, _rot(grads_u[0], cos, sin, 0, d, True))
    assert torch.equal(dk_f, _rot(grads_u[1], cos, sin, 0, d, True))
    assert torch.equal(dv_f, grads_u[2])


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_rope_folded_with_dropout_is_bitwise_the_unfused_chain(dtype):
    """RoPE folded in and dropout together: the same keep bits, the same
    outputs and gradients as rotating first and dropping on the plain kernels."""
    b, hq, hkv, s, d = 2, 4, 2, 160, 128
    say(f"fused rope + dropout {dtype}")
    rng = np.random.default_rng(99)
    q, k, v, g = (abi.dev_tensor(rows(rng, shape, dtype, 0.7), dtype)
                  for shape in ((b, hq, s, d), (b, hkv, s, d), (b, hkv, s, d), (b, hq, s, d)))
    cos, sin = tables(s + 1, d, dtype)
    k_rot = _rot(k, cos, sin, 0, d, False)
    kw = dict(causal=True, dropout=(0.2, 0xABCDEF0123456789, 5))
    bits_u = abi.dropout_bits_buffer(q, k, v, **kw)
    q_rot = _rot(q, cos, sin, 0, d, False)
    out_u, lse_u, _ = abi.forward(q_rot, k_rot, v, dropout_bits=bits_u, **kw)
    dq_r, dk_r, dv_u, _ = abi.backward(q_rot, k_rot, v, out_u, g, lse_u, dropout_bits=bits_u, **kw)
    desc = abi.rope_desc(cos, sin, d, 0, 0)
    bits_f = abi.dropout_bits_buffer(q, k, v, **kw)
    out_f, lse_f, path = abi.forward_rope(q, k_rot, v, desc, dropout_bits=bits_f, **kw)
    assert path == _lib.PATH_MFMA
    dq_f, dk_f, dv_f = abi.backward_rope(q, k_rot, v, out_f, g, lse_f, desc, dropout_bits=bits_f,
                                         **kw)
    torch.cuda.synchronize()
    assert torch.equal(bits_f, bits_u)
    assert torch.equal(out_f, out_u) and torch.equal(lse_f, lse_u)
    assert torch.equal(dq_f, _rot(dq_r, cos, sin, 0, d, True))
    assert torch.equal(dk_f, _rot(dk_r, cos, sin, 0, d, True))
    assert torch.equal(dv_f, dv_u)


def test_rope_folded_refuses_problems_outside_the_mfma_kernels():
    q = torch.zeros((1, 1, 8, 32), dtype=torch.float32, device="cuda")
    cos, sin = tables(9, 32, "float32")
    desc = abi.rope_desc(cos, sin, 32, 0, 0)
    with pytest.raises(NotImplementedError, match="tsattn_rope"):
        abi.forward_rope(q, q, q, desc)
    h = torch.zeros((1, 1, 8, 96), dtype=torch.float16, device="cuda")  # D = 96: not an MFMA shape
    c16, s16 = tables(9, 96, "float16")
    with pytest.raises(NotImplementedError):
        abi.forward_rope(h, h, h, abi.rope_desc(c16, s16, 96, 0, 0))
    with pytest.raises(ValueError, match="rotary"):
        abi.forward_rope(h, h, h, abi.rope_desc(c16, s16, 97, 0, 0))


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_attention_module_fused_rope_is_bitwise_the_two_step_path(dtype):
    from tensorsmith_hip.nn import attention as attn_mod
    from tensorsmith_hip.nn import transformer as tr_mod

    say(f"MHA fused rope {dtype}")
    plain = attn_mod.scaled_dot_product_attention

    def two_step(q, k, v, *args, _rope=None, **kw):
        if _rope is not None:
            q = attn_mod.rotary_embedding(q, _rope[0], _rope[2])
            k = attn_mod.rotary_embedding(k, _rope[1], _rope[2])
        return plain(q, k, v, *args, **kw)

    def step(patched):
        ts.seed(5)
        mha = nn.MultiHeadAttention(256, 2, num_kv_heads=1, device="hip")
        mha.to(dtype=dtype)
        x = ts.tensor(np.random.default_rng(5).standard_normal((2, 96, 256)).astype(np.float32),
                      device="hip", dtype=dtype, requires_grad=True)
        _lib.profile_enable(True)
        _lib.profile_reset()
        gy = ts.tensor(np.random.default_rng(6).standard_normal((2, 96, 256)).astype(np.float32),
                       device="hip", dtype=dtype)
        if patched:
            with patch.object(tr_mod, "scaled_dot_product_attention", two_step):
                y = mha(x, is_causal=True)
                y.backward(gy)
        else:
            y = mha(x, is_causal=True)
            y.backward(gy)
        probes = _lib.profile_read()
        _lib.profile_enable(False)
        grads = [p.grad.numpy() for p in mha.parameters()] + [x.grad.numpy()]
        return y.numpy(), grads, probes

    y_f, g_f, probes_f = step(False)
    y_u, g_u, probes_u = step(True)
    assert probes_f["rope"][0] == 1 and probes_u["rope"][0] == 4  # keys only / q, k and both VJPs
    np.testing.assert_array_equal(y_f, y_u)
    for a_, b_ in zip(g_f, g_u):
        np.testing.assert_array_equal(a_, b_)


def test_rope_attention_in_float64_rotates_then_attends():
    """float64 has no RoPE kernel: the mirror rotates with rotary_embedding
    and runs the generic kernels -- against the oracle's float64 RoPE and
    dense attention, forward and VJP (1e-10)."""
    from tensorsmith_hip.nn import attention as attn_mod

    rng = np.random.default_rng(8)
    q, k, v, g = (rng.standard_normal((1, 2, 40, 16)) for _ in range(4))
    tq, tk, tv = (ts.tensor(a, device="hip", dtype="float64", requires_grad=True) for a in (q, k, v))
    out = attn_mod.scaled_dot_product_attention(tq, tk, tv, is_causal=True, _rope=(3, 3, 10000.0))
    out.backward(ts.tensor(g, device="hip", dtype="float64"))
    qr, kr = R.rope(q, 3, dtype="float64"), R.rope(k, 3, dtype="float64")
    ref = A.sdpa(qr, kr, v, None, True, dtype="float64", backend="dense")
    dq_r, dk_r, dv = ref.backward(g)
    want = (ref.out, R.rope(dq_r, 3, dtype="float64", inverse=True),
            R.rope(dk_r, 3, dtype="float64", inverse=True), dv)
    for got, w in zip((out.numpy(), tq.grad.numpy(), tk.grad.numpy(), tv.grad.numpy()), want):
        np.testing.assert_allclose(got, w, rtol=1e-10, atol=1e-10)


def test_rope_folded_backward_takes_an_expanded_upstream_gradient():
    """An upstream gradient with stride 0 (an expand, as a sum's VJP gives)
    cannot be read by the MFMA kernels as it is: the mirror makes it
    contiguous and the folded backward runs -- same bits as the two-step
    path (rotary_embedding, plain attention)."""
    from tensorsmith_hip.nn import attention as attn_mod

    rng = np.random.default_rng(12)
    b, h, s, d = 1, 2, 96, 64
    q, k, v = (rng.standard_normal((b, h, s, d)).astype(np.float32) for _ in range(3))
    g_row = torch.from_numpy(rng.standard_normal((1, 1, 1, d)).astype(np.float32))

    def run(fused):
        tq, tk, tv = (ts.tensor(a, device="hip", dtype="bfloat16", requires_grad=True) for a in (q, k, v))
        up = ts.Tensor(g_row.to("cuda", torch.bfloat16).expand(b, h, s, d), device="hip")
        if fused:
            out = attn_mod.scaled_dot_product_attention(tq, tk, tv, is_causal=True, _rope=(0, 0, 10000.0))
        else:
            out = attn_mod.scaled_dot_product_attention(attn_mod.rotary_embedding(tq, 0),
                                                        attn_mod.rotary_embedding(tk, 0), tv, is_causal=True)
        out.backward(up)
        return [out.numpy()] + [t.grad.numpy() for t in (tq, tk, tv)]

    for a_, b_ in zip(run(True), run(False)):
        np.testing.assert_array_equal(a_, b_)
