"""The attention workloads at full size (needs an MI355X).

Every (batch, head) pair is checked against the oracle, each on its own at the
bounds of test_gpu_parity.py (bf16: rel-L2 1e-2 for O, 2e-2 for gradients,
max-abs 2e-2 * max|ref|; fp16: 2e-3 / 5e-3, 5e-3 * max|ref|; LSE max-abs
1e-3): the XCD-aware, heaviest-first grid order sends each head to its own
schedule slot, so a head-dependent indexing mistake cannot hide behind a
sample.  The causal bf16 fwd+bwd at B16 H16 S2048 D128 checks O, LSE, dQ, dK
and dV of all 256 heads; the fp16 decode at B64 H32 all 2048 heads; the 32k
key-padded prefill all 64 heads at every 16th 64-row query block, the blocks
around each sequence's valid length (L - 1 and L among them) and the last
block; the causal fwd+bwd at S8192 (stored dS in chunks) sampled heads from
every chunk.
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


def check_heads(got, ref, dtype, kind, name):
    """check_half's bounds for every (batch, head) slice of [B, H, ...] arrays;
    prints the worst pair."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.isfinite(got).all(), name
    b, h = ref.shape[:2]
    d = (got - ref).reshape(b, h, -1)
    r = ref.reshape(b, h, -1)
    norm = np.linalg.norm(r, axis=-1)
    rel = np.linalg.norm(d, axis=-1) / np.where(norm > 0, norm, 1.0)
    scale = np.abs(r).max(axis=-1)
    mx = np.abs(d).max(axis=-1) / np.where(scale > 0, scale, 1.0)
    wb, wh = np.unravel_index(np.argmax(rel), rel.shape)
    say(f"  {name}: {b * h} heads, worst rel_l2={rel.max():.2e} (b{wb} h{wh}), "
        f"worst max_abs/max|ref|={mx.max():.2e}")
    from test_gpu_parity import TOL
    bad = np.argwhere(rel > TOL[dtype][kind])
    assert not bad.size, f"{name}: rel_l2 over bound at (b, h) {bad[:8].tolist()}"
    bad = np.argwhere(mx > TOL[dtype]["mx"])
    assert not bad.size, f"{name}: max-abs over bound at (b, h) {bad[:8].tolist()}"


def check_lse_heads(got, ref, name):
    np.testing.assert_array_equal(np.isneginf(got), np.isneginf(ref), err_msg=name)
    live = np.isfinite(ref)
    err = np.abs(np.where(live, got - ref, 0.0))
    say(f"  {name}: lse max-abs={err.max():.2e}")
    assert err.max() <= 1e-3, name


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
    hg = host(g)
    for b0 in range(0, 16, 2):  # the oracle two batch rows at a time (all 16 heads)
        sl = slice(b0, b0 + 2)
        ref = A.sdpa(host(q[sl]), host(k[sl]), host(v[sl]), None, True, dtype="bfloat16",
                     backend="streaming")
        check_heads(host(out[sl]), ref.out, "bfloat16", "o", f"O b{b0}-{b0 + 1}")
        check_lse_heads(host(lse[sl]), ref.lse[..., 0], f"LSE b{b0}-{b0 + 1}")
        for got, want, n in zip((dq, dk, dv), ref.backward_compute(hg[sl]), ("dQ", "dK", "dV")):
            check_heads(host(got[sl]), want, "bfloat16", "g", f"{n} b{b0}-{b0 + 1}")


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
    for b in range(B):  # every sequence, all 32 heads
        L = int(lens[b])
        ref = A.sdpa(host(q[b:b + 1]), host(k[b:b + 1, :, :L]), host(v[b:b + 1, :, :L]), None,
                     False, dtype="float16", backend="dense")
        check_heads(got[b:b + 1], ref.out, "float16", "o", f"decode b{b} len{L}")


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
    # Every head at every 16th 64-row block across the whole sequence (each
    # (head, query block) runs in a schedule slot of its own), plus the blocks
    # around the valid length L and the last block.  Rows r0 .. r0 + 63 see
    # keys below min(r0 + 64, L) only, so the oracle takes that prefix.
    for b in range(B):  # all 32 heads of each sequence at once
        L = int(lens[b])
        kh, vh = host(k[b:b + 1]), host(v[b:b + 1])
        r_mid = min(max(L - 32, 0), S - 64)
        starts = sorted(set(range(0, S, 16 * 64)) | {r_mid, (L // 64) * 64 if L < S else S - 64,
                                                     S - 64})
        for r0 in starts:
            kend = min(r0 + 64, S)
            ref = A.sdpa(host(q[b:b + 1, :, r0:r0 + 64]), kh[:, :, :kend], vh[:, :, :kend],
                         kmh[b][None, None, None, :kend], True, dtype="bfloat16",
                         causal_offset=r0, backend="dense")
            check_heads(host(out._data[b:b + 1, :, r0:r0 + 64]), ref.out, "bfloat16", "o",
                        f"prefill b{b} rows {r0}..{r0 + 63} (len {L})")


def test_long_causal_fwd_bwd_bf16_b16h16s8192d128_chunked_stored_ds():
    """B16 H16 S8192 D128 causal bf16: the stored dS of all 256 heads (17.4 GB)
    exceeds the backward's 8 GiB region, so the stored-dS pipeline runs over
    chunks of heads that reuse one region -- dK/dV (storing the chunk's dS),
    then dQ = dS K, per chunk -- instead of the kernels that recompute S and
    dP for dQ.  Heads from every chunk (the first and the last of the problem
    among them) against the oracle at the bf16 bounds."""
    gen = torch.Generator(device="cuda").manual_seed(7)
    shape = (16, 16, 8192, 128)
    q, k, v = (draw(gen, shape, 0.5, torch.bfloat16) for _ in range(3))
    g = draw(gen, shape, 1.0, torch.bfloat16)
    say("full-size bf16 causal fwd+bwd at S8192 (chunked stored dS)")
    out, lse, path = abi.forward(q, k, v, causal=True)
    assert path == _lib.PATH_MFMA
    _lib.profile_enable(True)
    _lib.profile_reset()
    dq, dk, dv, bpath = abi.backward(q, k, v, out, g, lse, causal=True)
    torch.cuda.synchronize()
    probes = _lib.profile_read()
    _lib.profile_enable(False)
    assert bpath == _lib.PATH_MFMA
    assert "bwd_dq_mfma" not in probes, sorted(probes)
    chunks = probes["bwd_dq_ds"][0]
    assert chunks >= 3 and probes["bwd_dkdv_mfma"][0] == chunks, probes
    say(f"  {chunks} chunks of stored dS")
    for t in (out, lse, dq, dk, dv):
        assert torch.isfinite(t).all()
    # 256 heads in `chunks` chunks of consecutive (b, head) groups: sample the
    # first and last head of each chunk and one in its middle
    per = -(-256 // chunks)
    heads = sorted({x for c0 in range(0, 256, per) for x in (c0, min(c0 + per, 256) - 1, c0 + per // 2)
                    if x < 256})
    for bh in heads:
        b, h = divmod(bh, 16)
        sl = (slice(b, b + 1), slice(h, h + 1))
        ref = A.sdpa(host(q[sl]), host(k[sl]), host(v[sl]), None, True, dtype="bfloat16",
                     backend="streaming", block_size=1024)
        check_heads(host(out[sl]), ref.out, "bfloat16", "o", f"O b{b} h{h}")
        check_lse_heads(host(lse[sl]), ref.lse[..., 0], f"LSE b{b} h{h}")
        for got, want, n in zip((dq, dk, dv), ref.backward_compute(host(g[sl])), ("dQ", "dK", "dV")):
            check_heads(host(got[sl]), want, "bfloat16", "g", f"{n} b{b} h{h}")
