"""int8 KV cache on the device: the fused quantising append and the decode
kernel that dequantises inside (needs an MI355X).

* Append: bit-exact against the oracle's restatement of the reference
  quantiser (src/tensorsmith/nn/cache.py:73-77) -- codes and fp32 scales --
  for f32 / f16 / bf16 rows, including all-zero rows (scale 1e-8) and values
  exactly half-way between two codes (round half to even), at an offset
  position and from a strided (permuted) source.
* Decode: against the fp32 oracle attention over the dequantised cache
  (codes * scale in fp32), at the fp16/bf16 bounds of the parity tests
  (relative L2 <= 2e-3 / 1e-2, max-abs <= 5e-3 / 2e-2 of max|ref|), for
  uniform and ragged (kv_len) lengths; and against the reference's order
  (dequantise, round to the cache dtype, then attend) within the same bound.
* Model level: an fp16 TransformerLM with a quantised cache projects, rotates
  and appends through the fused projection kernel and decodes through the
  int8 kernel (their timing probes fire) and agrees with the same steps
  taken in the reference's order (dequantised fp16 views, fp decode kernel)
  at the fp16 bound; both stay within relative L2 3e-2 of the unquantised
  model.  (The reference's rtol 0.08 / atol 0.006 int8 check,
  tests/test_transformer.py:335, is run at its own model size in
  test_gpu_lm.py.)
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
from oracle import attention as A  # noqa: E402
from oracle.halfprec import round_to  # noqa: E402
from tensorsmith_hip import _lib, nn  # noqa: E402


def say(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("dim", [64, 128, 256])
def test_append_is_bit_exact_with_the_reference_quantiser(dtype, dim):
    say(f"append int8 {dtype} D{dim}")
    rng = np.random.default_rng(dim)
    b, h, t, pos, cap = 3, 4, 7, 5, 16
    x = rng.standard_normal((b, t, h, dim)).astype(np.float32) * 3
    x[0, 1] = 0.0  # all-zero rows: scale 1e-8, codes 0
    # rows whose max is 127 (scale 1.0 exactly) holding k + 0.5 values: ties
    x[1, 2, :, :] = (np.arange(dim) % 9 - 4).astype(np.float32) + 0.5
    x[1, 2, :, 0] = 127.0
    x = round_to(x, dtype)
    src = abi.dev_tensor(x, dtype).permute(0, 2, 1, 3)  # [B,H,T,D] strided view
    codes = torch.zeros((b, h, cap, dim), dtype=torch.int8, device="cuda")
    scales = torch.ones((b, h, cap, 1), dtype=torch.float32, device="cuda")
    abi.kv_append_int8(src, codes, scales, pos)
    want_q, want_s = A.quantize_int8(x.transpose(0, 2, 1, 3))
    np.testing.assert_array_equal(codes[:, :, pos:pos + t].cpu().numpy(), want_q)
    np.testing.assert_array_equal(scales[:, :, pos:pos + t].cpu().numpy(), want_s)
    assert (codes[:, :, :pos] == 0).all() and (codes[:, :, pos + t:] == 0).all()
    assert (scales[:, :, :pos] == 1).all() and (scales[:, :, pos + t:] == 1).all()
    assert (codes[1, :, pos + 2] == torch.as_tensor(want_q[1, :, 2], device="cuda")).all()


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("d,t", [(64, 509), (128, 512), (256, 501)])
def test_append_many_rows_bit_exact_near_rounding_ties(dtype, d, t):
    """Thousands of rows through the vectorised append, with row counts per
    head that do and do not fill the kernel's row chunks: random rows (whose
    quotients come within 5e-5 of a half-integer many times: the kernel
    multiplies by 1 / scale and divides only there), rows whose quotients are
    exact half-integers (scale exactly 1), and rows of tiny values (scale at
    the 1e-8 floor); codes and scales bit-identical to the reference
    quantiser."""
    say(f"append int8 many rows {dtype} D{d} T{t}")
    rng = np.random.default_rng(11)
    b, h, pos = 2, 8, 3
    cap = pos + t + 5
    x = rng.standard_normal((b, h, t, d)).astype(np.float32) * 4
    # rows with max 127 (scale exactly 1): quotients k + 0.5 and their neighbours
    ties = (rng.integers(-120, 120, (b, h, 64, d)) + 0.5).astype(np.float32)
    ties[..., 0] = 127.0
    x[:, :, :64] = ties
    x[:, :, 64:96] *= np.float32(1e-9)  # scales at the 1e-8 floor
    x = round_to(x, dtype)
    src = abi.dev_tensor(x, dtype)
    codes = torch.zeros((b, h, cap, d), dtype=torch.int8, device="cuda")
    scales = torch.zeros((b, h, cap, 1), dtype=torch.float32, device="cuda")
    abi.kv_append_int8(src, codes, scales, pos)
    want_q, want_s = A.quantize_int8(x)
    np.testing.assert_array_equal(codes[:, :, pos:pos + t].cpu().numpy(), want_q)
    np.testing.assert_array_equal(scales[:, :, pos:pos + t].cpu().numpy(), want_s)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_append_scale_is_exact_for_every_16bit_row_maximum(dtype):
    """One row per finite non-negative fp16 / bf16 value m, holding m and
    smaller values of both signs: the kernel's division-free row scale
    max(m / 127, 1e-8) and every code equal the reference quantiser's, over
    the whole range of the format."""
    say(f"append int8 every row maximum {dtype}")
    if dtype == "float16":
        m = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    else:
        m = (np.arange(0, 0x7F80, dtype=np.uint32) << 16).view(np.float32)
    d = 64
    rng = np.random.default_rng(5)
    x = m[:, None] * rng.uniform(-1.0, 1.0, (m.size, d)).astype(np.float32)
    x[:, 0] = m
    x = round_to(x, dtype)
    rows = m.size
    x = x.reshape(1, 1, rows, d)
    src = abi.dev_tensor(x, dtype)
    codes = torch.zeros((1, 1, rows, d), dtype=torch.int8, device="cuda")
    scales = torch.zeros((1, 1, rows, 1), dtype=torch.float32, device="cuda")
    abi.kv_append_int8(src, codes, scales, 0)
    want_q, want_s = A.quantize_int8(x)
    np.testing.assert_array_equal(scales.cpu().numpy(), want_s)
    np.testing.assert_array_equal(codes.cpu().numpy(), want_q)


def _int8_cache(rng, b, hkv, cap, d, dtype):
    k = round_to(rng.standard_normal((b, hkv, cap, d)).astype(np.float32), dtype)
    v = round_to(rng.standard_normal((b, hkv, cap, d)).astype(np.float32), dtype)
    kq, ks = A.quantize_int8(k)
    vq, vs = A.quantize_int8(v)
    dev = lambda a, t: torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(t)
    return (kq, ks, vq, vs), (dev(kq, torch.int8), dev(ks, torch.float32), dev(vq, torch.int8),
                              dev(vs, torch.float32))


@pytest.mark.parametrize("dtype,rows", [("float16", 1), ("bfloat16", 4), ("float16", 8)])
@pytest.mark.parametrize("ragged", [False, True])
def test_int8_decode_matches_oracle_on_dequantised_cache(dtype, rows, ragged):
    say(f"int8 decode {dtype} rows{rows} ragged={ragged}")
    rng = np.random.default_rng(rows + 10 * ragged)
    b, hkv, d, cap, length = 4, 4, 128, 3072, 2900
    rep = rows
    hq = hkv * rep
    (kq, ks, vq, vs), (k8, ksd, v8, vsd) = _int8_cache(rng, b, hkv, cap, d, dtype)
    q = round_to(rng.standard_normal((b, hq, 1, d)).astype(np.float32), dtype)
    lens = rng.integers(200, length + 1, size=b).astype(np.int32) if ragged else np.full(b, length, np.int32)
    kw = {}
    if ragged:
        kw["kv_len"] = torch.from_numpy(lens).to("cuda")
    out, path = abi.decode_int8(abi.dev_tensor(q, dtype), k8, v8, ksd, vsd, length,
                                causal=True, offset=length - 1, **kw)
    assert path == _lib.PATH_DECODE
    got = abi.host(out)
    kf, vf = kq.astype(np.float32) * ks, vq.astype(np.float32) * vs  # fp32 dequantisation
    ref = np.zeros_like(got)
    ref_rd = np.zeros_like(got)
    for bi in range(b):
        n = lens[bi]
        sl = (slice(bi, bi + 1), slice(None), slice(0, n))
        kk = np.repeat(kf[sl], rep, axis=1)
        vv = np.repeat(vf[sl], rep, axis=1)
        ref[bi:bi + 1] = A.sdpa(q[bi:bi + 1], kk, vv, None, False, dtype="float32",
                                backend="dense").out
        # the reference's order: dequantise, round to the cache dtype, attend
        kr, vr = round_to(kk, dtype), round_to(vv, dtype)
        ref_rd[bi:bi + 1] = A.sdpa(q[bi:bi + 1], kr, vr, None, False, dtype="float32",
                                   backend="dense").out
    l2, mx = (2e-3, 5e-3) if dtype == "float16" else (1e-2, 2e-2)
    for want in (ref, ref_rd):
        assert rel_l2(got, want) <= l2
        assert np.abs(got - want).max() <= mx * np.abs(want).max()


def test_lm_with_int8_cache_decodes_through_the_int8_kernel():
    """Same prompt and steps twice over int8 caches: once through the int8
    kernel, once in the reference's order (an all-allowed key mask sends the
    steps through KVCache.get's dequantised fp16 views and the fp decode
    kernel).  The two agree at the fp16 bound; both sit within the
    quantisation error of the unquantised model (relative L2 <= 3e-2)."""
    say("LM int8 cache decode")
    ts.seed(8)
    cfg = nn.TransformerConfig(97, dim=512, num_heads=4, num_kv_heads=4, num_layers=2,
                               max_seq_len=256)
    model = nn.TransformerLM(cfg, device="hip").eval()
    model.to(dtype="float16")
    tokens = ts.tensor(np.random.default_rng(8).integers(0, 97, (2, 204)), device="hip")

    def run(reference_order: bool):
        caches = model.new_cache(2, quantized=True)
        parts = [model(tokens[:, :200], caches=caches).numpy().astype(np.float32)]
        _lib.profile_enable(True)
        _lib.profile_reset()
        for t in range(200, 204):
            mask = (ts.tensor(np.ones((2, 1, 1, t + 1), dtype=bool), device="hip")
                    if reference_order else None)
            parts.append(model(tokens[:, t:t + 1], caches=caches, attn_mask=mask)
                         .numpy().astype(np.float32))
        probes = _lib.profile_read()
        _lib.profile_enable(False)
        assert all(c.length == 204 for c in caches)
        return np.concatenate(parts, axis=1)[:, 200:], probes

    with ts.no_grad():
        full = model(tokens).numpy().astype(np.float32)[:, 200:]
        got, probes = run(False)
        want, probes_ref = run(True)
    assert probes["decode_split_int8"][0] == 4 * cfg.num_layers
    # one fused projection + RoPE + quantising append (q, K and V) per layer and step
    assert probes["qkv_rope_append_int8"][0] == 4 * cfg.num_layers
    assert "kv_append_int8" not in probes and "rope_append_int8" not in probes
    # the queries come out of it rotated: no separate RoPE launch
    assert "rope" not in probes and "rope" not in probes_ref
    assert "decode_split_int8" not in probes_ref and "decode_split" in probes_ref
    assert rel_l2(got, want) <= 5e-3
    assert np.abs(got - want).max() <= 5e-3 * np.abs(want).max()
    assert rel_l2(got, full) <= 3e-2 and rel_l2(want, full) <= 3e-2
