"""Decoder-only TransformerLM and cached generation on the hip device -- the
reference's own LM tests (tests/test_transformer.py:287-407), run through
``tensorsmith_hip`` (needs an MI355X).

Tolerances are the reference's: cached vs full-prefix logits rtol 3e-4 /
atol 3e-5 in fp32 (:330-331), the int8 cache rtol 0.08 / atol 0.006 (:335),
exact token equality for greedy generation (:376).  The half-precision case
checks cached decode logits against the full-prefix forward at the stated
fp16 bound (relative L2 <= 5e-3) and that the one-token steps ran on the
split-K decode kernel.
"""

from __future__ import annotations

from unittest.mock import patch

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("no GPU", allow_module_level=True)

import tensorsmith_hip as ts  # noqa: E402
from conftest import rel_l2  # noqa: E402
from tensorsmith_hip import _lib, nn  # noqa: E402
from tensorsmith_hip.nn import functional as F  # noqa: E402

HIP = "hip"


def tok(rows):
    return ts.tensor(np.asarray(rows, dtype=np.int64), device=HIP)


def test_failed_model_forward_rolls_back_cache_lengths():
    ts.seed(1)
    model = nn.TransformerLM(nn.TransformerConfig(11, dim=16, num_heads=2, num_layers=2,
                                                  max_seq_len=8), device=HIP).eval()
    caches = model.new_cache(1)
    x = tok([[1, 2]])
    with ts.no_grad():
        model(x, caches=caches)
        with patch.object(model.blocks[1], "forward", side_effect=ValueError("bad layer")):
            with pytest.raises(ValueError):
                model(x, caches=caches)
        assert [c.length for c in caches] == [2, 2]
        with pytest.raises(ValueError):
            model(x, caches=caches, attn_mask=ts.zeros(7, 7, device=HIP))
        assert [c.length for c in caches] == [2, 2]


@pytest.mark.parametrize("backend", ["auto", "streaming", "hip"])
def test_cached_logits_match_full_prefix(backend):
    ts.seed(2)
    model = nn.TransformerLM(nn.TransformerConfig(17, dim=16, num_heads=4, num_kv_heads=2,
                                                  num_layers=2, max_seq_len=16,
                                                  attention_backend=backend), device=HIP).eval()
    tokens = tok([[1, 2, 3, 4, 5, 6], [4, 3, 2, 1, 0, 7]])
    with ts.no_grad():
        expected = model(tokens).numpy()
        caches = model.new_cache(2)
        chunks = [model(tokens[:, :3], caches=caches), model(tokens[:, 3:5], caches=caches),
                  model(tokens[:, 5:], caches=caches)]
        np.testing.assert_allclose(ts.cat(chunks, dim=1).numpy(), expected, rtol=3e-4, atol=3e-5)
        assert all(c.length == 6 for c in caches)
        quantized = model.new_cache(2, quantized=True)
        actual = model(tokens, caches=quantized).numpy()
        np.testing.assert_allclose(actual, expected, rtol=0.08, atol=0.006)


def test_causal_no_future_leakage_and_gradients():
    ts.seed(3)
    model = nn.TransformerLM(nn.TransformerConfig(11, dim=16, num_heads=4, num_kv_heads=1,
                                                  num_layers=2, max_seq_len=8), device=HIP)
    tokens = tok([[1, 2, 3, 4]])
    logits = model(tokens)
    altered = model(tok([[1, 2, 9, 8]]))
    np.testing.assert_allclose(logits.numpy()[:, :2], altered.numpy()[:, :2], atol=1e-6)
    loss = F.cross_entropy(logits, tok([[2, 3, 4, 5]]), axis=-1)
    loss.backward()
    parameters = list(model.parameters())
    assert all(p.grad is not None and np.isfinite(p.grad.numpy()).all() for p in parameters)
    assert sum(p is model.token_embedding.weight for p in parameters) == 1
    clone = nn.TransformerLM(model.config, device=HIP)
    clone.load_state_dict(model.state_dict())
    np.testing.assert_allclose(clone(tokens).numpy(), logits.numpy(), atol=1e-6)
    np.testing.assert_allclose(model(tokens, logits_to_keep=1).numpy(), logits.numpy()[:, -1:],
                               atol=1e-6)
    with pytest.raises(ValueError):
        model(tokens, logits_to_keep=5)


def test_greedy_generation_cache_equivalence_and_mode():
    ts.seed(4)
    model = nn.TransformerLM(nn.TransformerConfig(13, dim=16, num_heads=4, num_kv_heads=1,
                                                  num_layers=1, max_seq_len=12), device=HIP)
    model.blocks[0].ffn.eval()
    modes = [m.training for m in model.modules()]
    prompt = tok([[1, 2, 3], [3, 1, 2]])
    cached = model.generate(prompt, 5, temperature=0)
    uncached = model.generate(prompt, 5, temperature=0, use_cache=False)
    np.testing.assert_array_equal(cached.numpy(), uncached.numpy())
    assert [m.training for m in model.modules()] == modes
    assert not cached.requires_grad
    assert model.generate(prompt, 0).shape == prompt.shape


def test_sampling_filters_and_eos():
    ts.seed(5)
    logits = ts.tensor(np.array([[1.0, 2.0, 9.0, 0.0]] * 128, dtype=np.float32), device=HIP)
    np.testing.assert_array_equal(nn.sample_logits(logits, top_k=1).numpy(), 2)
    np.testing.assert_array_equal(nn.sample_logits(logits, top_p=0.1).numpy(), 2)
    sampled = nn.sample_logits(logits, temperature=10, top_k=2).numpy()
    assert np.isin(sampled, [1, 2]).all()
    with patch("tensorsmith_hip.nn.transformer.random_uniform",
               return_value=logits._data[:, :1] * 0 + (1 - 2**-24)):
        sampled = nn.sample_logits(logits, temperature=10, top_k=2).numpy()
        assert np.isin(sampled, [1, 2]).all()
    with pytest.raises(ValueError):
        nn.sample_logits(logits, top_k=5)
    model = nn.TransformerLM(nn.TransformerConfig(4, dim=8, num_heads=2, num_layers=1,
                                                  max_seq_len=8), device=HIP)
    with patch("tensorsmith_hip.nn.transformer.sample_logits",
               return_value=ts.tensor(np.array([2]), device=HIP)):
        result = model.generate(tok([[1]]), 5, eos_token_id=2)
        np.testing.assert_array_equal(result.numpy(), [[1, 2]])


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_half_precision_cached_decode_runs_split_k_kernel(dtype):
    """Prefill 200 tokens, then one-token steps over the caches: the steps run
    on the decode kernel and match the full-prefix logits."""
    ts.seed(6)
    cfg = nn.TransformerConfig(101, dim=512, num_heads=4, num_kv_heads=2, num_layers=2,
                               max_seq_len=256)
    model = nn.TransformerLM(cfg, device=HIP).eval()
    model.to(dtype=dtype)
    tokens = tok(np.random.default_rng(6).integers(0, 101, (2, 203)))
    with ts.no_grad():
        full = model(tokens).numpy().astype(np.float32)
        caches = model.new_cache(2)
        parts = [model(tokens[:, :200], caches=caches).numpy().astype(np.float32)]
        for t in range(200, 203):
            parts.append(model(tokens[:, t:t + 1], caches=caches).numpy().astype(np.float32))
            assert _lib.last_kernel_path() == _lib.PATH_DECODE
    got = np.concatenate(parts, axis=1)
    tol = 5e-3 if dtype == "float16" else 2e-2
    assert rel_l2(got, full) <= tol
    assert all(c.length == 203 for c in caches)
