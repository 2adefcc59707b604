"""Activation checkpointing with attention dropout on the hip device (needs an
MI355X), and two mirror fall-backs around the folded-RoPE kernels.

* The reference's own test (tests/test_checkpoint.py:108-136): a 2-layer LM
  with dropout 0.2 trained once plainly and once with
  ``activation_checkpointing=True`` from the same seed gives the same loss
  (5 places) and gradients (rtol 2e-4, atol 2e-5) -- here with the attention
  dropout inside the kernels (backends "dense" and "hip", fp32 generic
  kernels) and, under fp16 autocast at head dim 64, on the MFMA kernels.
* The recomputation replays the attention-dropout keys of the first pass (the
  kernels' keep mask is a function of the key, so equal keys are equal
  masks); with the replay switched off the gradients no longer match, so the
  comparison above is sensitive to the mask.
* A float64 rotary MultiHeadAttention (generic kernels, operands rotated
  first) matches the NumPy oracle; the folded-RoPE backward accepts an
  expanded upstream gradient.
"""

from __future__ import annotations

import importlib
from dataclasses import replace
from unittest.mock import patch

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("no GPU", allow_module_level=True)

import tensorsmith_hip as ts  # noqa: E402
from oracle import attention as A  # noqa: E402
from oracle import rope as R  # noqa: E402
from tensorsmith_hip import _lib, nn  # noqa: E402

attn_mod = importlib.import_module("tensorsmith_hip.nn.attention")
HIP = "hip"


def say(msg):
    print(msg, flush=True)


def tok(rows):
    return ts.tensor(np.asarray(rows, dtype=np.int64), device=HIP)


def train_once(config, tokens, targets, seed, amp=False):
    ts.seed(123)
    model = nn.TransformerLM(config, device=HIP)
    ts.seed(seed)
    if amp:
        with ts.autocast(HIP):
            loss = model.loss(tokens, targets)
    else:
        loss = model.loss(tokens, targets)
    loss.backward()
    return loss.item(), [p.grad.numpy() for p in model.parameters()]


@pytest.mark.parametrize("backend", ["dense", "hip"])
def test_checkpoint_lm_training_matches_regular(backend):
    say(f"checkpointed LM, fp32, backend {backend}")
    config = nn.TransformerConfig(11, dim=16, num_heads=4, num_layers=2, dropout=0.2,
                                  max_seq_len=8, attention_backend=backend)
    x, y = tok([[1, 2, 3, 4]]), tok([[2, 3, 4, 5]])
    loss, grads = train_once(config, x, y, 7)
    loss_c, grads_c = train_once(replace(config, activation_checkpointing=True), x, y, 7)
    assert loss == pytest.approx(loss_c, abs=1e-5)
    for a, b in zip(grads, grads_c):
        np.testing.assert_allclose(a, b, rtol=2e-4, atol=2e-5)


def test_checkpoint_replays_mfma_dropout_masks_under_autocast():
    say("checkpointed LM, fp16 autocast, MFMA dropout")
    config = nn.TransformerConfig(64, dim=256, num_heads=4, num_layers=2, dropout=0.2,
                                  max_seq_len=128, attention_backend="hip")
    rng = np.random.default_rng(4)
    x, y = tok(rng.integers(0, 64, (2, 96))), tok(rng.integers(0, 64, (2, 96)))
    keys = []
    draw = attn_mod.attention_dropout_key

    def logged():
        keys.append(draw())
        return keys[-1]

    _lib.profile_enable(True)
    _lib.profile_reset()
    loss, grads = train_once(config, x, y, 9, amp=True)
    probes = _lib.profile_read()
    _lib.profile_enable(False)
    assert probes.get("fwd_mfma_dropout", (0, 0))[0] == 2  # one per layer, on the MFMA kernel
    with patch.object(attn_mod, "attention_dropout_key", logged):
        loss_c, grads_c = train_once(replace(config, activation_checkpointing=True), x, y, 9,
                                     amp=True)
    # forward (no grad), then the recomputations in backward order (layer 2
    # first): each block replays its own key
    assert len(keys) == 4 and keys[2:] == keys[1::-1] and keys[0] != keys[1]
    assert loss == pytest.approx(loss_c, abs=1e-5)
    for a, b in zip(grads, grads_c):
        np.testing.assert_allclose(a, b, rtol=2e-4, atol=2e-5)
    # without the replay the recomputation drops other elements: gradients move
    fresh = iter(range(1, 100))
    with patch.object(attn_mod, "attention_dropout_key", lambda: next(fresh) * 0x9E3779B97F4A7C15):
        _, grads_x = train_once(replace(config, activation_checkpointing=True), x, y, 9, amp=True)
    assert any(not np.allclose(a, b, rtol=2e-4, atol=2e-5) for a, b in zip(grads, grads_x))


def test_float64_rotary_attention_matches_oracle():
    """float64 MultiHeadAttention with rotary embeddings: the operands are
    rotated before the generic kernels (the kernels fold RoPE for f32 / f16 /
    bf16 only)."""
    say("float64 rotary MHA")
    ts.seed(3)
    mha = nn.MultiHeadAttention(32, 4, num_kv_heads=2, device=HIP)
    mha.to(dtype="float64")
    xh = np.random.default_rng(3).standard_normal((2, 9, 32))
    x = ts.tensor(xh, device=HIP, dtype="float64", requires_grad=True)
    y = mha(x, is_causal=True)
    y.sum().backward()
    w = {n: p.numpy().astype(np.float64) for n, p in mha.named_parameters()}

    def heads(t, n):
        return t.reshape(2, 9, n, 8).transpose(0, 2, 1, 3)

    def rope64(t):  # the reference's rotation in the operand dtype (attention.py:269-285)
        c, s_ = (np.repeat(a, 2, axis=-1).astype(np.float64) for a in R.tables(t.shape[-2], 8))
        turned = np.stack((-t[..., 1::2], t[..., 0::2]), axis=-1).reshape(t.shape)
        return t * c + turned * s_

    q = rope64(heads(xh @ w["q_proj.weight"].T, 4))
    k = rope64(heads(xh @ w["k_proj.weight"].T, 2))
    v = heads(xh @ w["v_proj.weight"].T, 2)
    ref = A.sdpa(q, k, v, None, True, dtype="float64", backend="dense", enable_gqa=True)
    want = ref.out.transpose(0, 2, 1, 3).reshape(2, 9, 32) @ w["out_proj.weight"].T
    np.testing.assert_allclose(y.numpy(), want, rtol=1e-10, atol=1e-12)
    assert np.isfinite(x.grad.numpy()).all() and np.abs(x.grad.numpy()).max() > 0


def test_folded_rope_backward_takes_an_expanded_gradient():
    """An upstream gradient with a zero sequence stride (an expand) reaches
    the folded-RoPE backward as a real tensor and gives the gradients of the
    same gradient materialised."""
    say("folded RoPE backward, expanded upstream gradient")
    gen = np.random.default_rng(8)
    shape = (1, 2, 64, 64)
    qh, kh, vh = (gen.standard_normal(shape).astype(np.float32) for _ in range(3))
    row = torch.from_numpy(gen.standard_normal((1, 2, 1, 64)).astype(np.float32)).cuda().half()

    def grads(expanded):
        q, k, v = (ts.tensor(a, device=HIP, dtype="float16", requires_grad=True)
                   for a in (qh, kh, vh))
        out = attn_mod.scaled_dot_product_attention(q, k, v, is_causal=True,
                                                    _rope=(0, 0, 10000.0))
        g = row.expand(shape) if expanded else row.expand(shape).contiguous()
        out.backward(ts.Tensor(g, device=HIP))
        return [t.grad.numpy() for t in (q, k, v)]

    for a, b in zip(grads(True), grads(False)):
        np.testing.assert_array_equal(a, b)
