"""Seeded synthetic inputs for the attention workloads (test infrastructure).

One recipe feeds the parity tests and the CPU baseline: a NumPy
``default_rng(seed)`` draws float32 N(0,1) arrays in the order Q, K, V, dO,
then per-sequence lengths; values are multiplied by ``value_scale`` *before*
rounding to the storage dtype.  Seed 42 matches ``ts.seed(42)`` in the
reference's ``benchmarks/bench_transformer.py:19``.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .halfprec import round_to


@dataclass
class AttentionInputs:
    q: np.ndarray
    k: np.ndarray
    v: np.ndarray
    do: np.ndarray | None
    lengths: np.ndarray | None
    dtype: str


def attention_inputs(
    batch: int,
    heads: int,
    seq_q: int,
    dim: int,
    dtype: str,
    *,
    seed: int = 42,
    heads_kv: int | None = None,
    seq_k: int | None = None,
    dim_v: int | None = None,
    value_scale: float = 1.0,
    with_grad: bool = True,
    length_range: tuple[int, int] | None = None,
) -> AttentionInputs:
    rng = np.random.default_rng(seed)
    hkv = heads if heads_kv is None else heads_kv
    sk = seq_q if seq_k is None else seq_k
    dv = dim if dim_v is None else dim_v

    def draw(shape, mult):
        x = rng.standard_normal(shape, dtype=np.float32)
        if mult != 1.0:
            x = x * np.float32(mult)
        return round_to(x, dtype)

    q = draw((batch, heads, seq_q, dim), value_scale)
    k = draw((batch, hkv, sk, dim), value_scale)
    v = draw((batch, hkv, sk, dv), value_scale)
    do = draw((batch, heads, seq_q, dv), 1.0) if with_grad else None
    lengths = None
    if length_range is not None:
        lo, hi = length_range
        lengths = rng.integers(lo, hi + 1, size=batch).astype(np.int32)
    return AttentionInputs(q, k, v, do, lengths, dtype)


# The five workloads, as (kwargs for attention_inputs, description).
WORKLOADS = {
    "causal_fwd_bwd_f32_b8h4s256d64": dict(
        batch=8, heads=4, seq_q=256, dim=64, dtype="float32"
    ),
    "causal_fwd_bwd_bf16_b16h16s2048d128": dict(
        batch=16, heads=16, seq_q=2048, dim=128, dtype="bfloat16", value_scale=0.5
    ),
    "decode_f16_b64h32d128_len512_8192": dict(
        batch=64, heads=32, seq_q=1, dim=128, dtype="float16", seq_k=8192,
        with_grad=False, length_range=(512, 8192),
    ),
    "padded_prefill_bf16_b2h32s32768d128": dict(
        batch=2, heads=32, seq_q=32768, dim=128, dtype="bfloat16", value_scale=0.5,
        with_grad=False, length_range=(16384, 32768),
    ),
}
