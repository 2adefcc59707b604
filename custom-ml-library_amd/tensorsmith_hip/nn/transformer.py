"""``MultiHeadAttention`` -- the reference's caller of the attention op.

Same constructor, forward signature, validation and data flow as
``src/tensorsmith/nn/transformer.py:48-155``: projections reshaped to
``[B,S,H,D]`` and permuted to ``[B,H,S,D]`` *views* (the HIP kernels take the
strides, so no copy is made), optional interleaved RoPE, KV-cache append with
``causal_offset = cache.length``, then ``scaled_dot_product_attention`` with
``backend`` (``"hip"`` added to the allowlist; ``"auto"`` picks it).
"""

from __future__ import annotations

import numpy as np

from ..tensor import Tensor, is_grad_enabled
from .attention import BACKENDS, rotary_embedding, scaled_dot_product_attention
from .cache import KVCache
from .layers import Linear
from .module import Module


class MultiHeadAttention(Module):
    """Self/cross attention with optional grouped-query heads and rotary positions."""

    def __init__(self, embed_dim: int, num_heads: int, *, num_kv_heads: int | None = None,
                 dropout: float = 0.0, bias: bool = False, rotary: bool = True,
                 backend: str = "auto", device=None):
        super().__init__()
        kv_heads = num_heads if num_kv_heads is None else num_kv_heads
        if min(embed_dim, num_heads, kv_heads) <= 0 or embed_dim % num_heads or num_heads % kv_heads:
            raise ValueError(
                "embed_dim must divide into heads and query heads must divide into KV groups")
        self.embed_dim, self.num_heads, self.num_kv_heads = embed_dim, num_heads, kv_heads
        self.head_dim = embed_dim // num_heads
        if rotary and self.head_dim % 2:
            raise ValueError("rotary attention requires an even head dimension")
        if not 0 <= dropout < 1 or backend not in BACKENDS:
            raise ValueError("invalid attention dropout/backend")
        self.rotary, self.backend, self.dropout_p = rotary, backend, dropout
        self.q_proj = Linear(embed_dim, embed_dim, bias=bias, device=device)
        self.k_proj = Linear(embed_dim, kv_heads * self.head_dim, bias=bias, device=device)
        self.v_proj = Linear(embed_dim, kv_heads * self.head_dim, bias=bias, device=device)
        self.out_proj = Linear(embed_dim, embed_dim, bias=bias, device=device)

    def new_cache(self, batch_size: int, max_seq_len: int, *, dtype="float32",
                  quantized: bool = False) -> KVCache:
        return KVCache(batch_size, self.num_kv_heads, self.head_dim, max_seq_len,
                       device=self.q_proj.weight.device, dtype=dtype, quantized=quantized)

    def forward(self, input: Tensor, context: Tensor | None = None, *, attn_mask=None,
                is_causal: bool = True, cache: KVCache | None = None) -> Tensor:
        if input.ndim != 3 or input.shape[-1] != self.embed_dim:
            raise ValueError("attention input must be [batch, sequence, embed_dim]")
        source = input if context is None else context
        if source.ndim != 3 or source.shape[0] != input.shape[0] or source.shape[-1] != self.embed_dim:
            raise ValueError("attention context must be [batch, sequence, embed_dim]")
        if cache is not None and (self.training or is_grad_enabled() or context is not None):
            raise RuntimeError(
                "cached self-attention requires eval() and no_grad(); "
                "cross-attention caching is not supported")
        batch, steps, _ = input.shape
        offset = 0 if cache is None else cache.length
        if self.backend == "native":
            raise ValueError("native attention requires Metal")
        if attn_mask is not None:
            if attn_mask.requires_grad or attn_mask.device != input.device:
                raise ValueError("attention mask must be non-differentiable and on the input device")
            try:
                expected = (batch, self.num_heads, steps, offset + source.shape[1])
                if np.broadcast_shapes(attn_mask.shape, expected) != expected:
                    raise ValueError("mask expands attention dimensions")
                if not any(name in str(attn_mask.dtype) for name in ("bool", "float")):
                    raise TypeError("attention masks must be boolean or floating point")
            except ValueError as error:
                raise ValueError("attention mask is not broadcastable to [B,H,Q,K]") from error
        q = self.q_proj(input).reshape(batch, steps, self.num_heads, self.head_dim).permute(0, 2, 1, 3)
        k = (self.k_proj(source).reshape(batch, source.shape[1], self.num_kv_heads, self.head_dim)
             .permute(0, 2, 1, 3))
        v = (self.v_proj(source).reshape(batch, source.shape[1], self.num_kv_heads, self.head_dim)
             .permute(0, 2, 1, 3))
        if self.rotary:
            q = rotary_embedding(q, offset)
            k = rotary_embedding(k, offset if context is None else 0)
        if cache is not None:
            k, v = cache.append(k, v)
        attended = scaled_dot_product_attention(
            q, k, v, attn_mask, self.dropout_p if self.training else 0.0, is_causal,
            causal_offset=offset, backend=self.backend,
            enable_gqa=self.num_kv_heads != self.num_heads)
        return self.out_proj(attended.permute(0, 2, 1, 3).reshape(batch, steps, self.embed_dim))
