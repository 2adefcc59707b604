"""Neural-network pieces on the attention path (reference ``tensorsmith.nn``)."""

from . import functional
from .attention import rotary_embedding, scaled_dot_product_attention
from .cache import KVCache
from .checkpoint import checkpoint
from .layers import GELU, Dropout, Embedding, LayerNorm, Linear
from .module import Module, Parameter
from .transformer import (
    MultiHeadAttention, RMSNorm, SiLU, SwiGLU, TransformerConfig, TransformerDecoderBlock,
    TransformerLM, sample_logits,
)

__all__ = [
    "Dropout", "Embedding", "GELU", "KVCache", "LayerNorm", "Linear", "Module",
    "MultiHeadAttention", "Parameter", "RMSNorm", "SiLU", "SwiGLU", "TransformerConfig",
    "TransformerDecoderBlock", "TransformerLM", "checkpoint", "functional", "rotary_embedding",
    "sample_logits", "scaled_dot_product_attention",
]
