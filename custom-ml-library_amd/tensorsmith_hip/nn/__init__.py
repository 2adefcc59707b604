"""Neural-network pieces on the attention path (reference ``tensorsmith.nn``)."""

from .attention import rotary_embedding, scaled_dot_product_attention

__all__ = ["rotary_embedding", "scaled_dot_product_attention"]
