from .attn import GroupedQueryAttention, MultiHeadAttention, RMSNorm
from .flashattn import FlashAttention
from .pos import ALiBiPositionalBias, LinearScaledRoPE, RoPE, alibi_slopes

__all__ = [
    "FlashAttention",
    "GroupedQueryAttention",
    "MultiHeadAttention",
    "RMSNorm",
    "RoPE",
    "LinearScaledRoPE",
    "ALiBiPositionalBias",
    "alibi_slopes",
]
