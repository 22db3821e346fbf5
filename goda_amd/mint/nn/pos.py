"""Positional encodings of goda's attention layer (mint/nn/pos.py), shaped for
the fused kernels: instead of rotating q/k in separate elementwise passes, the
modules hand the attention kernels fp32 cos/sin tables (RoPE) or per-head
slopes (ALiBi), and the rotation / bias happens inside the kernels.

`forward(q, k, start_pos)` is kept with the reference's signature and
semantics for callers that want the unfused result.
"""

from __future__ import annotations

import math

import torch
from torch import nn


def rope_tables(seq_len: int, head_dim: int, base: float, scale_factor: float = 1.0):
    """fp32 cos/sin [seq_len, head_dim/2] of goda's RoPE buffers
    (mint/nn/pos.py:71-88): inv_freq_i = base^(-2i/D), theta = t * inv_freq,
    with t = position / scale_factor for LinearScaledRoPE (:127-148)."""
    channel_range = torch.arange(0, head_dim, 2, dtype=torch.float32)
    inv_freq = 1.0 / (base ** (channel_range / head_dim))
    t = torch.arange(seq_len, dtype=torch.float32)
    if scale_factor != 1.0:
        t = t / scale_factor
    freqs = torch.outer(t, inv_freq)
    return freqs.cos(), freqs.sin()


class PosEmbeddings(nn.Module):
    """Base of the fusable encodings (mint/nn/pos.py:8-15)."""


class RoPE(PosEmbeddings):
    """mint/nn/pos.py:51-112: inv_freq_i = base^(-2i/D), theta = p * inv_freq,
    half-split rotation y = [x1 cos - x2 sin, x1 sin + x2 cos].

    The tables stay fp32 (the reference rounds them to the model dtype first,
    mint/nn/pos.py:86); the kernels rotate in fp32 and round once."""

    def __init__(self, seq_len: int, head_dim: int, rope_base_theta: int = 100000, dtype: torch.dtype = torch.float32) -> None:
        super().__init__()
        self.head_dim = head_dim
        cos, sin = rope_tables(seq_len, head_dim, float(rope_base_theta), self._scale_factor())
        self.register_buffer("cos", cos, persistent=False)
        self.register_buffer("sin", sin, persistent=False)
        self.cos: torch.Tensor
        self.sin: torch.Tensor

    def _scale_factor(self) -> float:
        return 1.0

    def forward(self, q: torch.Tensor, k: torch.Tensor, start_pos: int = 0):
        t = q.shape[1]
        cos = self.cos[start_pos : start_pos + t][None, :, None, :].to(q.dtype)
        sin = self.sin[start_pos : start_pos + t][None, :, None, :].to(q.dtype)

        def rot(x):
            d = x.shape[-1] // 2
            x1, x2 = x[..., :d], x[..., d:]
            return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1)

        return rot(q), rot(k), None


class LinearScaledRoPE(RoPE):
    """mint/nn/pos.py:115-148: positions divided by scale_factor."""

    def __init__(
        self,
        seq_len: int,
        head_dim: int,
        scale_factor: float = 4.0,
        rope_base_theta: int = 100000,
        dtype: torch.dtype = torch.float32,
    ) -> None:
        self.scale_factor = scale_factor
        super().__init__(seq_len, head_dim, rope_base_theta, dtype)

    def _scale_factor(self) -> float:
        return float(self.scale_factor)


def alibi_slopes(n_heads: int) -> list[float]:
    """mint/nn/pos.py:171-184: start = 2^(-8/n) for a power of two n, slope_h
    = start^(h+1); otherwise the slopes of the nearest lower power of two,
    then every other slope of twice that."""

    def pow2(n: int) -> list[float]:
        start = 2 ** (-(2 ** -(math.log2(n) - 3)))
        return [start * (start**i) for i in range(n)]

    if math.log2(n_heads).is_integer():
        return pow2(n_heads)
    closest = 2 ** math.floor(math.log2(n_heads))
    return pow2(closest) + alibi_slopes(2 * closest)[0::2][: n_heads - closest]


class ALiBiPositionalBias(PosEmbeddings):
    """mint/nn/pos.py:162-207. The bias slope_h * (j - i_abs) is added to the
    scaled scores inside the kernel (the reference computes it but never
    feeds it to attention, mint/nn/attn.py:62)."""

    def __init__(self, n_heads: int) -> None:
        super().__init__()
        self.n_heads = n_heads
        self.register_buffer("slopes", torch.tensor(alibi_slopes(n_heads), dtype=torch.float32), persistent=False)
        self.slopes: torch.Tensor

    def forward(self, q: torch.Tensor, k: torch.Tensor, start_pos: int = 0):
        seq_len_q = q.shape[1]
        total = start_pos + seq_len_q
        q_idx = torch.arange(start_pos, total, device=q.device)[:, None]
        k_idx = torch.arange(0, total, device=k.device)[None, :]
        bias = self.slopes.to(q.device)[None, :, None, None] * (k_idx - q_idx)[None, None]
        return q, k, bias.to(q.dtype)
