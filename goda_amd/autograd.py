"""Differentiable prefill attention on the HIP kernels.

`attention_prefill(q, k, v, **options)` takes the options of
`ops.attention_prefill` and returns o; when grad mode is on and q, k or v
requires grad it runs through `PrefillAttention`, whose backward calls
`goda_attn_prefill_bwd` with the forward's saved o and lse (the structure of
FlashAttentionGQAKernel.backward, kernels_/flash_attn_gqa/cuda.py:577-658).
Tensors among the options (RoPE tables, ALiBi slopes, cu_seqlens, the
boolean mask) are treated as constants.
"""

from __future__ import annotations

import torch

from . import ops


class PrefillAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, options: dict):
        o, lse = ops.attention_prefill(q, k, v, return_lse=True, **options)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.options = options
        return o

    @staticmethod
    def backward(ctx, d_o):
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = ops.attention_prefill_bwd(q, k, v, o, lse, d_o, **ctx.options)
        return dq, dk, dv, None


def attention_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, **options) -> torch.Tensor:
    m = options.get("attn_mask")
    if m is not None and not isinstance(m, ops.PackedMask) and q.dim() == 4:
        # Packed once, shared by the forward and the backward.
        options["attn_mask"] = ops.pack_mask(m, q.shape[0], q.shape[2], q.shape[1], k.shape[1], q.device)
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        options.pop("return_lse", None)
        return PrefillAttention.apply(q, k, v, options)
    return ops.attention_prefill(q, k, v, **options)
