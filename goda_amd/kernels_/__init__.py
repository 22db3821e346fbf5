"""Drop-in for goda's `kernels_` package (kernels_/__init__.py:15).

`FlashAttentionGQAKernel` and `FlashAttentionMQAKernel` keep the reference's
autograd signature `apply(Q, K, V, causal, tau) -> O` on [B, H, T, D] tensors
(kernels_/flash_attn_gqa/cuda.py:515-575, kernels_/flash_attn_mqa/cuda.py:470-527),
and extend it compatibly:
  - K and V may carry Hkv heads with Hkv | Hq (query head h reads KV head
    h // (Hq/Hkv)); the reference indexes K/V with Q's head and so only
    handles Hq == Hkv (kernels_/flash_attn_gqa/cuda.py:394);
  - optional trailing positional arguments fuse RoPE and ALiBi:
    apply(Q, K, V, causal, tau, rope_cos, rope_sin, alibi_slopes, window_left)
    with fp32 tables [positions, D/2] (rotation at positions 0..T-1 for Q and
    K) and fp32 slopes [Hq];
  - any T (the reference requires T to be a multiple of its block size);
  - any head dim D <= 256: D outside {64, 128, 256} runs zero-padded to the
    next one (goda_amd.headdim), RoPE then applied by torch ops.
The forward saves O and the log-sum-exp M (natural log, fp32 [B, H, T]) like
the reference (:571-575); the backward returns (dQ, dK, dV, None, ...) from
them through `goda_attn_prefill_bwd` (:577-658), with dK/dV in K's and V's
head count (summed over each KV head's query group).
"""

from __future__ import annotations

import torch

from .. import headdim, ops


class _FlashAttentionBase(torch.autograd.Function):
    @classmethod
    def apply(cls, Q, K, V, causal, tau, rope_cos=None, rope_sin=None, alibi_slopes=None, window_left=-1):  # noqa: N803
        d = Q.shape[-1]
        if headdim.is_native(d):
            return super().apply(Q, K, V, causal, tau, rope_cos, rope_sin, alibi_slopes, window_left)
        # zero-padded head dim (differentiable pad / slice around the kernel)
        if rope_cos is not None:
            t_q, t_k = Q.shape[2], K.shape[2]
            cos, sin = rope_cos.float(), rope_sin.float()
            Q = headdim.rotate(Q.transpose(1, 2), cos, sin, torch.arange(t_k - t_q, t_k)).transpose(1, 2)  # noqa: N806
            K = headdim.rotate(K.transpose(1, 2), cos, sin, torch.arange(t_k)).transpose(1, 2)  # noqa: N806
        dp = headdim.padded(d)
        O = super().apply(headdim.pad(Q, dp), headdim.pad(K, dp), headdim.pad(V, dp), causal, tau,  # noqa: N806
                          None, None, alibi_slopes, window_left)
        return O[..., :d]

    @staticmethod
    def forward(ctx, Q, K, V, causal, tau, rope_cos=None, rope_sin=None, alibi_slopes=None, window_left=-1):  # noqa: N803
        if Q.dim() != 4 or K.dim() != 4 or V.dim() != 4:
            raise ValueError("Q, K, V must be [B, H, T, D]")
        rope = rope_cos is not None
        o, lse = ops.attention_prefill(
            Q.transpose(1, 2),
            K.transpose(1, 2),
            V.transpose(1, 2),
            causal=bool(causal),
            softmax_scale=float(tau),
            window_left=int(window_left),
            alibi_slopes=alibi_slopes,
            rope_cos=rope_cos,
            rope_sin=rope_sin,
            rope_q=rope,
            rope_k=rope,
            return_lse=True,
        )
        O = o.transpose(1, 2)  # noqa: N806  [B, H, T, D] view of a [B, T, H, D] buffer
        ctx.save_for_backward(Q, K, V, O, lse)
        ctx.options = dict(
            causal=bool(causal),
            softmax_scale=float(tau),
            window_left=int(window_left),
            alibi_slopes=alibi_slopes,
            rope_cos=rope_cos,
            rope_sin=rope_sin,
            rope_q=rope,
            rope_k=rope,
        )
        return O

    @staticmethod
    def backward(ctx, dO):  # noqa: N803
        Q, K, V, O, lse = ctx.saved_tensors  # noqa: N806
        dq, dk, dv = ops.attention_prefill_bwd(
            Q.transpose(1, 2), K.transpose(1, 2), V.transpose(1, 2), O.transpose(1, 2), lse, dO.transpose(1, 2),
            **ctx.options,
        )
        return dq.transpose(1, 2), dk.transpose(1, 2), dv.transpose(1, 2), None, None, None, None, None, None


class FlashAttentionGQAKernel(_FlashAttentionBase):
    """kernels_/flash_attn_gqa/cuda.py:510-658 — same call, real GQA."""


class FlashAttentionMQAKernel(_FlashAttentionBase):
    """kernels_/flash_attn_mqa/cuda.py:468-610 — same call, real MQA (Hkv = 1)."""


__all__ = ["FlashAttentionGQAKernel", "FlashAttentionMQAKernel"]
