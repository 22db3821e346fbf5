"""Differentiable prefill attention on the HIP kernels.

`attention_prefill(q, k, v, **options)` takes the options of
`ops.attention_prefill` and returns o; when grad mode is on and q, k, v or a
fused QK-RMSNorm weight requires grad it runs through `PrefillAttention`,
whose backward calls `goda_attn_prefill_bwd` with the forward's saved o and
lse (the structure of FlashAttentionGQAKernel.backward,
kernels_/flash_attn_gqa/cuda.py:577-658). The norm weights
(`q_norm_weight`, `k_norm_weight`) get their gradients from the same call;
the other tensors among the options (RoPE tables, ALiBi slopes, cu_seqlens,
the boolean mask) are treated as constants.
"""

from __future__ import annotations

import math

import torch

from . import headdim, ops


class PrefillAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, q_norm_weight, k_norm_weight, options: dict):
        opts = dict(options)
        if q_norm_weight is not None:
            opts["q_norm_weight"] = q_norm_weight
        if k_norm_weight is not None:
            opts["k_norm_weight"] = k_norm_weight
        o, lse = ops.attention_prefill(q, k, v, return_lse=True, **opts)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.options = opts
        ctx.norm_dtypes = (None if q_norm_weight is None else q_norm_weight.dtype,
                           None if k_norm_weight is None else k_norm_weight.dtype)
        return o

    @staticmethod
    def backward(ctx, d_o):
        q, k, v, o, lse = ctx.saved_tensors
        grads = ops.attention_prefill_bwd(q, k, v, o, lse, d_o, **ctx.options)
        if len(grads) == 3:
            return (*grads, None, None, None)
        dq, dk, dv, dqn, dkn = grads
        dqn = None if dqn is None else dqn.to(ctx.norm_dtypes[0])
        dkn = None if dkn is None else dkn.to(ctx.norm_dtypes[1])
        return dq, dk, dv, dqn, dkn, None


def attention_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, **options) -> torch.Tensor:
    if not headdim.is_native(q.shape[-1]):
        return _padded(q, k, v, options)
    m = options.get("attn_mask")
    if m is not None and not isinstance(m, ops.PackedMask) and q.dim() == 4:
        # Packed once, shared by the forward and the backward.
        options["attn_mask"] = ops.pack_mask(m, q.shape[0], q.shape[2], q.shape[1], k.shape[1], q.device)
    qn, kn = options.get("q_norm_weight"), options.get("k_norm_weight")
    wants = [t for t in (q, k, v, qn, kn) if t is not None]
    if torch.is_grad_enabled() and any(t.requires_grad for t in wants):
        options = dict(options)
        options.pop("return_lse", None)
        options.pop("q_norm_weight", None)
        options.pop("k_norm_weight", None)
        return PrefillAttention.apply(q, k, v, qn, kn, options)
    return ops.attention_prefill(q, k, v, **options)


def _row_positions(cu: torch.Tensor, total: int) -> torch.Tensor:
    """Position of each packed row inside its sequence (rows of sequence b
    are cu[b] .. cu[b+1]-1)."""
    rows = torch.arange(total, device=cu.device)
    seq = torch.searchsorted(cu[1:].to(torch.int64), rows, right=True)
    return rows - cu.to(torch.int64)[seq]


def _padded(q, k, v, options: dict) -> torch.Tensor:
    """A head dim the kernels do not instantiate (see goda_amd.headdim): the
    fused QK-RMSNorm and RoPE options run as torch ops at the positions the
    kernels would use, then q, k, v are zero-padded to the next instantiated
    head dim, attended with the 1/sqrt(D) scale of the real head dim, and the
    output sliced back; gradients flow through the pad and the slice."""
    opts = dict(options)
    d = q.shape[-1]
    dp = headdim.padded(d)
    qn, kn = opts.pop("q_norm_weight", None), opts.pop("k_norm_weight", None)
    eps = opts.pop("norm_eps", 1e-6)
    if qn is not None:
        q = headdim.rms_norm(q, qn, eps)
    if kn is not None:
        k = headdim.rms_norm(k, kn, eps)
    cos, sin = opts.pop("rope_cos", None), opts.pop("rope_sin", None)
    rq, rk = opts.pop("rope_q", False), opts.pop("rope_k", False)
    qo, ko = int(opts.pop("rope_q_offset", 0)), int(opts.pop("rope_k_offset", 0))
    pabs = bool(opts.pop("rope_pos_abs", False))
    if (rq or rk) and cos is None:
        raise ValueError("goda_amd: rope_q/rope_k need rope_cos and rope_sin")
    varlen = opts.get("cu_seqlens_q") is not None
    if rq or rk:
        cos = cos.reshape(-1, d // 2).float()
        sin = sin.reshape(-1, d // 2).float()
        if varlen:
            cu_q, cu_k = opts["cu_seqlens_q"], opts["cu_seqlens_k"]
            iq = _row_positions(cu_q, q.shape[0])
            jk = _row_positions(cu_k, k.shape[0])
            if rq:
                seq = torch.searchsorted(cu_q[1:].to(torch.int64), torch.arange(q.shape[0], device=q.device), right=True)
                lk = (cu_k[1:] - cu_k[:-1]).to(torch.int64)[seq]
                lq = (cu_q[1:] - cu_q[:-1]).to(torch.int64)[seq]
                pos = qo + iq if pabs else qo + (lk - lq) + iq
                q = headdim.rotate(q[None], cos, sin, pos[None])[0]
            if rk:
                k = headdim.rotate(k[None], cos, sin, (ko + jk)[None])[0]
        else:
            tq, tk = q.shape[1], k.shape[1]
            if rq:
                i = torch.arange(tq, device=q.device)
                used = opts.get("seqused_k")
                if pabs:
                    pos = qo + i
                elif used is not None:
                    pos = qo + (used.to(torch.int64)[:, None] - tq) + i[None]
                else:
                    pos = qo + (tk - tq) + i
                q = headdim.rotate(q, cos, sin, pos)
            if rk:
                k = headdim.rotate(k, cos, sin, ko + torch.arange(tk, device=k.device))
    if opts.get("softmax_scale") is None:
        opts["softmax_scale"] = 1.0 / math.sqrt(d)
    o = attention_prefill(headdim.pad(q, dp), headdim.pad(k, dp), headdim.pad(v, dp), **opts)
    return o[..., :d]
