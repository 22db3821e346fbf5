"""Shared helpers for the parity tests: run the HIP path and the CPU oracle on
the same inputs and compare within the north-star tolerances
(max abs error <= 1e-4 for fp32, <= 2e-2 for bf16/fp16, against fp32)."""

from __future__ import annotations

import torch

from oracle import attention as ref

TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def rope_oracle(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
    """Rotate x [B, T, H, D] (fp32 copy on the CPU) at the given positions."""
    return ref.apply_rope(x.to("cpu", torch.float32), cos.cpu(), sin.cpu(), positions.cpu())


def max_err(a: torch.Tensor, b: torch.Tensor) -> float:
    return (a.to("cpu", torch.float32) - b.to("cpu", torch.float32)).abs().max().item()


def lse_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """Max abs difference of two lse tensors, treating matching -inf as equal."""
    a = a.to("cpu", torch.float32)
    b = b.to("cpu", torch.float32)
    both_inf = torch.isinf(a) & torch.isinf(b) & (torch.sign(a) == torch.sign(b))
    d = (a - b).abs()
    d[both_inf] = 0.0
    return d.max().item() if d.numel() else 0.0
