"""Float64 brute-force attention with explicit loops (numpy) — TEST
INFRASTRUCTURE ONLY (see oracle/__init__.py).

Independent of torch's SDPA: scores, masks, biases and the softmax are written
out per query row, so a mistake in oracle/attention.py's use of SDPA (mask
polarity, GQA head mapping, bias sign, window edge) shows up as a mismatch.
Small shapes only.
"""

from __future__ import annotations

import math

import numpy as np


def attention(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    *,
    causal: bool,
    window_left: int = -1,
    slopes: np.ndarray | None = None,
    doc_ids: np.ndarray | None = None,
    mask: np.ndarray | None = None,
    scale: float | None = None,
):
    """q [B, Tq, Hq, D], k/v [B, Tk, Hkv, D] -> (o [B, Tq, Hq, D], lse [B, Hq, Tq]).

    Query row i of Tq sits at absolute position i_abs = Tk - Tq + i; key j is
    visible iff (not causal or j <= i_abs) and (window: i_abs - j <= W, with
    causal or Tq == 1) and (doc ids equal) and (mask[b, h, i, j], a boolean
    array broadcastable to [B, Hq, Tq, Tk]). Bias slope_h * (j - i_abs).
    A row with no visible key gives o = 0, lse = -inf.
    """
    q = q.astype(np.float64)
    k = k.astype(np.float64)
    v = v.astype(np.float64)
    b_, tq, hq, d = q.shape
    tk, hkv = k.shape[1], k.shape[2]
    group = hq // hkv
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    if mask is not None:
        mask = np.broadcast_to(mask, (b_, hq, tq, tk))
    o = np.zeros((b_, tq, hq, d))
    lse = np.full((b_, hq, tq), -np.inf)
    for b in range(b_):
        for h in range(hq):
            hk = h // group
            for i in range(tq):
                iabs = tk - tq + i
                logits = []
                idx = []
                for j in range(tk):
                    if causal and j > iabs:
                        continue
                    if window_left >= 0 and (causal or tq == 1) and iabs - j > window_left:
                        continue
                    if doc_ids is not None and doc_ids[b, i] != doc_ids[b, j]:
                        continue
                    if mask is not None and not mask[b, h, i, j]:
                        continue
                    s = float(np.dot(q[b, i, h], k[b, j, hk])) * scale
                    if slopes is not None:
                        s += float(slopes[h]) * (j - iabs)
                    logits.append(s)
                    idx.append(j)
                if not idx:
                    continue
                m = max(logits)
                w = [math.exp(x - m) for x in logits]
                z = sum(w)
                acc = np.zeros(d)
                for wj, j in zip(w, idx):
                    acc += wj * v[b, j, hk]
                o[b, i, h] = acc / z
                lse[b, h, i] = m + math.log(z)
    return o, lse


def rope(x: np.ndarray, positions: np.ndarray, base: float, scale_factor: float = 1.0) -> np.ndarray:
    """Half-split RoPE computed per element in float64 from the angle
    definition theta_{p,i} = (p / scale_factor) * base^(-2i/D)."""
    x = x.astype(np.float64)
    d = x.shape[-1]
    half = d // 2
    out = np.empty_like(x)
    for t, p in enumerate(positions):
        for i in range(half):
            theta = (p / scale_factor) * base ** (-(2.0 * i) / d)
            c, s = math.cos(theta), math.sin(theta)
            x1 = x[..., t, :, i]
            x2 = x[..., t, :, i + half]
            out[..., t, :, i] = x1 * c - x2 * s
            out[..., t, :, i + half] = x1 * s + x2 * c
    return out


def attention_backward(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    d_o: np.ndarray,
    *,
    causal: bool,
    window_left: int = -1,
    slopes: np.ndarray | None = None,
    doc_ids: np.ndarray | None = None,
    mask: np.ndarray | None = None,
    scale: float | None = None,
    plant: str | None = None,
):
    """Gradients (dq, dk, dv) of `attention` for upstream d_o, written out per
    (row, key) pair in float64 — the FlashAttention-2 backward formulas that
    kernels_/flash_attn_gqa/cuda.py:6-246 implements:
        p_ij = exp(s_ij - lse_i),  delta_i = sum_d dO_i * o_i,
        dv_j += p_ij dO_i,  ds_ij = p_ij (dO_i . v_j - delta_i),
        dq_i += scale ds_ij k_j,  dk_j += scale ds_ij q_i,
    with dk/dv of KV head h // group summed over the group's query heads.
    Rows with no visible key contribute nothing.

    `plant` is for the oracle's own tests only: "no_delta" drops delta_i,
    "first_head_only" keeps only the first query head of each group in dk/dv.
    """
    q = q.astype(np.float64)
    k = k.astype(np.float64)
    v = v.astype(np.float64)
    d_o = d_o.astype(np.float64)
    b_, tq, hq, d = q.shape
    tk, hkv = k.shape[1], k.shape[2]
    group = hq // hkv
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    o, lse = attention(q, k, v, causal=causal, window_left=window_left, slopes=slopes, doc_ids=doc_ids, mask=mask,
                       scale=scale)
    if mask is not None:
        mask = np.broadcast_to(mask, (b_, hq, tq, tk))
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    for b in range(b_):
        for h in range(hq):
            hk = h // group
            keep_kv = plant != "first_head_only" or h % group == 0
            for i in range(tq):
                if not np.isfinite(lse[b, h, i]):
                    continue
                iabs = tk - tq + i
                delta = 0.0 if plant == "no_delta" else float(np.dot(d_o[b, i, h], o[b, i, h]))
                for j in range(tk):
                    if causal and j > iabs:
                        continue
                    if window_left >= 0 and (causal or tq == 1) and iabs - j > window_left:
                        continue
                    if doc_ids is not None and doc_ids[b, i] != doc_ids[b, j]:
                        continue
                    if mask is not None and not mask[b, h, i, j]:
                        continue
                    s = float(np.dot(q[b, i, h], k[b, j, hk])) * scale
                    if slopes is not None:
                        s += float(slopes[h]) * (j - iabs)
                    p = math.exp(s - lse[b, h, i])
                    ds = p * (float(np.dot(d_o[b, i, h], v[b, j, hk])) - delta)
                    dq[b, i, h] += scale * ds * k[b, j, hk]
                    if keep_kv:
                        dv[b, j, hk] += p * d_o[b, i, h]
                        dk[b, j, hk] += scale * ds * q[b, i, h]
    return dq, dk, dv
