"""Restatement of goda's eager attention path on the CPU (torch, fp32/fp64).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Layouts follow the reference: module tensors are [B, T, H, D]
(mint/nn/attn.py:53-55); SDPA operands are [B, H, T, D]
(mint/nn/flashattn.py:157-159).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F  # noqa: N812


# ---------------------------------------------------------------------------
# positional encodings
# ---------------------------------------------------------------------------
def rope_tables(seq_len: int, head_dim: int, base: float, scale_factor: float = 1.0):
    """cos/sin tables [seq_len, head_dim/2] in fp32.

    mint/nn/pos.py:71-88 (RoPE._precompute_rotary_embeddings): inv_freq =
    1 / base^(arange(0, D, 2)/D), freqs = outer(t, inv_freq). With
    scale_factor != 1 it is LinearScaledRoPE (mint/nn/pos.py:127-148):
    t = arange(seq_len) / scale_factor.
    """
    channel_range = torch.arange(0, head_dim, 2, dtype=torch.float32)
    inv_freq = 1.0 / (base ** (channel_range / head_dim))
    t = torch.arange(seq_len, dtype=torch.float32)
    if scale_factor != 1.0:
        t = t / scale_factor
    freqs = torch.outer(t, inv_freq)
    return freqs.cos(), freqs.sin()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor):
    """Half-split rotation of x [..., T, H, D] at integer positions [T].

    mint/nn/pos.py:90-98 (_apply_rotary_embs): x1 = x[..., :D/2],
    x2 = x[..., D/2:], y = cat(x1 cos - x2 sin, x1 sin + x2 cos), with the
    tables sliced at start_pos .. start_pos+T-1 (mint/nn/pos.py:100-112).
    Computed in the dtype of x (use fp32/fp64 inputs for the oracle).
    """
    c = cos[positions].to(x.dtype)[:, None, :]  # [T, 1, D/2]
    s = sin[positions].to(x.dtype)[:, None, :]
    d = x.shape[-1] // 2
    x1, x2 = x[..., :d], x[..., d:]
    return torch.cat([x1 * c - x2 * s, x1 * s + x2 * c], dim=-1)


def alibi_slopes(n_heads: int) -> list[float]:
    """ALiBi slopes per head (mint/nn/pos.py:171-184).

    Power of two n: start = 2^(-2^-(log2 n - 3)) = 2^(-8/n), slope_h =
    start^(h+1). Otherwise the first 2^floor(log2 n) slopes, then every other
    slope of the 2*2^floor(log2 n) set.
    """

    def pow2(n: int) -> list[float]:
        start = 2 ** (-(2 ** -(math.log2(n) - 3)))
        return [start * (start**i) for i in range(n)]

    if math.log2(n_heads).is_integer():
        return pow2(n_heads)
    closest = 2 ** math.floor(math.log2(n_heads))
    return pow2(closest) + alibi_slopes(2 * closest)[0::2][: n_heads - closest]


def alibi_bias(slopes: torch.Tensor, q_len: int, k_len: int, dtype=torch.float32) -> torch.Tensor:
    """Additive bias [1, H, q_len, k_len]: slope_h * (j - i_abs).

    mint/nn/pos.py:186-207 builds it for k_len = start_pos + q_len with query
    positions start_pos .. start_pos+q_len-1; here the query positions are
    bottom-right aligned, i_abs = (k_len - q_len) + i, which is the same thing.
    """
    q_idx = torch.arange(k_len - q_len, k_len)[:, None]
    k_idx = torch.arange(k_len)[None, :]
    rel = (k_idx - q_idx).to(dtype)
    return slopes.to(dtype)[None, :, None, None] * rel[None, None]


# ---------------------------------------------------------------------------
# SDPA with goda's masks
# ---------------------------------------------------------------------------
def build_mask(
    q_len: int,
    k_len: int,
    *,
    causal: bool,
    window_size: tuple[int, int] = (-1, -1),
    doc_ids: torch.Tensor | None = None,
    base_attn_mask: torch.Tensor | None = None,
):
    """Boolean mask of mint/nn/flashattn.py:236-255 (None when unmasked)."""
    mask = None
    if doc_ids is not None:
        mask = doc_ids.unsqueeze(1).unsqueeze(-1) == doc_ids.unsqueeze(1).unsqueeze(-2)
    if base_attn_mask is not None:
        mask = base_attn_mask if mask is None else (mask & base_attn_mask)
    if causal:
        row_idx = (k_len - q_len) + torch.arange(q_len).unsqueeze(1)
        col_idx = torch.arange(k_len).unsqueeze(0)
        causal_mask = col_idx <= row_idx
        left = window_size[0]
        if 0 <= left < k_len:
            causal_mask = causal_mask & ((row_idx - col_idx) <= left)
        mask = causal_mask if mask is None else (mask & causal_mask)
    return mask


def sdpa_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    causal: bool,
    window_size: tuple[int, int] = (-1, -1),
    base_attn_mask: torch.Tensor | None = None,
    doc_ids: torch.Tensor | None = None,
    alibi: torch.Tensor | None = None,
    scale: float | None = None,
) -> torch.Tensor:
    """FlashAttention._sdpa_attention (mint/nn/flashattn.py:221-273).

    q [B, Hq, Lq, D], k/v [B, Hkv, Lk, D]; enable_gqa when Hq != Hkv
    (mint/nn/flashattn.py:160). `alibi` [1|B, Hq, Lq, Lk] is the additive
    bias the reference computes (mint/nn/pos.py:186-207) but never feeds to
    attention (mint/nn/attn.py:62); it is composed as SDPA's float mask with
    -inf where the boolean mask is False.
    """
    q_len, k_len = q.size(2), k.size(2)
    enable_gqa = q.size(1) != k.size(1)
    mask = build_mask(
        q_len, k_len, causal=causal, window_size=window_size, doc_ids=doc_ids, base_attn_mask=base_attn_mask
    )
    if q_len == 1 and not causal:
        left = window_size[0]
        if 0 <= left < k_len:
            start = max(0, k_len - (left + 1))
            k = k[:, :, start:, :]
            v = v[:, :, start:, :]
            if alibi is not None:
                alibi = alibi[..., start:]
        if alibi is not None:
            return F.scaled_dot_product_attention(q, k, v, attn_mask=alibi.to(q.dtype), enable_gqa=enable_gqa, scale=scale)
        return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=enable_gqa, scale=scale)
    if alibi is not None:
        fmask = alibi.to(q.dtype)
        if mask is not None:
            fmask = fmask.masked_fill(~mask, float("-inf"))
        return F.scaled_dot_product_attention(q, k, v, attn_mask=fmask, enable_gqa=enable_gqa, scale=scale)
    return F.scaled_dot_product_attention(
        q, k, v, attn_mask=mask, is_causal=(causal and mask is None), enable_gqa=enable_gqa, scale=scale
    )


def attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    causal: bool,
    window_size: tuple[int, int] = (-1, -1),
    doc_ids: torch.Tensor | None = None,
    alibi_slopes: torch.Tensor | None = None,
    base_attn_mask: torch.Tensor | None = None,
    scale: float | None = None,
    dtype=torch.float32,
) -> torch.Tensor:
    """FlashAttention._attention's SDPA branch (mint/nn/flashattn.py:156-172).

    q [B, Tq, Hq, D], k/v [B, Tk, Hkv, D] -> [B, Tq, Hq, D], computed in
    `dtype` on the CPU. `base_attn_mask` is goda's boolean mask, broadcastable
    to [B, Hq, Tq, Tk] (mint/nn/flashattn.py:242-243). A row that sees no key
    comes out as 0 (this torch's SDPA zeroes fully masked rows).
    """
    qs = q.to("cpu", dtype).transpose(1, 2)
    ks = k.to("cpu", dtype).transpose(1, 2)
    vs = v.to("cpu", dtype).transpose(1, 2)
    alibi = None
    if alibi_slopes is not None:
        alibi = alibi_bias(alibi_slopes.to("cpu", dtype), qs.size(2), ks.size(2), dtype)
    if base_attn_mask is not None:
        base_attn_mask = base_attn_mask.to("cpu")
    out = sdpa_attention(qs, ks, vs, causal=causal, window_size=window_size, doc_ids=doc_ids, alibi=alibi,
                         base_attn_mask=base_attn_mask, scale=scale)
    return out.transpose(1, 2)


def attention_rows(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    rows: torch.Tensor,
    *,
    causal: bool,
    window_left: int = -1,
    alibi_slopes: torch.Tensor | None = None,
    scale: float | None = None,
    dtype=torch.float32,
    lk: torch.Tensor | None = None,
    base_attn_mask: torch.Tensor | None = None,
):
    """Same semantics as `attention` for a subset of query rows, one batch
    entry at a time, without materialising [Tq, Tk] for all rows: returns
    (o [B, len(rows), Hq, D], lse [B, Hq, len(rows)]). Used to check full-size
    configurations on sampled rows. `lk` optionally gives per-sequence key
    counts (keys >= lk[b] are absent); `base_attn_mask` is goda's boolean
    mask broadcastable to [B, Hq, Tq, Tk].
    """
    b_, tq, hq, d = q.shape
    tk, hkv = k.shape[1], k.shape[2]
    g = hq // hkv
    scale = scale if scale is not None else 1.0 / math.sqrt(d)
    rows = rows.to(torch.long)
    outs, lses = [], []
    for b in range(b_):
        L = int(lk[b]) if lk is not None else tk
        qb = q[b, rows].to("cpu", dtype)  # [R, Hq, D]
        kb = k[b, :L].to("cpu", dtype).repeat_interleave(g, dim=1)  # [L, Hq, D]
        vb = v[b, :L].to("cpu", dtype).repeat_interleave(g, dim=1)
        s = torch.einsum("rhd,jhd->hrj", qb, kb) * scale  # [Hq, R, L]
        iabs = (L - tq) + rows  # bottom-right aligned query positions
        j = torch.arange(L)
        vis = torch.ones(len(rows), L, dtype=torch.bool)
        if causal:
            vis &= j[None, :] <= iabs[:, None]
            if 0 <= window_left < L:
                vis &= (iabs[:, None] - j[None, :]) <= window_left
        elif tq == 1 and 0 <= window_left < L:
            vis &= j[None, :] >= L - (window_left + 1)
        if alibi_slopes is not None:
            rel = (j[None, :] - iabs[:, None]).to(dtype)
            s = s + alibi_slopes.to("cpu", dtype)[:, None, None] * rel[None]
        visb = vis[None]
        if base_attn_mask is not None:
            m = base_attn_mask.to("cpu")
            while m.dim() < 4:
                m = m.unsqueeze(0)
            m = m.expand(b_, hq, tq, m.shape[-1] if m.shape[-1] != 1 else tk)
            visb = visb & m[b][:, rows, :L]
        s = s.masked_fill(~visb, float("-inf"))
        lse = torch.logsumexp(s, dim=-1)  # [Hq, R]
        p = torch.exp(s - lse[..., None])
        p = torch.nan_to_num(p, nan=0.0)
        o = torch.einsum("hrj,jhd->rhd", p, vb)
        outs.append(o)
        lses.append(lse)
    return torch.stack(outs), torch.stack(lses)


def lse_reference(q, k, v, *, causal, window_left=-1, alibi_slopes=None, scale=None, dtype=torch.float32):
    """Natural-log log-sum-exp of the scaled, biased, masked scores
    [B, Hq, Tq] — the `M` output of kernels_/flash_attn_gqa/cuda.py:496-499
    (m + ln l over tau-scaled scores)."""
    rows = torch.arange(q.shape[1])
    return attention_rows(
        q, k, v, rows, causal=causal, window_left=window_left, alibi_slopes=alibi_slopes, scale=scale, dtype=dtype
    )[1]


def varlen_attention(q, k, v, cu_q, cu_k, *, causal, window_left=-1, alibi_slopes=None, scale=None, dtype=torch.float32):
    """Packed sequences (mint/nn/flashattn.py:98-134): each sequence b of rows
    cu[b]..cu[b+1]-1 attends only to itself. q [Σ, Hq, D] -> [Σ, Hq, D]."""
    out = torch.empty(q.shape, dtype=dtype)
    for b in range(len(cu_q) - 1):
        qs, qe = int(cu_q[b]), int(cu_q[b + 1])
        ks_, ke = int(cu_k[b]), int(cu_k[b + 1])
        if qe == qs:
            continue
        o = attention(
            q[qs:qe][None],
            k[ks_:ke][None],
            v[ks_:ke][None],
            causal=causal,
            window_size=(window_left, -1),
            alibi_slopes=alibi_slopes,
            scale=scale,
            dtype=dtype,
        )
        out[qs:qe] = o[0]
    return out


def doc_ids_to_cu_seqlens(doc_ids: torch.Tensor) -> torch.Tensor:
    """Segment boundaries of packed documents, per row of doc_ids [B, T]: a new
    segment starts at every row start and wherever the id changes. Within a
    row this is the mask doc_ids[i] == doc_ids[j] of mint/nn/flashattn.py:238-240
    when each id occupies one contiguous run."""
    b_, t = doc_ids.shape
    starts = torch.ones(b_, t, dtype=torch.bool)
    starts[:, 1:] = doc_ids[:, 1:] != doc_ids[:, :-1]
    flat = starts.reshape(-1).nonzero().reshape(-1).to(torch.int32)
    return torch.cat([flat, torch.tensor([b_ * t], dtype=torch.int32)])


# ---------------------------------------------------------------------------
# KV cache and decode
# ---------------------------------------------------------------------------
class KVCacheOracle:
    """KVCache semantics (mint/kvcache/base.py:4-65) with per-sequence
    lengths: append writes rows [p_b, p_b + T) at p_b = seqlens[b] and sets
    seqlens[b] = p_b + T. The reference keeps one position for the whole batch
    (mint/nn/flashattn.py:202); with equal lengths the two coincide."""

    def __init__(self, batch, max_seq_len, n_kv_heads, head_dim, dtype=torch.float32):
        self.k = torch.zeros(batch, max_seq_len, n_kv_heads, head_dim, dtype=dtype)
        self.v = torch.zeros(batch, max_seq_len, n_kv_heads, head_dim, dtype=dtype)
        self.seqlens = torch.zeros(batch, dtype=torch.int32)

    def append(self, k, v):
        for b in range(k.shape[0]):
            p = int(self.seqlens[b])
            self.k[b, p : p + k.shape[1]] = k[b].to(self.k.dtype)
            self.v[b, p : p + v.shape[1]] = v[b].to(self.v.dtype)
            self.seqlens[b] = p + k.shape[1]


def decode_attention(q, k_cache, v_cache, seqlens, *, window_left=-1, alibi_slopes=None, scale=None, dtype=torch.float32):
    """FlashAttention._attention_with_kvcache for one new token
    (mint/nn/flashattn.py:174-219): q [B, Hq, D] attends to keys
    [0, seqlens[b]) of cache [B, Lmax, Hkv, D] with the bottom-right causal
    mask (which admits every cached key) and the optional left window.
    Returns (o [B, Hq, D], lse [B, Hq])."""
    outs, lses = [], []
    for b in range(q.shape[0]):
        L = int(seqlens[b])
        o, lse = attention_rows(
            q[b][None, None],
            k_cache[b : b + 1, :L],
            v_cache[b : b + 1, :L],
            torch.tensor([0]),
            causal=True,
            window_left=window_left,
            alibi_slopes=alibi_slopes,
            scale=scale,
            dtype=dtype,
        )
        outs.append(o[0, 0])
        lses.append(lse[0, :, 0])
    return torch.stack(outs), torch.stack(lses)


def decode_attention_sdpa(q, k_cache, v_cache, seqlens, *, window_left=-1, dtype=torch.float32):
    """The reference's own decode call chain, restated: per sequence,
    KVCache.update has made keys [0, L) valid (mint/kvcache/base.py:35-50),
    then _attention_with_kvcache transposes to [B, H, L, D]
    (mint/nn/flashattn.py:204-207) and calls _sdpa_attention with causal=True
    and q_len = 1 (mint/nn/flashattn.py:209-218), which builds the
    bottom-right boolean mask and runs SDPA with enable_gqa.
    q [B, Hq, D], caches [B, >=L, Hkv, D] -> o [B, Hq, D] in `dtype`."""
    outs = []
    for b in range(q.shape[0]):
        L = int(seqlens[b])
        qs = q[b].to("cpu", dtype)[None, :, None, :]  # [1, Hq, 1, D]
        ks = k_cache[b, :L].to("cpu", dtype).transpose(0, 1)[None]  # [1, Hkv, L, D]
        vs = v_cache[b, :L].to("cpu", dtype).transpose(0, 1)[None]
        o = sdpa_attention(qs, ks, vs, causal=True, window_size=(window_left, -1))
        outs.append(o[0, :, 0])
    return torch.stack(outs)


def merge_splits(o_parts: torch.Tensor, lse_parts: torch.Tensor):
    """Log-sum-exp merge of split-K partials: lse = log Σ_s exp(lse_s),
    o = Σ_s exp(lse_s - lse) o_s. o_parts [S, ..., D], lse_parts [S, ...]."""
    lse = torch.logsumexp(lse_parts, dim=0)
    w = torch.exp(lse_parts - lse[None])
    w = torch.nan_to_num(w, nan=0.0)
    return (w[..., None] * o_parts).sum(0), lse


def split_attention(q, k, v, splits: list[int], *, scale=None, dtype=torch.float64):
    """Attention of q [Hq, D] over keys k/v [L, Hq, D] computed as independent
    splits at the given boundaries and merged with `merge_splits`."""
    scale = scale if scale is not None else 1.0 / math.sqrt(q.shape[-1])
    bounds = [0, *splits, k.shape[0]]
    ops, lps = [], []
    for s, e in zip(bounds[:-1], bounds[1:]):
        sc = torch.einsum("hd,jhd->hj", q.to(dtype), k[s:e].to(dtype)) * scale
        lse = torch.logsumexp(sc, dim=-1)
        p = torch.exp(sc - lse[:, None])
        ops.append(torch.einsum("hj,jhd->hd", p, v[s:e].to(dtype)))
        lps.append(lse)
    return merge_splits(torch.stack(ops), torch.stack(lps))


# ---------------------------------------------------------------------------
# gradients
# ---------------------------------------------------------------------------
def attention_grads(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    d_o: torch.Tensor,
    *,
    causal: bool,
    window_size: tuple[int, int] = (-1, -1),
    doc_ids: torch.Tensor | None = None,
    alibi_slopes: torch.Tensor | None = None,
    base_attn_mask: torch.Tensor | None = None,
    rope: tuple | None = None,
    scale: float | None = None,
    qk_norm: tuple | None = None,
    dtype=torch.float32,
):
    """(dq, dk, dv) of `attention` for the upstream gradient d_o [B, Tq, Hq, D].

    Torch autograd through the same SDPA restatement: what goda's eager
    training path back-propagates (mint/nn/flashattn.py:221-273 under
    loss.backward()), and what FlashAttentionGQAKernel.backward
    (kernels_/flash_attn_gqa/cuda.py:577-658) computes for Hq == Hkv. With
    Hkv < Hq, dk/dv of a KV head sum its query heads (SDPA's enable_gqa).
    `rope` = (cos, sin, q_positions, k_positions) rotates q and k first
    (mint/nn/pos.py:90-112, applied before attention at mint/nn/attn.py:60),
    so dq/dk refer to the unrotated inputs. `qk_norm` = (q_scale, k_scale,
    eps) applies goda's QK-RMSNorm (`rms_norm`) to q and k before RoPE
    (mint/nn/attn.py:57-60); the result is then (dq, dk, dv, d_q_scale,
    d_k_scale), dq/dk referring to the rows before the norm. Every query row
    must see at least one key, or come out of `attention` as 0 (then its
    gradients are 0).
    """
    qs = q.to("cpu", dtype).detach().requires_grad_(True)
    ks = k.to("cpu", dtype).detach().requires_grad_(True)
    vs = v.to("cpu", dtype).detach().requires_grad_(True)
    with torch.enable_grad():
        qr, kr = qs, ks
        if qk_norm is not None:
            wq = qk_norm[0].to("cpu", dtype).detach().requires_grad_(True)
            wk = qk_norm[1].to("cpu", dtype).detach().requires_grad_(True)
            qr, kr = rms_norm(qr, wq, qk_norm[2]), rms_norm(kr, wk, qk_norm[2])
        if rope is not None:
            cos, sin, qpos, kpos = rope
            qr = apply_rope(qr, cos, sin, qpos)
            kr = apply_rope(kr, cos, sin, kpos)
        o = attention(qr, kr, vs, causal=causal, window_size=window_size, doc_ids=doc_ids,
                      alibi_slopes=alibi_slopes, base_attn_mask=base_attn_mask, scale=scale, dtype=dtype)
        o.backward(d_o.to("cpu", dtype))
    if qk_norm is not None:
        return qs.grad, ks.grad, vs.grad, wq.grad, wk.grad
    return qs.grad, ks.grad, vs.grad


def rms_norm(x: torch.Tensor, scale: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """goda's RMSNorm (mint/nn/norm.py:17-27), as applied to every q and k head
    row before RoPE (mint/nn/attn.py:57-60): in fp32,
    x * rsqrt(mean(x^2, -1) + eps) * (1 + scale), cast back to x's dtype."""
    x_f = x.float() if x.dtype != torch.float64 else x
    var = x_f.pow(2).mean(dim=-1, keepdim=True)
    out = x_f * torch.rsqrt(var + eps) * (1.0 + scale.to(x_f.dtype))
    return out.to(x.dtype)


def attention_grads_chunked(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    d_o: torch.Tensor,
    *,
    causal: bool,
    alibi_slopes: torch.Tensor | None = None,
    scale: float | None = None,
    rows: torch.Tensor | None = None,
    chunk: int = 1024,
    dtype=torch.float32,
):
    """Gradients of one sequence's attention for one KV head's query group,
    computed over query-row chunks so that no [Tq, Tk] matrix of the whole
    sequence is held: q / d_o [Tq, G, D] (the G query heads that share the KV
    head), k / v [Tk, D]. Returns (dq [len(rows), G, D], dk [Tk, D],
    dv [Tk, D]); dk / dv sum the G heads (the GQA reduction) and are complete
    only when `rows` is every row (the default).

    The FlashAttention-2 backward of kernels_/flash_attn_gqa/cuda.py:6-246
    per chunk, with the chunk's own exact softmax: P = softmax(s), o = P v,
    delta = rowsum(dO * o), dS = P * (dO v^T - delta), dq = scale dS k,
    dk += scale dS^T q, dv += P^T dO. Causal alignment is bottom-right, ALiBi
    adds slope_h * (j - i_abs). Inputs are already rotated (RoPE is the
    caller's). Rows with no visible key contribute nothing.
    """
    tq, g, d = q.shape
    tk = k.shape[0]
    scale = scale if scale is not None else 1.0 / math.sqrt(d)
    rows = torch.arange(tq) if rows is None else rows.to(torch.long)
    qd, od = q.to("cpu", dtype), d_o.to("cpu", dtype)
    kd, vd = k.to("cpu", dtype), v.to("cpu", dtype)
    dq = torch.zeros(len(rows), g, d, dtype=dtype)
    dk = torch.zeros(tk, d, dtype=dtype)
    dv = torch.zeros(tk, d, dtype=dtype)
    for c0 in range(0, len(rows), chunk):
        r = rows[c0 : c0 + chunk]
        iabs = (tk - tq) + r  # [R]
        kmax = int(iabs.max()) + 1 if causal else tk  # keys any row of the chunk can see
        kmax = max(0, min(kmax, tk))
        kc, vc = kd[:kmax], vd[:kmax]
        j = torch.arange(kmax)
        s = torch.einsum("rgd,jd->grj", qd[r], kc) * scale  # [G, R, J]
        if alibi_slopes is not None:
            s = s + alibi_slopes.to("cpu", dtype)[:, None, None] * (j[None, :] - iabs[:, None]).to(dtype)[None]
        if causal:
            s = s.masked_fill((j[None, :] > iabs[:, None])[None], float("-inf"))
        lse = torch.logsumexp(s, dim=-1, keepdim=True)
        p = torch.nan_to_num(torch.exp(s - lse), nan=0.0)  # rows with no key: 0
        o = torch.einsum("grj,jd->rgd", p, vc)
        delta = (od[r] * o).sum(-1)  # [R, G]
        dp = torch.einsum("rgd,jd->grj", od[r], vc)
        ds = p * (dp - delta.T[:, :, None])
        dq[c0 : c0 + chunk] = torch.einsum("grj,jd->rgd", ds, kc) * scale
        dk[:kmax] += torch.einsum("grj,rgd->jd", ds, qd[r]) * scale
        dv[:kmax] += torch.einsum("grj,rgd->jd", p, od[r])
    return dq, dk, dv
