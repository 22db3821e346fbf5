"""Pins the CPU oracle (oracle/attention.py) before it is trusted as the
checker of the HIP kernels. The reference ships no golden vectors for this
path, so each function is pinned by an independent float64 brute force
(oracle/brute.py, explicit loops), closed forms, or invariants — chosen so
that a dropped term, a wrong sign or index, or a transposed operand fails.
The `test_planted_*` cases plant such mistakes in a copy of the oracle's
inputs/formulas and assert that the checks catch them."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as ref
from oracle import brute

F64 = torch.float64


def _rand(shape, seed, dtype=F64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float64).to(dtype)


def _brute(q, k, v, **kw):
    o, lse = brute.attention(q.numpy(), k.numpy(), v.numpy(), **kw)
    return torch.from_numpy(o), torch.from_numpy(lse)


# ---------------------------------------------------------------------------
# attention core: SDPA restatement vs explicit-loop brute force
# ---------------------------------------------------------------------------
CASES = [
    # b, tq, tk, hq, hkv, d, causal
    (1, 5, 5, 2, 2, 8, True),
    (2, 7, 7, 4, 2, 8, True),
    (2, 3, 9, 6, 2, 16, True),  # Lq < Lk: bottom-right alignment
    (1, 6, 6, 4, 1, 8, False),  # MQA
    (2, 4, 11, 8, 4, 8, False),
]


@pytest.mark.parametrize("b,tq,tk,hq,hkv,d,causal", CASES)
def test_sdpa_matches_brute(b, tq, tk, hq, hkv, d, causal):
    q, k, v = _rand((b, tq, hq, d), 1), _rand((b, tk, hkv, d), 2), _rand((b, tk, hkv, d), 3)
    o = ref.attention(q, k, v, causal=causal, dtype=F64)
    o_b, lse_b = _brute(q, k, v, causal=causal)
    assert torch.allclose(o, o_b, atol=1e-12)
    o_r, lse_r = ref.attention_rows(q, k, v, torch.arange(tq), causal=causal, dtype=F64)
    assert torch.allclose(o_r, o_b, atol=1e-12)
    assert torch.allclose(lse_r, lse_b, atol=1e-12)


@pytest.mark.parametrize("window", [0, 1, 3, 20])
def test_window_matches_brute(window):
    b, tq, tk, hq, hkv, d = 2, 6, 10, 4, 2, 8
    q, k, v = _rand((b, tq, hq, d), 4), _rand((b, tk, hkv, d), 5), _rand((b, tk, hkv, d), 6)
    o = ref.attention(q, k, v, causal=True, window_size=(window, -1), dtype=F64)
    o_b, lse_b = _brute(q, k, v, causal=True, window_left=window)
    assert torch.allclose(o, o_b, atol=1e-12)
    o_r, lse_r = ref.attention_rows(q, k, v, torch.arange(tq), causal=True, window_left=window, dtype=F64)
    assert torch.allclose(o_r, o_b, atol=1e-12) and torch.allclose(lse_r, lse_b, atol=1e-12)


@pytest.mark.parametrize("causal", [True, False])
def test_alibi_matches_brute(causal):
    b, tq, tk, hq, hkv, d = 1, 5, 8, 4, 1, 8
    q, k, v = _rand((b, tq, hq, d), 7), _rand((b, tk, hkv, d), 8), _rand((b, tk, hkv, d), 9)
    slopes = torch.tensor(ref.alibi_slopes(hq), dtype=F64)
    o = ref.attention(q, k, v, causal=causal, alibi_slopes=slopes, dtype=F64)
    o_b, lse_b = _brute(q, k, v, causal=causal, slopes=slopes.numpy())
    assert torch.allclose(o, o_b, atol=1e-12)
    o_r, lse_r = ref.attention_rows(q, k, v, torch.arange(tq), causal=causal, alibi_slopes=slopes, dtype=F64)
    assert torch.allclose(o_r, o_b, atol=1e-12) and torch.allclose(lse_r, lse_b, atol=1e-12)


def test_scale_matches_brute():
    q, k, v = _rand((1, 4, 2, 8), 10), _rand((1, 4, 2, 8), 11), _rand((1, 4, 2, 8), 12)
    o = ref.attention(q, k, v, causal=True, scale=0.37, dtype=F64)
    o_b, _ = _brute(q, k, v, causal=True, scale=0.37)
    assert torch.allclose(o, o_b, atol=1e-12)


def test_doc_ids_match_brute_and_varlen():
    b, t, hq, hkv, d = 2, 9, 4, 2, 8
    q, k, v = _rand((b, t, hq, d), 13), _rand((b, t, hkv, d), 14), _rand((b, t, hkv, d), 15)
    doc = torch.tensor([[0, 0, 0, 1, 1, 2, 2, 2, 2], [5, 5, 5, 5, 5, 6, 6, 7, 7]])
    o = ref.attention(q, k, v, causal=True, doc_ids=doc, dtype=F64)
    o_b, _ = _brute(q, k, v, causal=True, doc_ids=doc.numpy())
    assert torch.allclose(o, o_b, atol=1e-12)
    cu = ref.doc_ids_to_cu_seqlens(doc)
    assert cu.tolist() == [0, 3, 5, 9, 14, 16, 18]
    o_v = ref.varlen_attention(q.reshape(-1, hq, d), k.reshape(-1, hkv, d), v.reshape(-1, hkv, d), cu, cu,
                               causal=True, dtype=F64)
    assert torch.allclose(o_v.reshape(b, t, hq, d), o_b, atol=1e-12)


def _bool(shape, seed, p=0.7):
    g = torch.Generator().manual_seed(seed)
    return torch.rand(shape, generator=g) < p


# base_attn_mask forms goda's callers pass (broadcast against [B, Hq, Tq, Tk])
MASK_FORMS = ["keypad", "full", "per_head", "two_d"]


def _mask_of(form, b, hq, tq, tk, seed):
    if form == "keypad":  # SFT padding: [B, 1, 1, Tk]
        m = _bool((b, 1, 1, tk), seed)
    elif form == "full":
        m = _bool((b, 1, tq, tk), seed)
    elif form == "per_head":
        m = _bool((b, hq, tq, tk), seed)
    else:
        m = _bool((tq, tk), seed)
    return m


@pytest.mark.parametrize("form", MASK_FORMS)
@pytest.mark.parametrize("causal,window,alibi", [(True, -1, False), (False, -1, False), (True, 2, True), (False, -1, True)])
def test_base_mask_matches_brute(form, causal, window, alibi):
    b, tq, tk, hq, hkv, d = 2, 5, 8, 4, 2, 8
    q, k, v = _rand((b, tq, hq, d), 31), _rand((b, tk, hkv, d), 32), _rand((b, tk, hkv, d), 33)
    m = _mask_of(form, b, hq, tq, tk, 34)
    slopes = torch.tensor(ref.alibi_slopes(hq), dtype=F64) if alibi else None
    o = ref.attention(q, k, v, causal=causal, window_size=(window, -1), alibi_slopes=slopes, base_attn_mask=m,
                      dtype=F64)
    o_b, lse_b = _brute(q, k, v, causal=causal, window_left=window, mask=m.numpy(),
                        slopes=None if slopes is None else slopes.numpy())
    assert torch.allclose(o, o_b, atol=1e-12)
    o_r, lse_r = ref.attention_rows(q, k, v, torch.arange(tq), causal=causal, window_left=window,
                                    alibi_slopes=slopes, base_attn_mask=m, dtype=F64)
    assert torch.allclose(torch.nan_to_num(o_r), o_b, atol=1e-12)
    assert torch.equal(torch.isinf(lse_r), torch.isinf(lse_b))
    fin = torch.isfinite(lse_b)
    assert torch.allclose(lse_r[fin], lse_b[fin], atol=1e-12)


def test_base_mask_rows_with_no_key_give_zero():
    """A row the mask hides entirely comes out as 0 with lse = -inf in the
    brute force, and the restatement (this torch's SDPA) agrees."""
    b, tq, tk, hq, d = 1, 4, 6, 2, 8
    q, k, v = _rand((b, tq, hq, d), 35), _rand((b, tk, hq, d), 36), _rand((b, tk, hq, d), 37)
    m = torch.ones(b, 1, tq, tk, dtype=torch.bool)
    m[0, 0, 2] = False
    o_b, lse_b = _brute(q, k, v, causal=False, mask=m.numpy())
    assert torch.all(o_b[0, 2] == 0) and torch.all(torch.isinf(lse_b[0, :, 2]))
    o = ref.attention(q, k, v, causal=False, base_attn_mask=m, dtype=F64)
    assert torch.allclose(o, o_b, atol=1e-12)


def test_base_mask_and_doc_ids_compose_as_a_conjunction():
    b, t, hq, hkv, d = 2, 7, 2, 1, 8
    q, k, v = _rand((b, t, hq, d), 38), _rand((b, t, hkv, d), 39), _rand((b, t, hkv, d), 40)
    doc = torch.tensor([[0, 0, 0, 1, 1, 1, 1], [3, 3, 4, 4, 4, 5, 5]])
    m = _bool((b, 1, 1, t), 41)
    o = ref.attention(q, k, v, causal=True, doc_ids=doc, base_attn_mask=m, dtype=F64)
    both = (doc[:, None, :, None] == doc[:, None, None, :]) & m
    o_b, _ = _brute(q, k, v, causal=True, mask=both.numpy())
    assert torch.allclose(o, o_b, atol=1e-12)


def test_planted_transposed_mask_is_caught():
    """Reading the mask as [.., key, query] instead of [.., query, key] fails
    the brute-force comparison."""
    b, t, hq, d = 1, 6, 2, 8
    q, k, v = _rand((b, t, hq, d), 42), _rand((b, t, hq, d), 43), _rand((b, t, hq, d), 44)
    m = _bool((b, 1, t, t), 45, p=0.5)
    o_wrong = ref.attention(q, k, v, causal=False, base_attn_mask=m.transpose(-1, -2), dtype=F64)
    o_b, _ = _brute(q, k, v, causal=False, mask=m.numpy())
    assert not torch.allclose(torch.nan_to_num(o_wrong), o_b, atol=1e-3)


def test_causal_square_equals_is_causal():
    """With Lq == Lk and no other mask, goda's explicit boolean mask equals
    SDPA's is_causal=True (mint/nn/flashattn.py:245-273)."""
    q, k, v = _rand((1, 3, 7, 8), 16), _rand((1, 3, 7, 8), 17), _rand((1, 3, 7, 8), 18)
    o_mask = ref.sdpa_attention(q, k, v, causal=True)
    o_is = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True)
    assert torch.allclose(o_mask, o_is, atol=1e-12)


def test_gqa_equals_repeated_mha():
    b, t, hq, hkv, d = 2, 6, 6, 2, 8
    q, k, v = _rand((b, t, hq, d), 19), _rand((b, t, hkv, d), 20), _rand((b, t, hkv, d), 21)
    o = ref.attention(q, k, v, causal=True, dtype=F64)
    rep = hq // hkv
    o_mha = ref.attention(q, k.repeat_interleave(rep, 2), v.repeat_interleave(rep, 2), causal=True, dtype=F64)
    assert torch.allclose(o, o_mha, atol=1e-12)


def test_brute_lse_closed_form():
    """One key: o = v, lse = the single scaled score."""
    q, k, v = _rand((1, 1, 1, 4), 22), _rand((1, 1, 1, 4), 23), _rand((1, 1, 1, 4), 24)
    o, lse = _brute(q, k, v, causal=True)
    s = float((q[0, 0, 0] * k[0, 0, 0]).sum()) / 2.0
    assert torch.allclose(o, v) and abs(float(lse[0, 0, 0]) - s) < 1e-12


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------
def test_rope_tables_closed_form():
    cos, sin = ref.rope_tables(64, 16, 10000.0)
    p, i = 37, 5
    theta = p * 10000.0 ** (-(2.0 * i) / 16)
    assert abs(float(cos[p, i]) - math.cos(theta)) < 1e-5
    assert abs(float(sin[p, i]) - math.sin(theta)) < 1e-5
    cos_s, _ = ref.rope_tables(64, 16, 10000.0, scale_factor=4.0)
    assert abs(float(cos_s[p, i]) - math.cos(theta / 4.0)) < 1e-5


def test_rope_matches_brute_and_invariants():
    t, h, d = 24, 3, 16
    x = _rand((2, t, h, d), 25)
    cos, sin = ref.rope_tables(t, d, 10000.0)
    pos = torch.arange(t)
    y = ref.apply_rope(x, cos.to(F64), sin.to(F64), pos)
    y_b = torch.from_numpy(brute.rope(x.numpy(), pos.numpy(), 10000.0))
    assert torch.allclose(y, y_b, atol=1e-5)
    # position 0 is the identity
    assert torch.allclose(y[:, 0], x[:, 0])
    # each (i, i + D/2) pair keeps its norm
    n_x = x[..., : d // 2] ** 2 + x[..., d // 2 :] ** 2
    n_y = y[..., : d // 2] ** 2 + y[..., d // 2 :] ** 2
    assert torch.allclose(n_x, n_y, atol=1e-10)


def test_rope_relative_positions():
    """q_m . k_n depends only on m - n (float64 tables from the closed form)."""
    d = 16
    q, k = _rand((1, 1, 1, d), 26), _rand((1, 1, 1, d), 27)
    half = torch.arange(0, d, 2, dtype=F64)
    inv = 1.0 / (10000.0 ** (half / d))
    ang = torch.outer(torch.arange(40, dtype=F64), inv)
    cos, sin = ang.cos(), ang.sin()

    def dot(m, n):
        qm = ref.apply_rope(q, cos, sin, torch.tensor([m]))
        kn = ref.apply_rope(k, cos, sin, torch.tensor([n]))
        return float((qm * kn).sum())

    assert abs(dot(10, 3) - dot(30, 23)) < 1e-10
    assert abs(dot(5, 5) - dot(0, 0)) < 1e-10
    assert abs(dot(10, 3) - dot(3, 10)) > 1e-6  # not symmetric in general


# ---------------------------------------------------------------------------
# ALiBi
# ---------------------------------------------------------------------------
def test_alibi_slopes_closed_form():
    # n = 16 (cfg3): s_h = 2^(-(h+1)/2) for 0-based h
    assert np.allclose(ref.alibi_slopes(16), [2.0 ** (-(h + 1) / 2) for h in range(16)], rtol=1e-14)
    # n = 8: 2^-1 ... 2^-8
    assert np.allclose(ref.alibi_slopes(8), [2.0 ** (-(h + 1)) for h in range(8)], rtol=1e-14)
    # non power of two: the 4 slopes of n=4, then every other slope of n=8
    assert np.allclose(ref.alibi_slopes(6), [2**-2, 2**-4, 2**-6, 2**-8, 2**-1, 2**-3], rtol=1e-14)


def test_alibi_bias_sign_and_diagonal():
    slopes = torch.tensor([0.5, 0.25], dtype=F64)
    bias = ref.alibi_bias(slopes, 3, 5, F64)  # queries at absolute 2, 3, 4
    assert bias.shape == (1, 2, 3, 5)
    assert float(bias[0, 0, 0, 2]) == 0.0 and float(bias[0, 1, 2, 4]) == 0.0
    assert float(bias[0, 0, 0, 0]) == -1.0  # key 2 positions back: 0.5 * -2
    assert float(bias[0, 1, 2, 1]) == -0.75


# ---------------------------------------------------------------------------
# decode, KV cache and split-K merge
# ---------------------------------------------------------------------------
def test_decode_equals_last_prefill_row_and_reference_chain():
    b, lmax, hq, hkv, d = 3, 20, 4, 2, 8
    lens = torch.tensor([1, 9, 20], dtype=torch.int32)
    q, kc, vc = _rand((b, hq, d), 28), _rand((b, lmax, hkv, d), 29), _rand((b, lmax, hkv, d), 30)
    o, lse = ref.decode_attention(q, kc, vc, lens, dtype=F64)
    o_sdpa = ref.decode_attention_sdpa(q, kc, vc, lens, dtype=F64)
    assert torch.allclose(o, o_sdpa, atol=1e-12)
    for i in range(b):
        L = int(lens[i])
        o_b, lse_b = _brute(q[i][None, None], kc[i : i + 1, :L], vc[i : i + 1, :L], causal=True)
        assert torch.allclose(o[i], o_b[0, 0], atol=1e-12)
        assert torch.allclose(lse[i], lse_b[0, :, 0], atol=1e-12)


def test_decode_window_matches_brute():
    b, lmax, hq, hkv, d, w = 2, 16, 2, 1, 8, 4
    lens = torch.tensor([3, 16], dtype=torch.int32)
    q, kc, vc = _rand((b, hq, d), 31), _rand((b, lmax, hkv, d), 32), _rand((b, lmax, hkv, d), 33)
    o, _ = ref.decode_attention(q, kc, vc, lens, window_left=w, dtype=F64)
    o2 = ref.decode_attention_sdpa(q, kc, vc, lens, window_left=w, dtype=F64)
    for i in range(b):
        L = int(lens[i])
        o_b, _ = _brute(q[i][None, None], kc[i : i + 1, :L], vc[i : i + 1, :L], causal=True, window_left=w)
        assert torch.allclose(o[i], o_b[0, 0], atol=1e-12) and torch.allclose(o2[i], o_b[0, 0], atol=1e-12)


@pytest.mark.parametrize("splits", [[], [1], [3, 7], [1, 2, 3, 4, 5, 6, 7, 8, 9]])
def test_split_merge_independent_of_splits(splits):
    L, h, d = 10, 3, 8
    q, k, v = _rand((h, d), 34), _rand((L, h, d), 35), _rand((L, h, d), 36)
    o, lse = ref.split_attention(q, k, v, splits)
    o_b, lse_b = _brute(q[None, None], k[None], v[None], causal=False)
    assert torch.allclose(o, o_b[0, 0], atol=1e-12)
    assert torch.allclose(lse, lse_b[0, :, 0], atol=1e-12)


def test_merge_handles_empty_split():
    o_parts = torch.stack([torch.ones(2, 4), torch.zeros(2, 4)]).to(F64)
    lse_parts = torch.tensor([[0.0, 1.0], [-math.inf, -math.inf]], dtype=F64)
    o, lse = ref.merge_splits(o_parts, lse_parts)
    assert torch.allclose(o, torch.ones(2, 4, dtype=F64)) and torch.allclose(lse, lse_parts[0])


def test_kvcache_oracle_matches_reference_update():
    """Equal lengths: append == KVCache.update at start_pos = seqlens[0]
    (mint/kvcache/base.py:35-50), restated with plain slicing."""
    b, lmax, h, d = 2, 10, 2, 4
    c = ref.KVCacheOracle(b, lmax, h, d, dtype=F64)
    k_ref = torch.zeros(b, lmax, h, d, dtype=F64)
    pos = 0
    for step, tn in enumerate([3, 1, 2]):
        kn = _rand((b, tn, h, d), 40 + step)
        c.append(kn, kn)
        k_ref[:b, pos : pos + tn] = kn
        pos += tn
        assert c.seqlens.tolist() == [pos] * b
    assert torch.equal(c.k, k_ref) and torch.equal(c.v, k_ref)


# ---------------------------------------------------------------------------
# planted mistakes: the checks above must catch each of them
# ---------------------------------------------------------------------------
def test_planted_wrong_gqa_mapping_is_caught():
    b, t, hq, hkv, d = 1, 5, 4, 2, 8
    q, k, v = _rand((b, t, hq, d), 50), _rand((b, t, hkv, d), 51), _rand((b, t, hkv, d), 52)
    o_b, _ = _brute(q, k, v, causal=True)
    # h % Hkv instead of h // (Hq/Hkv)
    idx = torch.tensor([h % hkv for h in range(hq)])
    o_bad = ref.attention(q, k[:, :, idx], v[:, :, idx], causal=True, dtype=F64)
    assert not torch.allclose(o_bad, o_b, atol=1e-6)


def test_planted_top_left_causal_is_caught():
    b, tq, tk, h, d = 1, 3, 8, 2, 8
    q, k, v = _rand((b, tq, h, d), 53), _rand((b, tk, h, d), 54), _rand((b, tk, h, d), 55)
    o_b, _ = _brute(q, k, v, causal=True)
    o_bad = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), is_causal=True
    ).transpose(1, 2)  # top-left aligned for Lq < Lk
    assert not torch.allclose(o_bad, o_b, atol=1e-6)


def test_planted_alibi_sign_is_caught():
    b, t, h, d = 1, 6, 2, 8
    q, k, v = _rand((b, t, h, d), 56), _rand((b, t, h, d), 57), _rand((b, t, h, d), 58)
    slopes = torch.tensor(ref.alibi_slopes(h), dtype=F64)
    o_b, _ = _brute(q, k, v, causal=True, slopes=slopes.numpy())
    o_bad = ref.attention(q, k, v, causal=True, alibi_slopes=-slopes, dtype=F64)
    assert not torch.allclose(o_bad, o_b, atol=1e-6)


def test_planted_rope_pairing_is_caught():
    """Interleaved (2i, 2i+1) pairing instead of goda's half-split pairing."""
    t, d = 6, 8
    x = _rand((1, t, 1, d), 59)
    pos = torch.arange(t)
    y_b = torch.from_numpy(brute.rope(x.numpy(), pos.numpy(), 10000.0))
    cos, sin = ref.rope_tables(t, d, 10000.0)
    xi = x.reshape(1, t, 1, d // 2, 2)
    c, s = cos.to(F64)[:, None, :], sin.to(F64)[:, None, :]
    y_bad = torch.stack([xi[..., 0] * c - xi[..., 1] * s, xi[..., 0] * s + xi[..., 1] * c], -1).reshape(1, t, 1, d)
    assert not torch.allclose(y_bad, y_b, atol=1e-4)


# ---------------------------------------------------------------------------
# gradients: explicit FA2 backward (brute) vs finite differences, and the
# autograd oracle vs the brute backward
# ---------------------------------------------------------------------------
def _loss_fd(fwd, args: list[np.ndarray], d_o: np.ndarray, h: float = 1e-5):
    """Central finite differences of L = sum(o * d_o) w.r.t. every element of
    every array in args (float64)."""
    grads = []
    for a_idx, a in enumerate(args):
        g = np.zeros_like(a)
        it = np.nditer(a, flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            old = a[idx]
            a[idx] = old + h
            lp = float((fwd(*args) * d_o).sum())
            a[idx] = old - h
            lm = float((fwd(*args) * d_o).sum())
            a[idx] = old
            g[idx] = (lp - lm) / (2 * h)
        grads.append(g)
    return grads


GRAD_CASES = [
    # name, tq, tk, hq, hkv, d, kwargs
    ("causal_gqa_bottom_right", 4, 6, 4, 2, 3, dict(causal=True)),
    ("causal_window", 5, 5, 2, 1, 3, dict(causal=True, window_left=2)),
    ("noncausal_alibi", 3, 4, 2, 1, 3, dict(causal=False, slopes=np.array([0.5, 0.25]))),
    ("causal_empty_rows", 6, 4, 2, 1, 3, dict(causal=True)),
    ("doc_ids", 5, 5, 2, 2, 3, dict(causal=True, doc_ids=np.array([[0, 0, 1, 1, 1]]))),
    # base_attn_mask with a row it hides entirely (row 1) and a per-head form
    ("base_mask", 4, 5, 2, 1, 3, dict(causal=False, mask=np.array(
        [[[[1, 0, 1, 1, 0], [0, 0, 0, 0, 0], [1, 1, 0, 1, 1], [0, 1, 1, 0, 1]],
          [[1, 1, 1, 0, 0], [0, 0, 0, 0, 0], [0, 1, 1, 1, 1], [1, 0, 0, 1, 1]]]], dtype=bool))),
]


@pytest.mark.parametrize("name,tq,tk,hq,hkv,d,kw", GRAD_CASES, ids=[c[0] for c in GRAD_CASES])
def test_brute_backward_matches_finite_differences(name, tq, tk, hq, hkv, d, kw):
    rng = np.random.default_rng(7)
    q = rng.standard_normal((1, tq, hq, d))
    k = rng.standard_normal((1, tk, hkv, d))
    v = rng.standard_normal((1, tk, hkv, d))
    d_o = rng.standard_normal((1, tq, hq, d))
    dq, dk, dv = brute.attention_backward(q, k, v, d_o, **kw)
    fq, fk, fv = _loss_fd(lambda a, b_, c: brute.attention(a, b_, c, **kw)[0], [q, k, v], d_o)
    assert np.abs(dq - fq).max() < 1e-7
    assert np.abs(dk - fk).max() < 1e-7
    assert np.abs(dv - fv).max() < 1e-7


@pytest.mark.parametrize("plant", ["no_delta", "first_head_only"])
def test_planted_backward_mistakes_are_caught(plant):
    rng = np.random.default_rng(8)
    q = rng.standard_normal((1, 4, 4, 3))
    k = rng.standard_normal((1, 4, 2, 3))
    v = rng.standard_normal((1, 4, 2, 3))
    d_o = rng.standard_normal((1, 4, 4, 3))
    kw = dict(causal=True)
    dq, dk, dv = brute.attention_backward(q, k, v, d_o, plant=plant, **kw)
    fq, fk, fv = _loss_fd(lambda a, b_, c: brute.attention(a, b_, c, **kw)[0], [q, k, v], d_o)
    worst = max(np.abs(dq - fq).max(), np.abs(dk - fk).max(), np.abs(dv - fv).max())
    assert worst > 1e-3


@pytest.mark.parametrize(
    "b,tq,tk,hq,hkv,d,causal,window,alibi",
    [
        (2, 6, 6, 4, 2, 8, True, -1, False),
        (1, 5, 9, 4, 1, 8, True, 3, False),
        (2, 7, 7, 2, 2, 8, False, -1, True),
        (1, 4, 4, 8, 2, 16, True, -1, True),
    ],
)
def test_autograd_oracle_matches_brute_backward(b, tq, tk, hq, hkv, d, causal, window, alibi):
    q, k, v = _rand((b, tq, hq, d), 11), _rand((b, tk, hkv, d), 12), _rand((b, tk, hkv, d), 13)
    d_o = _rand((b, tq, hq, d), 14)
    slopes = torch.tensor(ref.alibi_slopes(hq), dtype=F64) if alibi else None
    dq, dk, dv = ref.attention_grads(q, k, v, d_o, causal=causal, window_size=(window, -1), alibi_slopes=slopes, dtype=F64)
    bq, bk, bv = brute.attention_backward(
        q.numpy(), k.numpy(), v.numpy(), d_o.numpy(), causal=causal, window_left=window,
        slopes=None if slopes is None else slopes.numpy(),
    )
    assert np.abs(dq.numpy() - bq).max() < 1e-10
    assert np.abs(dk.numpy() - bk).max() < 1e-10
    assert np.abs(dv.numpy() - bv).max() < 1e-10


@pytest.mark.parametrize("form", MASK_FORMS)
def test_autograd_oracle_with_base_mask_matches_brute_backward(form):
    b, tq, tk, hq, hkv, d = 2, 5, 7, 4, 2, 8
    q, k, v = _rand((b, tq, hq, d), 46), _rand((b, tk, hkv, d), 47), _rand((b, tk, hkv, d), 48)
    d_o = _rand((b, tq, hq, d), 49)
    m = _mask_of(form, b, hq, tq, tk, 50)
    dq, dk, dv = ref.attention_grads(q, k, v, d_o, causal=True, base_attn_mask=m, dtype=F64)
    bq, bk, bv = brute.attention_backward(q.numpy(), k.numpy(), v.numpy(), d_o.numpy(), causal=True, mask=m.numpy())
    assert np.abs(dq.numpy() - bq).max() < 1e-10
    assert np.abs(dk.numpy() - bk).max() < 1e-10
    assert np.abs(dv.numpy() - bv).max() < 1e-10


def test_autograd_oracle_through_rope_matches_finite_differences():
    """dq, dk refer to the unrotated inputs: the rotation's transpose is applied
    to the gradients of the rotated rows (checked against finite differences of
    brute-force attention over brute-force RoPE)."""
    tq, tk, hq, hkv, d, base = 3, 5, 2, 1, 4, 10000.0
    rng = np.random.default_rng(9)
    q = rng.standard_normal((1, tq, hq, d))
    k = rng.standard_normal((1, tk, hkv, d))
    v = rng.standard_normal((1, tk, hkv, d))
    d_o = rng.standard_normal((1, tq, hq, d))
    qpos, kpos = np.arange(tk - tq, tk) + 3, np.arange(tk) + 3
    cos, sin = ref.rope_tables(16, d, base)
    dq, dk, dv = ref.attention_grads(
        torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), torch.from_numpy(d_o), causal=True,
        rope=(cos.double(), sin.double(), torch.from_numpy(qpos), torch.from_numpy(kpos)), dtype=F64,
    )

    def fwd(a, b_, c):
        return brute.attention(brute.rope(a, qpos, base), brute.rope(b_, kpos, base), c, causal=True)[0]

    fq, fk, fv = _loss_fd(fwd, [q, k, v], d_o)
    # the fp32 cos/sin tables limit agreement to ~1e-7
    assert np.abs(dq.numpy() - fq).max() < 1e-5
    assert np.abs(dk.numpy() - fk).max() < 1e-5
    assert np.abs(dv.numpy() - fv).max() < 1e-7


# ---------------------------------------------------------------------------
# QK-RMSNorm
# ---------------------------------------------------------------------------
def test_rms_norm_matches_library_and_closed_form():
    x = _rand((2, 5, 3, 16), 21)
    scale = _rand((16,), 22) * 0.1
    y = ref.rms_norm(x, scale, 1e-6)
    # library routine: torch's rms_norm with weight (1 + scale)
    assert torch.allclose(y, torch.nn.functional.rms_norm(x, (16,), weight=1.0 + scale, eps=1e-6), atol=1e-12)
    # closed form: a constant row c maps to sign(c) * (1 + scale) (eps -> 0)
    c = torch.full((16,), -3.0, dtype=F64)
    assert torch.allclose(ref.rms_norm(c, scale, 0.0), -(1.0 + scale), atol=1e-12)
    # zero-initialised scale (mint/nn/norm.py:13) gives unit RMS rows
    y0 = ref.rms_norm(x, torch.zeros(16, dtype=F64), 0.0)
    assert torch.allclose(y0.pow(2).mean(-1), torch.ones(2, 5, 3, dtype=F64), atol=1e-12)


def test_planted_rms_norm_without_one_plus_is_caught():
    x = _rand((4, 16), 23)
    scale = _rand((16,), 24) * 0.1
    wrong = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * scale  # drops the "1 +"
    lib = torch.nn.functional.rms_norm(x, (16,), weight=1.0 + scale, eps=1e-6)
    assert not torch.allclose(wrong, lib, atol=1e-3)
    assert torch.allclose(ref.rms_norm(x, scale, 1e-6), lib, atol=1e-12)


def test_autograd_oracle_through_qk_norm_matches_finite_differences():
    """With the QK-RMSNorm before RoPE, dq / dk refer to the rows before the
    norm and the scales get their own gradients: checked against finite
    differences of brute-force attention over torch's library rms_norm and
    brute-force RoPE."""
    tq, tk, hq, hkv, d, base, eps = 3, 4, 2, 1, 4, 10000.0, 1e-6
    rng = np.random.default_rng(12)
    q = rng.standard_normal((1, tq, hq, d))
    k = rng.standard_normal((1, tk, hkv, d))
    v = rng.standard_normal((1, tk, hkv, d))
    wq = 0.3 * rng.standard_normal(d)
    wk = 0.3 * rng.standard_normal(d)
    d_o = rng.standard_normal((1, tq, hq, d))
    qpos, kpos = np.arange(tk - tq, tk), np.arange(tk)
    cos, sin = ref.rope_tables(8, d, base)
    t = torch.from_numpy
    dq, dk, dv, dwq, dwk = ref.attention_grads(
        t(q), t(k), t(v), t(d_o), causal=True, rope=(cos.double(), sin.double(), t(qpos), t(kpos)),
        qk_norm=(t(wq), t(wk), eps), dtype=F64,
    )

    def norm(x, w):
        return torch.nn.functional.rms_norm(t(x), (d,), weight=1.0 + t(w), eps=eps).numpy()

    def fwd(a, b_, c, wa, wb):
        qa = brute.rope(norm(a, wa), qpos, base)
        kb = brute.rope(norm(b_, wb), kpos, base)
        return brute.attention(qa, kb, c, causal=True)[0]

    fq, fk, fv, fwq, fwk = _loss_fd(fwd, [q, k, v, wq, wk], d_o)
    # the fp32 cos/sin tables limit agreement to ~1e-7
    for got, want in ((dq, fq), (dk, fk), (dv, fv), (dwq, fwq), (dwk, fwk)):
        assert np.abs(got.numpy() - want).max() < 1e-5
    # a dropped "1 +" in the norm's backward would scale dq by w / (1 + w)
    assert np.abs(fq).max() > 1e-2


@pytest.mark.parametrize("causal,alibi,tq,tk", [(True, False, 13, 13), (True, True, 9, 17), (False, False, 11, 7),
                                                (False, True, 6, 6)])
def test_chunked_grads_match_autograd_oracle(causal, alibi, tq, tk):
    """The row-chunked backward (used on full-size shapes) equals the autograd
    oracle for one (sequence, KV head) group: chunk sizes that do and do not
    divide the rows, bottom-right alignment, ALiBi, and sampled dq rows."""
    g, d = 3, 8
    q, k, v = _rand((1, tq, g, d), 61), _rand((1, tk, 1, d), 62), _rand((1, tk, 1, d), 63)
    d_o = _rand((1, tq, g, d), 64)
    slopes = torch.tensor([0.5, 0.25, 0.125], dtype=F64) if alibi else None
    dq, dk, dv = ref.attention_grads(q, k, v, d_o, causal=causal, alibi_slopes=slopes, dtype=F64)
    for chunk in (1, 4, 64):
        cq, ck, cv = ref.attention_grads_chunked(q[0], k[0, :, 0], v[0, :, 0], d_o[0], causal=causal,
                                                 alibi_slopes=slopes, chunk=chunk, dtype=F64)
        assert torch.allclose(cq, dq[0], atol=1e-10)
        assert torch.allclose(ck, dk[0, :, 0], atol=1e-10) and torch.allclose(cv, dv[0, :, 0], atol=1e-10)
    rows = torch.tensor([0, tq // 2, tq - 1])
    cq, _, _ = ref.attention_grads_chunked(q[0], k[0, :, 0], v[0, :, 0], d_o[0], causal=causal, alibi_slopes=slopes,
                                           rows=rows, chunk=2, dtype=F64)
    assert torch.allclose(cq, dq[0, rows], atol=1e-10)
