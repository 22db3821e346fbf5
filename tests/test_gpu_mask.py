"""base_attn_mask parity (mint/nn/flashattn.py:236-255): the bit-packed mask
applied inside the HIP forward and backward kernels (through the C-ABI)
against the CPU oracle, whose mask path tests/test_oracle.py pins against the
float64 brute force.

Mask forms: SFT key padding [B, 1, 1, Lk], a full [B, 1, Lq, Lk] mask, a
per-head [B, Hq, Lq, Lk] mask and a 2-D [Lq, Lk] mask, composed with causal
(bottom-right), left windows, ALiBi and doc_ids. Rows the mask hides entirely
give o = 0 and lse = -inf. Tolerances: the north-star bounds of
tests/helpers.py (forward, absolute) and tests/test_gpu_backward.py
(gradients)."""

from __future__ import annotations

import pytest
import torch

from goda_amd import ops
from goda_amd import workloads as wl
from goda_amd.mint.nn import FlashAttention
from oracle import attention as ref
from tests.helpers import TOL, lse_err, max_err
from tests.test_gpu_backward import _check

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rand(shape, dtype, seed, std=0.5):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).to(dtype)


def _mask(form, b, hq, tq, tk, seed, p=0.75, hidden_row=None):
    g = torch.Generator().manual_seed(seed)
    shape = {"keypad": (b, 1, 1, tk), "full": (b, 1, tq, tk), "per_head": (b, hq, tq, tk), "two_d": (tq, tk)}[form]
    m = torch.rand(shape, generator=g) < p
    if form == "keypad":
        m[..., -(tk // 5):] = False  # padded tail, as SFT batches have
        m[..., 0] = True
    if hidden_row is not None and form in ("full", "per_head", "two_d"):
        m[..., hidden_row, :] = False
    return m


def _fwd_case(b, tq, tk, hq, hkv, d, dtype, form, *, causal, window=-1, alibi=False, rope=False, seed=0):
    q = _rand((b, tq, hq, d), dtype, seed)
    k = _rand((b, tk, hkv, d), dtype, seed + 1)
    v = _rand((b, tk, hkv, d), dtype, seed + 2)
    m = _mask(form, b, hq, tq, tk, seed + 3, hidden_row=tq // 3)
    kw, okw = {}, {}
    if alibi:
        slopes = torch.tensor(wl.alibi_slopes(hq), dtype=torch.float32)
        kw["alibi_slopes"], okw["alibi_slopes"] = slopes.to(DEV), slopes
    qr, kr = q.float(), k.float()
    if rope:
        cos, sin = wl.rope_tables(tk + 8, d, 10000.0)
        kw.update(rope_cos=cos.to(DEV), rope_sin=sin.to(DEV), rope_q=True, rope_k=True)
        qr = ref.apply_rope(qr, cos, sin, torch.arange(tk - tq, tk))
        kr = ref.apply_rope(kr, cos, sin, torch.arange(tk))
    o, lse = ops.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal, window_left=window,
                                   attn_mask=m.to(DEV), return_lse=True, **kw)
    torch.cuda.synchronize()
    o_ref, lse_ref = ref.attention_rows(qr, kr, v.float(), torch.arange(tq), causal=causal, window_left=window,
                                        base_attn_mask=m, **okw)
    o_ref = torch.nan_to_num(o_ref)
    eo, el = max_err(o, o_ref), lse_err(lse, lse_ref)
    what = f"{form} b{b} tq{tq} tk{tk} h{hq}/{hkv} d{d} {dtype} causal={causal} w={window}"
    assert eo <= TOL[dtype], f"{what}: o err {eo}"
    assert el <= (5e-3 if dtype != torch.float32 else 1e-4), f"{what}: lse err {el}"
    # the oracle's SDPA restatement of the whole call agrees too
    o_sdpa = ref.attention(qr, kr, v.float(), causal=causal, window_size=(window, -1), base_attn_mask=m, **okw)
    assert max_err(o, torch.nan_to_num(o_sdpa)) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("form", ["keypad", "full", "per_head", "two_d"])
def test_mask_forward_forms(dtype, d, form):
    _fwd_case(2, 150, 150, 8, 2, d, dtype, form, causal=True, seed=d)
    _fwd_case(1, 70, 200, 4, 4, d, dtype, form, causal=False, seed=d + 1)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_mask_forward_with_window_alibi_rope_and_bottom_right(dtype):
    _fwd_case(2, 130, 130, 8, 2, 128, dtype, "full", causal=True, window=33, seed=5)
    _fwd_case(2, 96, 96, 16, 1, 256 if dtype != torch.float32 else 128, dtype, "keypad", causal=True, alibi=True,
              seed=6)
    _fwd_case(1, 60, 180, 8, 2, 128, dtype, "per_head", causal=True, rope=True, seed=7)  # Lq < Lk
    _fwd_case(2, 64, 64, 4, 1, 64, dtype, "two_d", causal=False, alibi=True, seed=8)


def test_mask_all_true_equals_no_mask_bitwise():
    """A mask of all ones takes the kernel's skip path on every tile and must
    give the unmasked kernel's bits exactly."""
    b, t, hq, hkv, d = 2, 333, 8, 2, 128
    q, k, v = (_rand((b, t, h, d), torch.bfloat16, s).to(DEV) for h, s in ((hq, 1), (hkv, 2), (hkv, 3)))
    m = torch.ones(b, 1, 1, t, dtype=torch.bool, device=DEV)
    o0, l0 = ops.attention_prefill(q, k, v, causal=True, return_lse=True)
    o1, l1 = ops.attention_prefill(q, k, v, causal=True, attn_mask=m, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(o0, o1) and torch.equal(l0, l1)


def _bwd_case(b, tq, tk, hq, hkv, d, dtype, form, *, causal, window=-1, alibi=False, seed=0):
    q = _rand((b, tq, hq, d), dtype, seed)
    k = _rand((b, tk, hkv, d), dtype, seed + 1)
    v = _rand((b, tk, hkv, d), dtype, seed + 2)
    d_o = _rand((b, tq, hq, d), dtype, seed + 3, std=1.0)
    m = _mask(form, b, hq, tq, tk, seed + 4, hidden_row=tq // 2)
    kw, okw = {}, {}
    if alibi:
        slopes = torch.tensor(wl.alibi_slopes(hq), dtype=torch.float32)
        kw["alibi_slopes"], okw["alibi_slopes"] = slopes.to(DEV), slopes
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    pm = ops.pack_mask(m.to(DEV), b, hq, tq, tk, DEV)
    o, lse = ops.attention_prefill(qg, kg, vg, causal=causal, window_left=window, attn_mask=pm, return_lse=True, **kw)
    dq, dk, dv = ops.attention_prefill_bwd(qg, kg, vg, o, lse, d_o.to(DEV), causal=causal, window_left=window,
                                           attn_mask=pm, **kw)
    torch.cuda.synchronize()
    refs = ref.attention_grads(q.float(), k.float(), v.float(), d_o.float(), causal=causal,
                               window_size=(window, -1), base_attn_mask=m, **okw)
    _check((dq, dk, dv), refs, dtype, f"mask {form} b{b} tq{tq} tk{tk} h{hq}/{hkv} d{d} {dtype} causal={causal}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("form", ["keypad", "full", "per_head"])
def test_mask_backward_forms(dtype, d, form):
    _bwd_case(2, 100, 100, 8, 2, d, dtype, form, causal=True, seed=d)
    _bwd_case(1, 40, 130, 4, 1, d, dtype, form, causal=False, seed=d + 1)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_mask_backward_window_alibi_and_split_walk(dtype):
    _bwd_case(2, 96, 96, 4, 2, 128, dtype, "full", causal=True, window=20, seed=31)
    # head_dim 256 MQA over several key blocks: the dk/dv walk is split over
    # workgroups whose partials are reduced
    _bwd_case(2, 100, 300, 16, 1, 256, dtype, "two_d", causal=True, alibi=True, seed=32)


def test_flashattention_base_mask_with_autograd_and_doc_ids():
    """The drop-in dispatcher: base_attn_mask alone and together with doc_ids
    (their conjunction, on the dense kernel), forward and backward, against
    the oracle's SDPA path with the same masks."""
    b, t, hq, hkv, d = 2, 120, 8, 2, 128
    q = _rand((b, t, hq, d), torch.bfloat16, 41)
    k = _rand((b, t, hkv, d), torch.bfloat16, 42)
    v = _rand((b, t, hkv, d), torch.bfloat16, 43)
    d_o = _rand((b, t, hq, d), torch.bfloat16, 44, std=1.0)
    m = _mask("keypad", b, hq, t, t, 45)
    doc = torch.cat([torch.zeros(b, 50, dtype=torch.long), torch.ones(b, 40, dtype=torch.long),
                     torch.full((b, 30), 2, dtype=torch.long)], dim=1)
    fa = FlashAttention()
    for docs in (None, doc):
        qg, kg, vg = (x.to(DEV).requires_grad_(True) for x in (q, k, v))
        o = fa(qg, kg, vg, causal=True, base_attn_mask=m.to(DEV), doc_ids=None if docs is None else docs.to(DEV))
        o.backward(d_o.to(DEV))
        torch.cuda.synchronize()
        o_ref = ref.attention(q.float(), k.float(), v.float(), causal=True, base_attn_mask=m, doc_ids=docs)
        assert max_err(o, o_ref) <= TOL[torch.bfloat16]
        refs = ref.attention_grads(q.float(), k.float(), v.float(), d_o.float(), causal=True, base_attn_mask=m,
                                   doc_ids=docs)
        _check((qg.grad, kg.grad, vg.grad), refs, torch.bfloat16, f"FlashAttention docs={docs is not None}")


def test_flashattention_right_window_is_ignored_like_the_reference():
    """mint/nn/flashattn.py:251-253 reads window_size[0] only: (W, R) gives
    the (W, -1) result."""
    b, t, hq, hkv, d = 1, 90, 4, 2, 64
    q, k, v = (_rand((b, t, h, d), torch.bfloat16, s).to(DEV) for h, s in ((hq, 51), (hkv, 52), (hkv, 53)))
    fa = FlashAttention()
    o_lr = fa(q, k, v, causal=True, window_size=(17, 5))
    o_l = fa(q, k, v, causal=True, window_size=(17, -1))
    torch.cuda.synchronize()
    assert torch.equal(o_lr, o_l)
    o_ref = ref.attention(q.cpu().float(), k.cpu().float(), v.cpu().float(), causal=True, window_size=(17, 5))
    assert max_err(o_lr, o_ref) <= TOL[torch.bfloat16]
