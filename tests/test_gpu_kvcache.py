"""The KV-cache path on the GPU: goda's attention layer driven through a
generate loop (mint/nn/models.py:102-150), start_pos semantics, loud cache
overflow (mint/kvcache/base.py:40-43) and chunked prefill over a cfg4-sized
cache, each against the CPU oracle."""

from __future__ import annotations

import ctypes

import pytest
import torch

from goda_amd import _lib, ops
from goda_amd import workloads as wl
from goda_amd.mint.kvcache import KVCache
from goda_amd.mint.nn import FlashAttention, GroupedQueryAttention, RoPE
from oracle import attention as ref
from tests.helpers import TOL, max_err

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rand(shape, dtype, seed, std=0.5):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).to(dtype)


class _CpuLayer:
    """goda's GroupedQueryAttention.forward with a KVCache
    (mint/nn/attn.py:39-77, mint/nn/flashattn.py:174-219), restated on the
    CPU in fp32 from the oracle's pieces: projections, RMSNorm
    (mint/nn/norm.py:17-27), RoPE at start_pos .. start_pos+T-1
    (mint/nn/pos.py:100-112), KVCache.update at the cache's current length
    (mint/nn/flashattn.py:202), bottom-right causal attention over the
    visible cache, output projection."""

    def __init__(self, layer: GroupedQueryAttention, batch: int, lmax: int):
        f = lambda t: t.detach().to("cpu", torch.float32)  # noqa: E731
        self.wq, self.wk, self.wv, self.wo = f(layer.wq.weight), f(layer.wk.weight), f(layer.wv.weight), f(layer.wo.weight)
        self.qs, self.ks = f(layer.q_norm.scale), f(layer.k_norm.scale)
        self.eps = layer.q_norm.eps
        self.hq, self.hkv, self.d = layer.n_heads, layer.n_kv_heads, layer.head_dim
        self.cos, self.sin = f(layer.pos_embeddings.cos), f(layer.pos_embeddings.sin)
        self.cache = ref.KVCacheOracle(batch, lmax, self.hkv, self.d)

    def __call__(self, x: torch.Tensor, start_pos: int) -> torch.Tensor:
        x = x.to("cpu", torch.float32)
        b, t, _ = x.shape
        q = (x @ self.wq.T).view(b, t, self.hq, self.d)
        k = (x @ self.wk.T).view(b, t, self.hkv, self.d)
        v = (x @ self.wv.T).view(b, t, self.hkv, self.d)
        q, k = ref.rms_norm(q, self.qs, self.eps), ref.rms_norm(k, self.ks, self.eps)
        pos = torch.arange(start_pos, start_pos + t)
        q, k = ref.apply_rope(q, self.cos, self.sin, pos), ref.apply_rope(k, self.cos, self.sin, pos)
        self.cache.append(k, v)
        end = int(self.cache.seqlens[0])
        o = ref.attention(q, self.cache.k[:b, :end], self.cache.v[:b, :end], causal=True)
        return o.reshape(b, t, -1) @ self.wo.T


def _layer(dtype, hq=8, hkv=2, d=128, embed=256, lmax=96, seed=0):
    torch.manual_seed(seed)
    rope = RoPE(seq_len=lmax, head_dim=d, rope_base_theta=10000)
    layer = GroupedQueryAttention(hq, hkv, d, embed, rope, dtype).to(DEV)
    with torch.no_grad():
        layer.q_norm.scale.copy_(torch.randn(d) * 0.1)
        layer.k_norm.scale.copy_(torch.randn(d) * 0.1)
    return layer


def _rel_err(a, b):
    a, b = a.to("cpu", torch.float32), b.to("cpu", torch.float32)
    return ((a - b).abs().max() / max(1.0, b.abs().max().item())).item()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_layer_generate_loop_prompt_then_tokens(dtype):
    """Prompt prefill through the cache (start_pos 0), then one token per step
    at start_pos = cache length: fused QK-RMSNorm + RoPE, the KV append, the
    chunked prefill and the split-K decode, against the CPU layer."""
    b, t0, steps, lmax = 2, 37, 6, 96
    layer = _layer(dtype, lmax=lmax)
    cpu = _CpuLayer(layer, b, lmax)
    cache = KVCache(max_batch_size=b, max_seq_len=lmax, n_kv_heads=2, head_dim=128, dtype=dtype, device=DEV)
    x = _rand((b, t0 + steps, 256), dtype, 1, std=1.0)
    with torch.no_grad():
        for s, (lo, hi) in enumerate([(0, t0)] + [(t, t + 1) for t in range(t0, t0 + steps)]):
            out = layer(x[:, lo:hi].to(DEV), kv_cache=cache, start_pos=lo)
            torch.cuda.synchronize()
            e = _rel_err(out, cpu(x[:, lo:hi], lo))
            assert e <= TOL[dtype], f"step {s}: err {e}"
    assert cache.cache_seqlens.cpu().tolist() == [t0 + steps] * b
    cache.check()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_layer_generate_loop_as_gemma_generate_calls_it(dtype):
    """Gemma.generate with kv_caches (mint/nn/models.py:113-121) never
    prefills the prompt: its first step forwards only the last prompt token,
    at start_pos = prompt length - 1, into an empty cache, so start_pos and
    the cache length differ by that amount for the whole loop. RoPE follows
    start_pos, the cache rows follow the cache length, as in the reference."""
    b, prompt, steps, lmax = 3, 20, 5, 64
    layer = _layer(dtype, lmax=lmax, seed=3)
    cpu = _CpuLayer(layer, b, lmax)
    cache = KVCache(max_batch_size=b, max_seq_len=lmax, n_kv_heads=2, head_dim=128, dtype=dtype, device=DEV)
    x = _rand((b, prompt + steps, 256), dtype, 2, std=1.0)
    with torch.no_grad():
        for t in range(prompt, prompt + steps + 1):
            start_pos = t - 1
            out = layer(x[:, t - 1 : t].to(DEV), kv_cache=cache, start_pos=start_pos)
            torch.cuda.synchronize()
            e = _rel_err(out, cpu(x[:, t - 1 : t], start_pos))
            assert e <= TOL[dtype], f"start_pos {start_pos}: err {e}"
    assert cache.cache_seqlens.cpu().tolist() == [steps + 1] * b


def test_flashattention_kv_path_honours_start_pos():
    """FlashAttention with a cache and fused RoPE: an integer start_pos
    rotates q and the new k at start_pos + t whatever the cache length; with
    start_pos None they rotate at their cache positions."""
    b, hq, hkv, d, lmax = 2, 8, 2, 128, 64
    cos, sin = wl.rope_tables(lmax, d, 10000.0)
    rope = (cos.to(DEV), sin.to(DEV))
    q = _rand((b, 1, hq, d), torch.float32, 5)
    k = _rand((b, 1, hkv, d), torch.float32, 6)
    v = _rand((b, 1, hkv, d), torch.float32, 7)
    fa = FlashAttention()
    for start_pos, pos in ((11, 11), (None, 0)):
        cache = KVCache(max_batch_size=b, max_seq_len=lmax, n_kv_heads=hkv, head_dim=d, dtype=torch.float32, device=DEV)
        o = fa(q.to(DEV), k.to(DEV), v.to(DEV), causal=True, kv_cache=cache, rope=rope, start_pos=start_pos)
        torch.cuda.synchronize()
        p = torch.tensor([pos])
        kr = ref.apply_rope(k, cos, sin, p)
        assert max_err(cache.k_cache[:, :1], kr) <= 1e-5
        o_ref = ref.attention(ref.apply_rope(q, cos, sin, p), kr, v, causal=True)
        assert max_err(o, o_ref) <= TOL[torch.float32]


def test_kv_append_overflow_is_loud():
    """Past max_seq_len: with the lengths known on the host the append fails
    before any launch; with lengths the host cannot know, the kernel keeps
    the rows that fit, stops the length at max_seq_len and raises through the
    cache's status word."""
    b, lmax, hkv, d = 2, 16, 2, 64
    cache = KVCache(max_batch_size=b, max_seq_len=lmax, n_kv_heads=hkv, head_dim=d, dtype=torch.bfloat16, device=DEV)
    cache.set_seqlens([14, 3])
    k = _rand((b, 3, hkv, d), torch.bfloat16, 8).to(DEV)
    v = _rand((b, 3, hkv, d), torch.bfloat16, 9).to(DEV)
    with pytest.raises(ValueError, match="max_seq_len"):
        cache.append(k, v)
    assert cache.cache_seqlens.cpu().tolist() == [14, 3] and int(cache.status.item()) == 0
    _, _, lens = cache.get_cache_tensors()  # the host bound is now unknown
    cache.append(k, v)
    torch.cuda.synchronize()
    assert cache.cache_seqlens.cpu().tolist() == [lmax, 6]
    assert torch.equal(cache.v_cache[0, 14:16].cpu(), v[0, :2].cpu())  # the rows that fit
    assert torch.equal(cache.v_cache[1, 3:6].cpu(), v[1].cpu())
    with pytest.raises(RuntimeError, match="max_seq_len"):
        cache.check()
    with pytest.raises(RuntimeError, match="max_seq_len"):
        cache.get()
    cache.reset()
    cache.check()


def test_kv_append_and_decode_rope_at_a_given_position():
    """rope_pos_abs: the appended row t rotates at rope_k_offset + t and the
    decode query at rope_q_offset, whatever the cache lengths."""
    b, hq, hkv, d, lmax = 3, 8, 2, 128, 80
    cos, sin = wl.rope_tables(lmax, d, 10000.0)
    kc = torch.zeros(b, lmax, hkv, d, dtype=torch.float32, device=DEV)
    vc = torch.zeros_like(kc)
    lens = torch.tensor([0, 7, 30], dtype=torch.int32, device=DEV)
    kn = _rand((b, 2, hkv, d), torch.float32, 10)
    vn = _rand((b, 2, hkv, d), torch.float32, 11)
    ops.kv_append(kn.to(DEV), vn.to(DEV), kc, vc, lens, rope_cos=cos.to(DEV), rope_sin=sin.to(DEV), rope_k=True,
                  rope_k_offset=40, rope_pos_abs=True)
    torch.cuda.synchronize()
    want = ref.apply_rope(kn, cos, sin, torch.tensor([40, 41]))
    for i, p in enumerate([0, 7, 30]):
        assert max_err(kc[i, p : p + 2], want[i]) <= 1e-5
    q = _rand((b, hq, d), torch.float32, 12)
    o = ops.attention_decode(q.to(DEV), kc, vc, lens, rope_cos=cos.to(DEV), rope_sin=sin.to(DEV), rope_q=True,
                             rope_q_offset=41, rope_pos_abs=True)
    torch.cuda.synchronize()
    qr = ref.apply_rope(q[:, None], cos, sin, torch.tensor([41]))[:, 0]
    o_ref, _ = ref.decode_attention(qr, kc.cpu(), vc.cpu(), lens.cpu())
    assert max_err(o, o_ref) <= TOL[torch.float32]


def test_chunked_prefill_on_a_cfg4_sized_cache_is_bounded_by_the_visible_prefix():
    """A 128-token chunk appended to a cfg4-sized cache (B=64, Lmax=32768,
    Hkv=8, D=128, bf16, head-major): the launch covers the keys the cache
    holds (its host-side length bound), not Lmax, so its workspace is the
    visible prefix's K/V bytes; sampled rows match the oracle."""
    b, lmax, hq, hkv, d, l0, tq = 64, 32768, 32, 8, 128, 8192, 128
    cache = KVCache(max_batch_size=b, max_seq_len=lmax, n_kv_heads=hkv, head_dim=d, dtype=torch.bfloat16, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(13)
    for t in (cache.k_cache, cache.v_cache):  # fill the visible prefix only
        t[:, :l0] = (torch.randn(b, l0, hkv, d, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    cache.set_seqlens([l0] * b)
    cos, sin = wl.rope_tables(l0 + tq, d, 10000.0)
    q = _rand((b, tq, hq, d), torch.bfloat16, 14)
    k = _rand((b, tq, hkv, d), torch.bfloat16, 15)
    v = _rand((b, tq, hkv, d), torch.bfloat16, 16)
    o = FlashAttention()(q.to(DEV), k.to(DEV), v.to(DEV), causal=True, kv_cache=cache,
                         rope=(cos.to(DEV), sin.to(DEV)), start_pos=l0)
    torch.cuda.synchronize()
    assert cache.len_bound == l0 + tq and cache.cache_seqlens.cpu().tolist() == [l0 + tq] * b
    # the workspace of the launch FlashAttention made
    kc, vc, lens = cache.cache_tensors()
    plan = ops.plan_prefill(q.to(DEV), kc[:, : l0 + tq], vc[:, : l0 + tq], causal=True, seqused_k=lens[:b],
                            rope_cos=cos.to(DEV), rope_sin=sin.to(DEV), rope_q=True, rope_q_offset=l0,
                            rope_pos_abs=True)
    ws = _lib.load().goda_attn_prefill_workspace_size(ctypes.byref(plan.args))
    visible = b * (l0 + tq) * hkv * d * 2 * 2
    assert 0 < ws <= visible, (ws, visible)
    del plan
    # sampled rows of a few sequences against the oracle
    rows = torch.tensor([0, 1, 63, 64, 100, 127])
    for bi in (0, 31, 63):
        kk = cache.k_cache[bi : bi + 1, : l0 + tq].cpu().float()
        vv = cache.v_cache[bi : bi + 1, : l0 + tq].cpu().float()
        assert max_err(kk[:, l0:], ref.apply_rope(k[bi : bi + 1].float(), cos, sin, torch.arange(l0, l0 + tq))) <= 1e-2
        qr = ref.apply_rope(q[bi : bi + 1].float(), cos, sin, torch.arange(l0, l0 + tq))
        o_ref, _ = ref.attention_rows(qr, kk, vv, rows, causal=True)
        assert max_err(o[bi : bi + 1, rows], o_ref) <= TOL[torch.bfloat16]
