"""goda_attn_decode_noalloc (the decode entry point that allocates nothing)
against goda_attn_decode, both called through the C-ABI on the same inputs.

The two run the same kernels over the same split, so their outputs must be
bit-identical; the oracle check on top keeps the pair honest. Two calls in a
row, the second smaller, exercise the shared device-resident scratch array
(which keeps the previous call's contents)."""

from __future__ import annotations

import ctypes

import pytest
import torch

from goda_amd import _lib, ops
from oracle import attention as ref
from tests.helpers import TOL, max_err

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _case(b, hq, hkv, d, lmax, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(1, lmax + 1, (b,), generator=g, dtype=torch.int32)
    lens[0] = lmax
    q = (torch.randn(b, hq, d, generator=g) * 0.5).to(dtype)
    kc = (torch.randn(b, lmax, hkv, d, generator=g) * 0.5).to(dtype)
    vc = (torch.randn(b, lmax, hkv, d, generator=g) * 0.5).to(dtype)
    return q, kc, vc, lens


def _run_pair(q, kc, vc, lens):
    qg, kg, vg, lg = q.to(DEV), kc.to(DEV), vc.to(DEV), lens.to(DEV)
    o_ref_gpu, lse_ref_gpu = ops.attention_decode(qg, kg, vg, lg, return_lse=True)
    plan = ops.plan_decode(qg, kg, vg, lg, return_lse=True, noalloc=True)
    assert plan.args.workspace is None and plan.args.workspace_bytes == 0
    # Straight through the C-ABI symbol (the plan only built the struct).
    lib = _lib.load()
    st = lib.goda_attn_decode_noalloc(ctypes.byref(plan.args), torch.cuda.current_stream().cuda_stream)
    _lib.check(st)
    torch.cuda.synchronize()
    o, lse = plan.result
    assert torch.equal(o, o_ref_gpu), "noalloc output differs from goda_attn_decode"
    assert torch.equal(lse, lse_ref_gpu), "noalloc lse differs from goda_attn_decode"
    o_cpu, _ = ref.decode_attention(q.float(), kc.float(), vc.float(), lens)
    assert max_err(o, o_cpu) <= TOL[q.dtype]
    return o


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_decode_noalloc_matches_decode_two_calls(dtype):
    # First call: 8 KV heads, group 4 (D 128); second, smaller: MQA at D 256
    # (another kernel instance, fewer and shorter sequences).
    q, kc, vc, lens = _case(24, 32, 8, 128, 3000, dtype, seed=11)
    _run_pair(q, kc, vc, lens)
    q, kc, vc, lens = _case(5, 8, 1, 256, 700, dtype, seed=12)
    _run_pair(q, kc, vc, lens)


def test_decode_noalloc_same_shape_twice_then_smaller():
    # Same instance back to back, then a smaller batch of the same shape: the
    # second and third calls run over partials the previous call left behind.
    q, kc, vc, lens = _case(32, 16, 4, 128, 2048, torch.bfloat16, seed=21)
    _run_pair(q, kc, vc, lens)
    _run_pair(q, kc, vc, lens)
    _run_pair(q[:3].clone(), kc[:3].clone(), vc[:3].clone(), lens[:3].clone())
