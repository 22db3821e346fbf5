"""CPU checks of the C-ABI boundary: the library loads, exports every symbol
include/goda_attn.h declares, its structs match the ctypes mirror, and host
validation rejects bad arguments (no GPU work is launched here)."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from goda_amd import _lib, ops

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))


def _declared_functions() -> set[str]:
    names = set()
    for h in HEADERS:
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(goda_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


@pytest.fixture(scope="module")
def lib():
    if not _lib.lib_path().exists():
        pytest.fail(f"{_lib.lib_path()} is missing: run `python -c 'import __graft_entry__ as g; g.build()'`")
    return _lib.load()


def test_header_declares_the_entry_points():
    names = _declared_functions()
    for n in ("goda_attn_prefill_fwd", "goda_attn_decode", "goda_attn_kv_append", "goda_attn_last_error"):
        assert n in names
    assert names == set(_lib.SYMBOLS), f"ctypes binding and header differ: {names ^ set(_lib.SYMBOLS)}"


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.lib_path())], capture_output=True, text=True)
    exported = {ln.split()[-1] for ln in out.stdout.splitlines() if ln.strip()}
    missing = _declared_functions() - exported
    assert not missing, f"not exported: {missing}"


def test_abi_version_and_struct_sizes(lib):
    assert lib.goda_attn_abi_version() == _lib.ABI_VERSION
    assert lib.goda_attn_sizeof_prefill_args() == ctypes.sizeof(_lib.PrefillArgs)
    assert lib.goda_attn_sizeof_decode_args() == ctypes.sizeof(_lib.DecodeArgs)
    assert lib.goda_attn_sizeof_kv_append_args() == ctypes.sizeof(_lib.KvAppendArgs)


def _prefill_args(**over):
    a = _lib.PrefillArgs()
    a.dtype = _lib.DTYPE_BF16
    a.batch, a.heads_q, a.heads_kv, a.head_dim = 2, 8, 2, 128
    a.seqlen_q = a.seqlen_k = 64
    a.causal, a.window_left, a.softmax_scale = 1, -1, 1.0 / 128**0.5
    for k, v in over.items():
        setattr(a, k, v)
    return a


def test_workspace_size_positive_for_mfma_path(lib):
    a = _prefill_args()
    need = lib.goda_attn_prefill_workspace_size(ctypes.byref(a))
    # K' and V^T tiles: 2 tensors x B x tiles x Hkv x 64 x D x 2 bytes
    assert need == 2 * 2 * 1 * 2 * 64 * 128 * 2
    # fp32 at D=128 runs the same kernel with 32-key tiles of 4-byte elements
    a32 = _prefill_args(dtype=_lib.DTYPE_F32)
    assert lib.goda_attn_prefill_workspace_size(ctypes.byref(a32)) == 2 * 2 * 2 * 2 * 32 * 128 * 4
    # fp32 at D=256 takes the generic kernel, which needs no workspace
    a32w = _prefill_args(dtype=_lib.DTYPE_F32, head_dim=256)
    assert lib.goda_attn_prefill_workspace_size(ctypes.byref(a32w)) == 0


@pytest.mark.parametrize(
    "over,code,needle",
    [
        ({"heads_q": 6, "heads_kv": 4}, _lib.ERR_INVALID_ARG, "not a multiple"),
        ({"head_dim": 96}, _lib.ERR_UNSUPPORTED, "head_dim"),
        ({"dtype": 7}, _lib.ERR_INVALID_ARG, "dtype"),
        ({"batch": -1}, _lib.ERR_INVALID_ARG, "negative"),
        ({"softmax_scale": 0.0}, _lib.ERR_INVALID_ARG, "softmax_scale"),
        ({"rope_q": 1}, _lib.ERR_INVALID_ARG, "RoPE"),
    ],
)
def test_prefill_rejects_bad_arguments(lib, over, code, needle):
    a = _prefill_args(**over)
    st = lib.goda_attn_prefill_workspace_size(ctypes.byref(a))
    assert st == code
    assert needle in lib.goda_attn_last_error().decode()
    # the launch entry point validates the same way before touching the GPU
    assert lib.goda_attn_prefill_fwd(ctypes.byref(a), None) == code


def test_prefill_rejects_null_tensors(lib):
    a = _prefill_args()
    assert lib.goda_attn_prefill_fwd(ctypes.byref(a), None) == _lib.ERR_INVALID_ARG
    assert "NULL" in lib.goda_attn_last_error().decode()


def test_decode_and_append_reject_bad_arguments(lib):
    d = _lib.DecodeArgs()
    d.dtype, d.batch, d.heads_q, d.heads_kv, d.head_dim = _lib.DTYPE_BF16, 1, 6, 4, 128
    d.max_seqlen, d.softmax_scale = 64, 0.1
    assert lib.goda_attn_decode(ctypes.byref(d), None) == _lib.ERR_INVALID_ARG
    d.heads_q, d.split_size = 8, 100
    assert lib.goda_attn_decode(ctypes.byref(d), None) == _lib.ERR_INVALID_ARG
    assert "split_size" in lib.goda_attn_last_error().decode()
    k = _lib.KvAppendArgs()
    k.dtype, k.batch, k.heads_kv, k.head_dim, k.seqlen_new = _lib.DTYPE_BF16, 1, 2, 127, 1
    assert lib.goda_attn_kv_append(ctypes.byref(k), None) == _lib.ERR_INVALID_ARG


def _decode_args(**over):
    d = _lib.DecodeArgs()
    d.dtype, d.batch, d.heads_q, d.heads_kv, d.head_dim = _lib.DTYPE_BF16, 1, 8, 8, 128
    d.max_seqlen, d.softmax_scale = 64, 0.1
    for k, v in over.items():
        setattr(d, k, v)
    return d


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("hq,hkv", [(8, 8), (32, 8), (64, 8), (128, 8), (16, 1), (8, 1)])
def test_decode_noalloc_scratch_holds_every_balanced_split(lib, d, hq, hkv):
    """With split_size 0 (the balanced default) the split-K partials of any
    batch and cache length fit the fixed scratch array of
    goda_attn_decode_noalloc."""
    a = _decode_args(batch=4096, heads_q=hq, heads_kv=hkv, head_dim=d, max_seqlen=1 << 20, split_size=0)
    need = lib.goda_attn_decode_workspace_size(ctypes.byref(a))
    assert 0 < need <= _lib.DECODE_NOALLOC_SCRATCH_BYTES


def test_decode_noalloc_rejects_partials_beyond_the_scratch_array(lib):
    """A fixed small split over a long cache needs more partial slots than
    the scratch array holds: the call fails before any GPU work (the tensor
    pointers here are never dereferenced)."""
    a = _decode_args(heads_q=128, heads_kv=8, max_seqlen=65536, split_size=64)
    a.q = a.k_cache = a.v_cache = a.o = a.cache_seqlens = 256
    need = lib.goda_attn_decode_workspace_size(ctypes.byref(a))
    assert need > _lib.DECODE_NOALLOC_SCRATCH_BYTES
    assert lib.goda_attn_decode_noalloc(ctypes.byref(a), None) == _lib.ERR_WORKSPACE
    assert "scratch" in lib.goda_attn_last_error().decode()
    # argument checks come first, as in goda_attn_decode
    a.split_size = 100
    assert lib.goda_attn_decode_noalloc(ctypes.byref(a), None) == _lib.ERR_INVALID_ARG


def test_empty_batch_is_a_no_op(lib):
    a = _prefill_args(batch=0)
    assert lib.goda_attn_prefill_fwd(ctypes.byref(a), None) == _lib.OK


def test_ops_refuse_cpu_tensors():
    q = torch.zeros(1, 4, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensor"):
        ops.attention_prefill(q, q, q, causal=True)
    with pytest.raises(ValueError, match="GPU tensor"):
        ops.attention_decode(q[:, 0], q, q, torch.zeros(1, dtype=torch.int32))


def test_missing_library_is_a_loud_error(tmp_path):
    """With no built library the package refuses to run (there is no CPU or
    SDPA fallback): loading raises and names the build command."""
    code = (
        "import goda_amd._lib as L\n"
        "try:\n"
        "    L.load()\n"
        "except RuntimeError as e:\n"
        "    print('raised:', e)\n"
        "else:\n"
        "    print('loaded')\n"
    )
    env = dict(os.environ, GODA_ATTN_LIB=str(tmp_path / "nope" / "libgoda_attn.so"))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=300, cwd=str(ROOT))
    assert "raised:" in out.stdout and "no non-HIP fallback" in out.stdout, out.stdout + out.stderr
