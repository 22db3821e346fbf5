"""ctypes binding of libgoda_attn.so (the C-ABI declared in include/goda_attn.h).

The structures below mirror the C structs field by field; `load()` checks
their sizes against the library's own `sizeof` exports so a stale build or an
edited header fails at load time instead of corrupting arguments.

There is no fallback: if the library is missing, `load()` raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

_LIB_ENV = "GODA_ATTN_LIB"
_DEFAULT = Path(__file__).resolve().parent / "lib" / "libgoda_attn.so"

ABI_VERSION = 5

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2

OK = 0
ERR_INVALID_ARG = -1
ERR_UNSUPPORTED = -2
ERR_WORKSPACE = -3
ERR_HIP = -4

# Size of the device-resident scratch array of goda_attn_decode_noalloc.
DECODE_NOALLOC_SCRATCH_BYTES = 36 << 20

_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_vp = ctypes.c_void_p


class PrefillArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", _i32),
        ("batch", _i32),
        ("heads_q", _i32),
        ("heads_kv", _i32),
        ("head_dim", _i32),
        ("seqlen_q", _i32),
        ("seqlen_k", _i32),
        ("causal", _i32),
        ("window_left", _i32),
        ("softmax_scale", _f32),
        ("q", _vp),
        ("k", _vp),
        ("v", _vp),
        ("o", _vp),
        ("q_stride_b", _i64),
        ("q_stride_t", _i64),
        ("q_stride_h", _i64),
        ("k_stride_b", _i64),
        ("k_stride_t", _i64),
        ("k_stride_h", _i64),
        ("v_stride_b", _i64),
        ("v_stride_t", _i64),
        ("v_stride_h", _i64),
        ("o_stride_b", _i64),
        ("o_stride_t", _i64),
        ("o_stride_h", _i64),
        ("lse", _vp),
        ("lse_stride_b", _i64),
        ("lse_stride_h", _i64),
        ("cu_seqlens_q", _vp),
        ("cu_seqlens_k", _vp),
        ("seqused_k", _vp),
        ("alibi_slopes", _vp),
        ("rope_cos", _vp),
        ("rope_sin", _vp),
        ("rope_len", _i32),
        ("rope_q", _i32),
        ("rope_k", _i32),
        ("rope_q_offset", _i32),
        ("rope_k_offset", _i32),
        ("norm_eps", _f32),
        ("rope_pos_abs", _i32),
        ("q_norm_weight", _vp),
        ("k_norm_weight", _vp),
        ("mask_bits", _vp),
        ("mask_stride_b", _i64),
        ("mask_stride_h", _i64),
        ("mask_stride_q", _i64),
        ("workspace", _vp),
        ("workspace_bytes", _i64),
        ("timing_begin", _vp),
        ("timing_end", _vp),
    ]


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", _i32),
        ("batch", _i32),
        ("heads_q", _i32),
        ("heads_kv", _i32),
        ("head_dim", _i32),
        ("max_seqlen", _i32),
        ("window_left", _i32),
        ("split_size", _i32),
        ("softmax_scale", _f32),
        ("rope_pos_abs", _i32),
        ("q", _vp),
        ("q_stride_b", _i64),
        ("q_stride_h", _i64),
        ("k_cache", _vp),
        ("k_stride_b", _i64),
        ("k_stride_t", _i64),
        ("k_stride_h", _i64),
        ("v_cache", _vp),
        ("v_stride_b", _i64),
        ("v_stride_t", _i64),
        ("v_stride_h", _i64),
        ("cache_seqlens", _vp),
        ("o", _vp),
        ("o_stride_b", _i64),
        ("o_stride_h", _i64),
        ("lse", _vp),
        ("lse_stride_b", _i64),
        ("alibi_slopes", _vp),
        ("rope_cos", _vp),
        ("rope_sin", _vp),
        ("rope_len", _i32),
        ("rope_q", _i32),
        ("rope_q_offset", _i32),
        ("norm_eps", _f32),
        ("q_norm_weight", _vp),
        ("workspace", _vp),
        ("workspace_bytes", _i64),
        ("timing_begin", _vp),
        ("timing_end", _vp),
    ]


class KvAppendArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", _i32),
        ("batch", _i32),
        ("heads_kv", _i32),
        ("head_dim", _i32),
        ("max_seqlen", _i32),
        ("seqlen_new", _i32),
        ("k_new", _vp),
        ("kn_stride_b", _i64),
        ("kn_stride_t", _i64),
        ("kn_stride_h", _i64),
        ("v_new", _vp),
        ("vn_stride_b", _i64),
        ("vn_stride_t", _i64),
        ("vn_stride_h", _i64),
        ("k_cache", _vp),
        ("k_stride_b", _i64),
        ("k_stride_t", _i64),
        ("k_stride_h", _i64),
        ("v_cache", _vp),
        ("v_stride_b", _i64),
        ("v_stride_t", _i64),
        ("v_stride_h", _i64),
        ("cache_seqlens", _vp),
        ("rope_cos", _vp),
        ("rope_sin", _vp),
        ("rope_len", _i32),
        ("rope_k", _i32),
        ("rope_k_offset", _i32),
        ("norm_eps", _f32),
        ("k_norm_weight", _vp),
        ("rope_pos_abs", _i32),
        ("reserved0", _i32),
        ("status", _vp),
    ]


class PrefillGrads(ctypes.Structure):
    _fields_ = [
        ("d_o", _vp),
        ("do_stride_b", _i64),
        ("do_stride_t", _i64),
        ("do_stride_h", _i64),
        ("dq", _vp),
        ("dq_stride_b", _i64),
        ("dq_stride_t", _i64),
        ("dq_stride_h", _i64),
        ("dk", _vp),
        ("dk_stride_b", _i64),
        ("dk_stride_t", _i64),
        ("dk_stride_h", _i64),
        ("dv", _vp),
        ("dv_stride_b", _i64),
        ("dv_stride_t", _i64),
        ("dv_stride_h", _i64),
        ("dq_norm_weight", _vp),
        ("dk_norm_weight", _vp),
        ("workspace", _vp),
        ("workspace_bytes", _i64),
        ("timing_begin", _vp),
        ("timing_end", _vp),
    ]


# Every symbol the header declares, with its ctypes signature.
SYMBOLS = {
    "goda_attn_abi_version": (_i32, []),
    "goda_attn_sizeof_prefill_args": (_i64, []),
    "goda_attn_sizeof_decode_args": (_i64, []),
    "goda_attn_sizeof_kv_append_args": (_i64, []),
    "goda_attn_sizeof_prefill_grads": (_i64, []),
    "goda_attn_last_error": (ctypes.c_char_p, []),
    "goda_attn_prefill_workspace_size": (_i64, [ctypes.POINTER(PrefillArgs)]),
    "goda_attn_prefill_fwd": (_i32, [ctypes.POINTER(PrefillArgs), _vp]),
    "goda_attn_prefill_bwd_workspace_size": (_i64, [ctypes.POINTER(PrefillArgs)]),
    "goda_attn_prefill_bwd": (_i32, [ctypes.POINTER(PrefillArgs), ctypes.POINTER(PrefillGrads), _vp]),
    "goda_attn_decode_workspace_size": (_i64, [ctypes.POINTER(DecodeArgs)]),
    "goda_attn_decode": (_i32, [ctypes.POINTER(DecodeArgs), _vp]),
    "goda_attn_decode_noalloc": (_i32, [ctypes.POINTER(DecodeArgs), _vp]),
    "goda_attn_kv_append": (_i32, [ctypes.POINTER(KvAppendArgs), _vp]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib_path() -> Path:
    env = os.environ.get(_LIB_ENV)
    return Path(env) if env else _DEFAULT


def load() -> ctypes.CDLL:
    """Load the library once, bind all symbols and check the struct mirrors."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        # torch bundles its own HIP runtime with the same SONAME
        # (libamdhip64.so.7); loading torch first makes the library bind to
        # that one copy, so streams and events from torch are valid here.
        try:
            import torch  # noqa: F401
        except ImportError:  # pragma: no cover - torch is a hard dependency
            pass
        path = lib_path()
        if not path.exists():
            raise RuntimeError(
                f"goda_amd: {path} is missing; build it with `python -m goda_amd.build` "
                "(there is no non-HIP fallback)"
            )
        lib = ctypes.CDLL(str(path))
        for name, (res, args) in SYMBOLS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.goda_attn_abi_version() != ABI_VERSION:
            raise RuntimeError(
                f"goda_amd: ABI version {lib.goda_attn_abi_version()} != binding {ABI_VERSION}"
            )
        for struct, fn in (
            (PrefillArgs, lib.goda_attn_sizeof_prefill_args),
            (DecodeArgs, lib.goda_attn_sizeof_decode_args),
            (KvAppendArgs, lib.goda_attn_sizeof_kv_append_args),
            (PrefillGrads, lib.goda_attn_sizeof_prefill_grads),
        ):
            if ctypes.sizeof(struct) != fn():
                raise RuntimeError(
                    f"goda_amd: ctypes {struct.__name__} is {ctypes.sizeof(struct)} bytes, "
                    f"library says {fn()}"
                )
        _lib = lib
        return lib


class GodaError(RuntimeError):
    """A C-ABI call returned a negative status."""

    def __init__(self, status: int, message: str) -> None:
        super().__init__(f"goda_attn status {status}: {message}")
        self.status = status


def check(status: int) -> None:
    if status != OK:
        msg = load().goda_attn_last_error().decode(errors="replace")
        if status in (ERR_INVALID_ARG, ERR_WORKSPACE):
            raise ValueError(f"goda_attn status {status}: {msg}")
        raise GodaError(status, msg)
