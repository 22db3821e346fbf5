"""goda_amd — MI355X (gfx950) attention hot path for goda.

The HIP kernels live in `goda_amd/csrc` and are reached through the C-ABI in
`include/goda_attn.h` (ctypes binding in `goda_amd._lib`). `goda_amd.ops` is
the torch-facing API; `goda_amd.kernels_` and `goda_amd.mint` mirror goda's
own `kernels_` and `mint.nn` / `mint.kvcache` interfaces.
"""

from . import ops
from .ops import attention_decode, attention_prefill, kv_append

__all__ = ["ops", "attention_prefill", "attention_decode", "kv_append"]
