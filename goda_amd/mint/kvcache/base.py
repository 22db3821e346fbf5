"""Drop-in for goda's static KV cache (mint/kvcache/base.py:4-65), backed by
the HIP append kernel.

Same constructor, same `update/get/get_cache_tensors/reset/clear`, same
tensor shape `[max_batch_size, max_seq_len, n_kv_heads, head_dim]` plus int32
`cache_seqlens [max_batch_size]`. The storage underneath is head-major
`[max_batch_size, n_kv_heads, max_seq_len, head_dim]` and the cache tensors
are strided views of it in goda's shape: a decode step then streams each
(sequence, KV head)'s keys contiguously (cfg4 decode kernel: 5.99 TB/s vs
5.32 TB/s with the keys of all heads interleaved). Every kernel here takes
strides, and slicing / element assignment behave as on the reference's
tensors; code that needs a contiguous tensor calls `.contiguous()`.
One addition: `append(k, v)` writes every sequence at its OWN current length,
read on the device (no host sync), which is what ragged decoding needs;
`update(k, v, start_pos)` keeps the reference's batch-uniform semantics.
"""

from __future__ import annotations

import torch

from ... import ops


class KVCache:
    def __init__(
        self,
        max_batch_size: int = 1,
        max_seq_len: int = 2048,
        n_kv_heads: int = 4,
        head_dim: int = 128,
        dtype: torch.dtype = torch.float32,
        device: str = "cpu",
    ) -> None:
        self.max_batch_size = max_batch_size
        self.max_seq_len = max_seq_len
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = device
        store = (max_batch_size, n_kv_heads, max_seq_len, head_dim)
        self.k_cache = torch.zeros(store, dtype=dtype, device=device).transpose(1, 2)
        self.v_cache = torch.zeros(store, dtype=dtype, device=device).transpose(1, 2)
        self.cache_seqlens = torch.zeros(max_batch_size, dtype=torch.int32, device=device)

    def append(
        self,
        k: torch.Tensor,
        v: torch.Tensor,
        *,
        rope_cos: torch.Tensor | None = None,
        rope_sin: torch.Tensor | None = None,
        k_norm_weight: torch.Tensor | None = None,
        norm_eps: float = 1e-6,
    ) -> None:
        """Write k/v [B, T, Hkv, D] at rows cache_seqlens[b] .. +T-1 of each
        sequence b and advance cache_seqlens[:B] by T, all on the device. With
        RoPE tables, k is rotated at its absolute cache position on the way in
        (goda caches post-RoPE keys, mint/nn/attn.py:60); with k_norm_weight it
        is first RMS-normalised like goda's k_norm (mint/nn/attn.py:58)."""
        ops.kv_append(
            k,
            v,
            self.k_cache,
            self.v_cache,
            self.cache_seqlens,
            rope_cos=rope_cos,
            rope_sin=rope_sin,
            rope_k=rope_cos is not None,
            k_norm_weight=k_norm_weight,
            norm_eps=norm_eps,
        )

    def update(self, k: torch.Tensor, v: torch.Tensor, start_pos: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
        """mint/kvcache/base.py:35-50: rows [start_pos, start_pos+T) of every
        sequence, cache_seqlens[:B] = start_pos + T, views up to that row."""
        batch_size, seq_len = k.shape[0], k.shape[1]
        if start_pos < 0 or start_pos + seq_len > self.max_seq_len:
            raise ValueError(f"KVCache.update: rows [{start_pos}, {start_pos + seq_len}) exceed max_seq_len {self.max_seq_len}")
        self.cache_seqlens[:batch_size].fill_(start_pos)
        self.append(k, v)
        end_pos = start_pos + seq_len
        return self.k_cache[:batch_size, :end_pos], self.v_cache[:batch_size, :end_pos]

    def get(self) -> tuple[torch.Tensor, torch.Tensor]:
        """mint/kvcache/base.py:52-54 (reads the length of sequence 0 on the host)."""
        pos = int(self.cache_seqlens[0].item())
        return self.k_cache[:, :pos], self.v_cache[:, :pos]

    def get_cache_tensors(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        return self.k_cache, self.v_cache, self.cache_seqlens

    def reset(self) -> None:
        self.cache_seqlens.zero_()

    def clear(self) -> None:
        self.k_cache.zero_()
        self.v_cache.zero_()
        self.cache_seqlens.zero_()
