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

Additions:
  - `append(k, v)` writes every sequence at its OWN current length, read on
    the device (no host sync), which is what ragged decoding needs;
    `update(k, v, start_pos)` keeps the reference's batch-uniform semantics.
  - Overflow is loud, as the reference's slice assignment is
    (mint/kvcache/base.py:40-43): while the lengths are known on the host
    (they only changed through this class), an append past `max_seq_len`
    raises before anything is written; otherwise the kernel keeps the rows
    that fit, stops the length at `max_seq_len` and sets a device status word
    that `check()` (and `get()`) turn into an error.
  - `len_bound` is a host-side upper bound of every sequence's length (None
    once the caller had the raw tensors, `get_cache_tensors()`, and could
    have changed them); attention over the cache sizes its launch by it
    instead of by `max_seq_len`.
  - A head_dim the kernels do not instantiate is stored zero-padded to the
    next one that they do (goda_amd.headdim); `k_cache` / `v_cache` stay
    [B, L, H, head_dim] views, `cache_tensors()` gives the padded storage.
"""

from __future__ import annotations

import torch

from ... import headdim, ops


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
        self.head_dim_padded = headdim.padded(head_dim)
        store = (max_batch_size, n_kv_heads, max_seq_len, self.head_dim_padded)
        self._k_store = torch.zeros(store, dtype=dtype, device=device).transpose(1, 2)
        self._v_store = torch.zeros(store, dtype=dtype, device=device).transpose(1, 2)
        self.k_cache = self._k_store[..., :head_dim]
        self.v_cache = self._v_store[..., :head_dim]
        self.cache_seqlens = torch.zeros(max_batch_size, dtype=torch.int32, device=device)
        self.status = torch.zeros(1, dtype=torch.int32, device=device)
        self.len_bound: int | None = 0

    def append(
        self,
        k: torch.Tensor,
        v: torch.Tensor,
        *,
        rope_cos: torch.Tensor | None = None,
        rope_sin: torch.Tensor | None = None,
        start_pos: int | None = None,
        k_norm_weight: torch.Tensor | None = None,
        norm_eps: float = 1e-6,
    ) -> None:
        """Write k/v [B, T, Hkv, D] at rows cache_seqlens[b] .. +T-1 of each
        sequence b and advance cache_seqlens[:B] by T, all on the device. With
        RoPE tables, k is rotated on the way in (goda caches post-RoPE keys,
        mint/nn/attn.py:60): row t at `start_pos + t` when a start position is
        given (goda's RoPE(q, k, start_pos), mint/nn/pos.py:100-112), else at
        its own cache position. With k_norm_weight it is first RMS-normalised
        like goda's k_norm (mint/nn/attn.py:58)."""
        t = k.shape[1]
        if self.len_bound is not None:
            if self.len_bound + t > self.max_seq_len:
                raise ValueError(
                    f"KVCache.append: {t} rows after up to {self.len_bound} cached exceed max_seq_len {self.max_seq_len}"
                )
            self.len_bound += t
        if self.head_dim_padded != self.head_dim:
            # Norm and RoPE as torch ops at the kernel's positions, then rows
            # zero-padded to the stored head dim.
            if k_norm_weight is not None:
                k = headdim.rms_norm(k, k_norm_weight, norm_eps)
            if rope_cos is not None:
                tt = torch.arange(t, device=k.device)
                pos = int(start_pos) + tt if start_pos is not None else self.cache_seqlens[: k.shape[0], None].long() + tt
                k = headdim.rotate(k, rope_cos.float(), rope_sin.float(), pos)
            k, v = headdim.pad(k, self.head_dim_padded), headdim.pad(v, self.head_dim_padded)
            rope_cos = rope_sin = k_norm_weight = None
        ops.kv_append(
            k,
            v,
            self._k_store,
            self._v_store,
            self.cache_seqlens,
            rope_cos=rope_cos,
            rope_sin=rope_sin,
            rope_k=rope_cos is not None,
            rope_k_offset=0 if start_pos is None else int(start_pos),
            rope_pos_abs=start_pos is not None,
            k_norm_weight=k_norm_weight,
            norm_eps=norm_eps,
            status=self.status,
        )

    def update(self, k: torch.Tensor, v: torch.Tensor, start_pos: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
        """mint/kvcache/base.py:35-50: rows [start_pos, start_pos+T) of every
        sequence, cache_seqlens[:B] = start_pos + T, views up to that row."""
        batch_size, seq_len = k.shape[0], k.shape[1]
        if start_pos < 0 or start_pos + seq_len > self.max_seq_len:
            raise ValueError(f"KVCache.update: rows [{start_pos}, {start_pos + seq_len}) exceed max_seq_len {self.max_seq_len}")
        self.cache_seqlens[:batch_size].fill_(start_pos)
        bound = self.len_bound
        self.len_bound = None  # the append below is checked by the explicit range above
        self.append(k, v)
        self.len_bound = None if bound is None else max(bound, start_pos + seq_len)
        end_pos = start_pos + seq_len
        return self.k_cache[:batch_size, :end_pos], self.v_cache[:batch_size, :end_pos]

    def set_seqlens(self, lengths) -> None:
        """Set cache_seqlens[:len(lengths)] (host values) and the host bound."""
        lengths = torch.as_tensor(lengths, dtype=torch.int32)
        if lengths.numel() and (int(lengths.min()) < 0 or int(lengths.max()) > self.max_seq_len):
            raise ValueError(f"KVCache.set_seqlens: lengths must lie in [0, {self.max_seq_len}]")
        self.cache_seqlens[: lengths.numel()] = lengths.to(self.cache_seqlens.device)
        if self.len_bound is not None:
            self.len_bound = max(self.len_bound, int(lengths.max()) if lengths.numel() else 0)

    def check(self) -> None:
        """Raise if an append ran past max_seq_len (reads the device status)."""
        if int(self.status.item()) != 0:
            raise RuntimeError(f"KVCache: an append ran past max_seq_len {self.max_seq_len}; rows past it were dropped")

    def get(self) -> tuple[torch.Tensor, torch.Tensor]:
        """mint/kvcache/base.py:52-54 (reads the length of sequence 0 on the host)."""
        self.check()
        pos = int(self.cache_seqlens[0].item())
        return self.k_cache[:, :pos], self.v_cache[:, :pos]

    def cache_tensors(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """The storage for this package's own kernels, padded to
        head_dim_padded (keeps len_bound)."""
        return self._k_store, self._v_store, self.cache_seqlens

    def get_cache_tensors(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        # The caller may write the lengths: the host bound is no longer known.
        self.len_bound = None
        return self.k_cache, self.v_cache, self.cache_seqlens

    def reset(self) -> None:
        self.cache_seqlens.zero_()
        self.status.zero_()
        self.len_bound = 0

    def clear(self) -> None:
        self._k_store.zero_()
        self._v_store.zero_()
        self.cache_seqlens.zero_()
        self.status.zero_()
        self.len_bound = 0
