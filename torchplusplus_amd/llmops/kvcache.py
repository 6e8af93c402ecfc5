"""KV cache (reference: torchpp/llmops/kvcache.py:6-116).

Same constructor and update/reset API, with the reference's defects fixed:
  * the cache is [B, n_kv_heads, max_seq_len, head_dim] for any batch B
    (batch was hard-coded to 1 at kvcache.py:40,45);
  * it is allocated once at full length on first use (kvcache.py:66 allocated
    a single position);
  * update() returns the prefix [:cache_len] as views, not one position
    (kvcache.py:79-80) and not `.contiguous()` copies (kvcache.py:106-107);
  * writing past max_seq_len raises instead of corrupting memory.
The attention kernels read and write this layout in place: K/V rows of
sequence b, head h are contiguous along positions.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch


class KVCache:
    def __init__(self, max_seq_len: int, n_kv_heads: int, head_dim: int,
                 dtype: torch.dtype = torch.float16, device=torch.device("cuda"),
                 batch_size: Optional[int] = None):
        self.max_seq_len = max_seq_len
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = device
        self.k_cache: Optional[torch.Tensor] = None
        self.v_cache: Optional[torch.Tensor] = None
        self.cache_len = 0
        if batch_size is not None:
            self.ensure(batch_size, 0)

    @property
    def batch_size(self) -> int:
        return 0 if self.k_cache is None else self.k_cache.shape[0]

    def ensure(self, batch_size: int, length: int) -> None:
        """Allocate (once) for `batch_size` sequences; check `length` fits."""
        if length > self.max_seq_len:
            raise ValueError(f"KV cache overflow: {length} > max_seq_len {self.max_seq_len}")
        if self.k_cache is None or self.k_cache.shape[0] < batch_size:
            shape = (batch_size, self.n_kv_heads, self.max_seq_len, self.head_dim)
            self.k_cache = torch.zeros(shape, dtype=self.dtype, device=self.device)
            self.v_cache = torch.zeros(shape, dtype=self.dtype, device=self.device)
            self.cache_len = 0

    def update(self, k: torch.Tensor, v: torch.Tensor, index: Optional[int] = None
               ) -> Tuple[torch.Tensor, torch.Tensor]:
        """Write k, v [B, n_kv_heads, S, head_dim] at cache_len (index None) or
        at `index`, and return the cached prefix [B, n_kv_heads, cache_len, D]."""
        bsz, _, seq_len, _ = k.shape
        start = self.cache_len if index is None else int(index)
        end = start + seq_len
        self.ensure(bsz, end)
        self.k_cache[:bsz, :, start:end] = k
        self.v_cache[:bsz, :, start:end] = v
        self.cache_len = max(self.cache_len, end) if index is not None else end
        return self.k_cache[:bsz, :, : self.cache_len], self.v_cache[:bsz, :, : self.cache_len]

    def reset(self) -> None:
        self.cache_len = 0
        if self.k_cache is not None:
            self.k_cache.zero_()
            self.v_cache.zero_()
