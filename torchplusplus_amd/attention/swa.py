"""Sliding-window attention (reference: torchpp/attention/swa.py:8-93):
causal attention limited to the last `window_size` keys,
flash_attn_func(..., window_size=(window_size - 1, 0)) (swa.py:85-89).
Same fixes as MultiHeadAttention (module init, head_dim QK-norm)."""
from __future__ import annotations

import torch

from torchplusplus_amd.attention._common import head_rmsnorm, rope_bshd
from torchplusplus_amd.attention.flash import flash_attn_func
from torchplusplus_amd.attention.mha import MultiHeadAttention
from torchplusplus_amd.dlops.linear import linear


class SlidingWindowAttention(MultiHeadAttention):
    def __init__(self, window_size: int, embed_dim: int, n_heads: int, qknorm: bool = True,
                 dtype: torch.dtype = torch.float16, device=None):
        super().__init__(embed_dim, n_heads, qknorm, dtype, device)
        self.window_size = window_size

    def forward(self, x: torch.Tensor, cos, sin):
        bsz, seq, _ = x.shape
        q = head_rmsnorm(self._heads(linear(x, self.Wq.weight), bsz, seq), self.q_norm)
        k = head_rmsnorm(self._heads(linear(x, self.Wk.weight), bsz, seq), self.k_norm)
        v = self._heads(linear(x, self.Wv.weight), bsz, seq)
        q, k = rope_bshd(q, cos, sin), rope_bshd(k, cos, sin)
        o = flash_attn_func(q, k, v, causal=True, window_size=(self.window_size - 1, 0))
        return linear(o.reshape(bsz, seq, self.embed_dim), self.out_projection.weight,
                      self.out_projection.bias)
