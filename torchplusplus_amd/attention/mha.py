"""Multi-head attention (reference: torchpp/attention/mha.py:8-88).

Same constructor/forward. Differences, all fixes: nn.Module is initialised
(the reference skips super().__init__(), mha.py:17), and the optional QK-norm
normalises over head_dim (the reference builds nn.RMSNorm(embed_dim) and
applies it to head_dim-wide rows, mha.py:52-54,71-74, which cannot run)."""
from __future__ import annotations

import torch
import torch.nn as nn

from torchplusplus_amd.attention._common import head_rmsnorm, rope_bshd
from torchplusplus_amd.attention.flash import flash_attn_func
from torchplusplus_amd.dlops.linear import linear


class MultiHeadAttention(nn.Module):
    def __init__(self, embed_dim: int, n_heads: int, qknorm: bool = True,
                 dtype: torch.dtype = torch.float16, device=None):
        super().__init__()
        assert embed_dim % n_heads == 0, "embed dimension should be divisible by number of heads"
        self.embed_dim, self.n_heads = embed_dim, n_heads
        self.head_dim = embed_dim // n_heads
        self.qknorm, self.dtype = qknorm, dtype
        kw = dict(dtype=dtype, device=device)
        self.Wq = nn.Linear(embed_dim, embed_dim, bias=False, **kw)
        self.Wk = nn.Linear(embed_dim, embed_dim, bias=False, **kw)
        self.Wv = nn.Linear(embed_dim, embed_dim, bias=False, **kw)
        self.out_projection = nn.Linear(embed_dim, embed_dim, **kw)
        if qknorm:
            self.q_norm = nn.RMSNorm(self.head_dim, eps=1e-6, **kw)
            self.k_norm = nn.RMSNorm(self.head_dim, eps=1e-6, **kw)
        else:
            self.q_norm = self.k_norm = None

    def _heads(self, t, bsz, seq):
        return t.view(bsz, seq, self.n_heads, self.head_dim)

    def forward(self, x: torch.Tensor, cos, sin):
        bsz, seq, _ = x.shape
        q = head_rmsnorm(self._heads(linear(x, self.Wq.weight), bsz, seq), self.q_norm)
        k = head_rmsnorm(self._heads(linear(x, self.Wk.weight), bsz, seq), self.k_norm)
        v = self._heads(linear(x, self.Wv.weight), bsz, seq)
        q, k = rope_bshd(q, cos, sin), rope_bshd(k, cos, sin)
        o = flash_attn_func(q, k, v, causal=True).reshape(bsz, seq, self.embed_dim)
        return linear(o, self.out_projection.weight, self.out_projection.bias)
