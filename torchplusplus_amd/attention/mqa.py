"""Multi-query attention (reference: torchpp/attention/mqa.py:9-93): Hq query
heads share one K/V head. Attention runs on the single KV head directly
(no broadcast copy). Fix: K is rotated from K (the reference rotates Q into
K, mqa.py:81)."""
from __future__ import annotations

import torch
import torch.nn as nn

from torchplusplus_amd.attention._common import head_rmsnorm, rope_bshd
from torchplusplus_amd.attention.flash import flash_attn_func
from torchplusplus_amd.dlops.linear import linear


class MultiQueryAttention(nn.Module):
    def __init__(self, num_q_heads: int, embed_dim: int, qk_norm: bool = True,
                 dtype: torch.dtype = torch.float16, device=None):
        super().__init__()
        self.embed_dim = embed_dim
        self.num_q_head = num_q_heads
        self.head_dim = embed_dim // num_q_heads
        kw = dict(dtype=dtype, device=device, bias=False)
        self.Wq = nn.Linear(embed_dim, embed_dim, **kw)
        self.Wk = nn.Linear(embed_dim, self.head_dim, **kw)
        self.Wv = nn.Linear(embed_dim, self.head_dim, **kw)
        self.out_projection = nn.Linear(embed_dim, embed_dim, **kw)
        self.qk_norm = qk_norm
        self.q_norm = nn.RMSNorm(self.head_dim, eps=1e-6, dtype=dtype, device=device)
        self.k_norm = nn.RMSNorm(self.head_dim, eps=1e-6, dtype=dtype, device=device)

    def forward(self, x, cos, sin):
        bsz, seq, _ = x.shape
        q = linear(x, self.Wq.weight).view(bsz, seq, self.num_q_head, self.head_dim)
        k = linear(x, self.Wk.weight).view(bsz, seq, 1, self.head_dim)
        v = linear(x, self.Wv.weight).view(bsz, seq, 1, self.head_dim)
        if self.qk_norm:
            q, k = head_rmsnorm(q, self.q_norm), head_rmsnorm(k, self.k_norm)
        q, k = rope_bshd(q, cos, sin), rope_bshd(k, cos, sin)
        o = flash_attn_func(q, k, v, causal=True)
        return linear(o.reshape(bsz, seq, self.embed_dim), self.out_projection.weight)
