"""Cross attention (reference: torchpp/attention/ca.py:10-87): queries from x,
keys/values from a context y [B, Skv, cross_dim], non-causal. Optional
KVCache: the projected context K/V are appended and attended as a prefix.
Fix: the context is unpacked as 3-D (the reference unpacks `_, s = y.shape`,
ca.py:68)."""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from torchplusplus_amd.attention.flash import flash_attn_func
from torchplusplus_amd.dlops.linear import linear
from torchplusplus_amd.llmops.kvcache import KVCache


class CrossAttention(nn.Module):
    def __init__(self, embed_dim: int, cross_dim: int, n_heads: int, qknorm: bool = True,
                 dtype: torch.dtype = torch.float16, device=None):
        super().__init__()
        assert embed_dim % n_heads == 0, "embed dimension should be divisible by number of heads"
        self.embed_dim, self.cross_dim, self.n_heads = embed_dim, cross_dim, n_heads
        self.head_dim = embed_dim // n_heads
        self.qknorm, self.dtype = qknorm, dtype
        self.hidden_dim = self.head_dim * n_heads
        kw = dict(dtype=dtype, device=device)
        self.Wq = nn.Linear(embed_dim, self.hidden_dim, bias=False, **kw)
        self.Wk = nn.Linear(cross_dim, self.hidden_dim, bias=False, **kw)
        self.Wv = nn.Linear(cross_dim, self.hidden_dim, bias=False, **kw)
        self.out_projection = nn.Linear(self.hidden_dim, embed_dim, **kw)

    def forward(self, x: torch.Tensor, y: torch.Tensor, kv_cache: Optional[KVCache] = None):
        bsz, sq, _ = x.shape
        q = linear(x, self.Wq.weight).view(bsz, sq, self.n_heads, self.head_dim)
        k = linear(y, self.Wk.weight).view(bsz, -1, self.n_heads, self.head_dim)
        v = linear(y, self.Wv.weight).view(bsz, -1, self.n_heads, self.head_dim)
        if kv_cache is not None:
            kc, vc = kv_cache.update(k.transpose(1, 2), v.transpose(1, 2))
            k, v = kc.transpose(1, 2), vc.transpose(1, 2)
        o = flash_attn_func(q, k, v).reshape(bsz, sq, self.embed_dim)
        return linear(o, self.out_projection.weight, self.out_projection.bias)
