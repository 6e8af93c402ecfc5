"""Grouped-query attention (reference: torchpp/attention/gqa.py:11-131).

Same constructor and forward signature. Per call the layer runs:
  1. one fused Q/K/V projection (MFMA GEMM, or the split-K GEMV for <= 16 tokens)
  2. one fused kernel: QK-RMSNorm over head_dim + RoPE at the absolute
     positions + K/V written into the cache (or a scratch buffer)
  3. flash attention with native GQA (no repeat_interleave / .contiguous()
     copies), or split-KV decode attention when a single token is appended
  4. the output projection.
The fused projection weight is built from Wq/Wk/Wv on first use and rebuilt
whenever one of them changes (load_state_dict, in-place edits), as the
reference reads its projection weights on every call (gqa.py:82-84).
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from torchplusplus_amd._native import ext as _ext
from torchplusplus_amd.attention.flash import flash_attn_func
from torchplusplus_amd.dlops.derived import DerivedWeight, attach
from torchplusplus_amd.dlops.linear import linear
from torchplusplus_amd.llmops.kvcache import KVCache

_C = _ext()

# one [bs] int32 positions tensor per device, reused by the layers of a
# forward pass (one fill launch per pass instead of one per layer)
_POSITIONS: dict = {}


def _positions(bs: int, start: int, dev: torch.device) -> torch.Tensor:
    """[bs] int32 tensor of `start`, filled on the current stream and reused
    only on that stream (so its fill is ordered before every kernel that
    reads it). Not cached while the stream is being captured: a tensor filled
    inside a capture holds its value only once the graph has been replayed."""
    if dev.type != "cuda" or torch.cuda.is_current_stream_capturing():
        return torch.full((bs,), start, dtype=torch.int32, device=dev)
    key = (bs, start, torch.cuda.current_stream(dev).cuda_stream)
    hit = _POSITIONS.get(dev)
    if hit is None or hit[0] != key:
        hit = (key, torch.full((bs,), start, dtype=torch.int32, device=dev))
        _POSITIONS[dev] = hit
    return hit[1]


class GroupedQueryAttention(nn.Module):
    def __init__(self, d_in: int, num_heads: int, n_kv_heads: int, head_dim: Optional[int] = None,
                 qk_norm: bool = True, dtype: torch.dtype = torch.float16, DEBUG: bool = False,
                 device=None):
        super().__init__()
        assert num_heads % n_kv_heads == 0, "Num heads is not divisible by num kv grps"
        self.num_heads = num_heads
        self.n_kv_heads = n_kv_heads
        self.num_kv_grps = num_heads // n_kv_heads
        if head_dim is None:
            assert d_in % num_heads == 0, "in dimension must be divisible by number of heads"
            head_dim = d_in // num_heads
        self.head_dim = head_dim
        self.d_out = head_dim * num_heads
        kw = dict(bias=False, dtype=dtype, device=device)
        self.Wq = nn.Linear(d_in, self.d_out, **kw)
        self.Wk = nn.Linear(d_in, n_kv_heads * head_dim, **kw)
        self.Wv = nn.Linear(d_in, n_kv_heads * head_dim, **kw)
        self.out_projection = nn.Linear(self.d_out, d_in, **kw)
        if qk_norm:
            self.q_norm = nn.RMSNorm(head_dim, eps=1e-6, dtype=dtype, device=device)
            self.k_norm = nn.RMSNorm(head_dim, eps=1e-6, dtype=dtype, device=device)
        else:
            self.q_norm = self.k_norm = None
        self.DEBUG = DEBUG
        self._wqkv = attach(self, DerivedWeight(lambda q, k, v: torch.cat([q, k, v], 0).contiguous()))

    def refresh_fused_weights(self):
        """Force a rebuild of the fused projection weight."""
        self._wqkv.invalidate()
        self.fused_qkv_weight()

    def fused_qkv_weight(self) -> torch.Tensor:
        """[(Hq+2Hkv)*D, d_in]: Wq, Wk, Wv stacked, current with the parameters."""
        return self._wqkv.get(self.Wq.weight, self.Wk.weight, self.Wv.weight)

    def rope_cache(self, qkv, cos, sin, k_dst, v_dst, positions):
        """Step 2 on a projected qkv [B, S, (Hq+2Hkv)*D]: returns q [B, S, Hq, D];
        K/V rows land in k_dst/v_dst ([B, Hkv, L, D]) at positions[b] + s."""
        bs, seq_len = qkv.shape[0], qkv.shape[1]
        q = torch.empty(bs, seq_len, self.num_heads, self.head_dim, dtype=qkv.dtype, device=qkv.device)
        eps = self.q_norm.eps if self.q_norm is not None and self.q_norm.eps is not None else 1e-6
        _C.qkv_rope_cache(qkv, q, k_dst, v_dst,
                          self.q_norm.weight if self.q_norm is not None else None,
                          self.k_norm.weight if self.k_norm is not None else None,
                          cos, sin, positions, eps)
        return q

    def decode_fused(self, qkv, cos, sin, k_cache, v_cache, seqlens):
        """One new token per sequence: QK-norm + RoPE at position seqlens-1,
        K/V appended to the caches, split-KV attention over seqlens keys;
        returns [B, 1, Hq, D]."""
        eps = self.q_norm.eps if self.q_norm is not None and self.q_norm.eps is not None else 1e-6
        return _C.attn_decode_fused(qkv, self.q_norm.weight if self.q_norm is not None else None,
                                    self.k_norm.weight if self.k_norm is not None else None,
                                    cos, sin, eps, k_cache, v_cache, seqlens)

    def decode_oproj(self, qkv, cos, sin, k_cache, v_cache, seqlens, residual):
        """decode_fused, then the output projection with the residual add:
        residual [B, 1, d_in] <- residual + out_projection(attention output),
        in place (one launch at the Qwen3-0.6B decode shape); returns the
        attention output [B, 1, Hq, D]."""
        eps = self.q_norm.eps if self.q_norm is not None and self.q_norm.eps is not None else 1e-6
        return _C.attn_decode_oproj(qkv, self.q_norm.weight if self.q_norm is not None else None,
                                    self.k_norm.weight if self.k_norm is not None else None,
                                    cos, sin, eps, k_cache, v_cache, seqlens,
                                    self.out_projection.weight, residual)

    def attend_oproj(self, qkv, cos, sin, kv_cache: KVCache, cache_pos: Optional[int],
                     residual: torch.Tensor) -> None:
        """One new token per sequence through the cache: steps 2-4 with the
        residual add, residual [B, 1, d_in] updated in place."""
        bs = qkv.shape[0]
        start = kv_cache.cache_len if cache_pos is None else int(cache_pos)
        kv_cache.ensure(bs, start + 1)
        seqlens = _positions(bs, start + 1, qkv.device)
        kv_cache.cache_len = max(kv_cache.cache_len, start + 1)
        self.decode_oproj(qkv, cos, sin, kv_cache.k_cache[:bs], kv_cache.v_cache[:bs], seqlens,
                          residual)

    def attend(self, qkv, cos, sin, kv_cache: Optional[KVCache] = None,
               cache_pos: Optional[int] = None) -> torch.Tensor:
        """Steps 2-3: rope/cache the projected qkv and attend; returns the
        attention output [B, S, Hq*D] (before the output projection)."""
        bs, seq_len = qkv.shape[0], qkv.shape[1]
        dev = qkv.device
        if kv_cache is not None:
            start = kv_cache.cache_len if cache_pos is None else int(cache_pos)
            kv_cache.ensure(bs, start + seq_len)
            total = start + seq_len
            # the cache may hold more sequences than this call (allocated for
            # an earlier, larger batch): the kernels get this batch's rows
            kc_b, vc_b = kv_cache.k_cache[:bs], kv_cache.v_cache[:bs]
            if seq_len == 1:
                # one new token: QK-norm + RoPE + cache append fused into the
                # split-KV decode kernel
                seqlens = _positions(bs, total, dev)
                kv_cache.cache_len = max(kv_cache.cache_len, total)
                return self.decode_fused(qkv, cos, sin, kc_b, vc_b,
                                         seqlens).reshape(bs, seq_len, self.d_out)
            positions = _positions(bs, start, dev)
            q = self.rope_cache(qkv, cos, sin, kc_b, vc_b, positions)
            kv_cache.cache_len = max(kv_cache.cache_len, start + seq_len)
            o = flash_attn_func(q, kc_b[:, :, :total].transpose(1, 2),
                                vc_b[:, :, :total].transpose(1, 2), causal=True)
        else:
            k = torch.empty(bs, self.n_kv_heads, seq_len, self.head_dim, dtype=qkv.dtype, device=dev)
            v = torch.empty_like(k)
            positions = _positions(bs, 0, dev)
            q = self.rope_cache(qkv, cos, sin, k, v, positions)
            o = flash_attn_func(q, k.transpose(1, 2), v.transpose(1, 2), causal=True)
        return o.reshape(bs, seq_len, self.d_out)

    def forward(self, x, cos, sin, kv_cache: Optional[KVCache] = None,
                cache_pos: Optional[int] = None):
        qkv = linear(x, self.fused_qkv_weight())
        return linear(self.attend(qkv, cos, sin, kv_cache, cache_pos), self.out_projection.weight)
