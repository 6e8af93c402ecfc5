"""CPU restatements of the reference's attention modules (test
infrastructure only), composed from the per-op oracle with the eager dtype
flow: each op computes in fp32 from model-dtype inputs and rounds once.

  mha / swa  torchpp/attention/mha.py:57-88, swa.py:59-93: q/k/v projections,
             per-head RMSNorm over head_dim (the reference builds
             nn.RMSNorm(embed_dim), mha.py:52-54, which cannot normalise
             head_dim-wide rows; the build normalises over head_dim with
             eps 1e-6), rotate-half RoPE with tables [S, D], causal attention
             (swa: window (w-1, 0), swa.py:85-89), output projection with bias.
  mqa        torchpp/attention/mqa.py:62-93: one K/V head; K rotated from K
             (mqa.py:81 rotates Q into K, a defect the build fixes).
  cross      torchpp/attention/ca.py:60-87: q from x, k/v from the context y,
             non-causal, output projection with bias; an optional cached
             prefix of context K/V is attended before the new context.
  GQAOracle  torchpp/attention/gqa.py:70-131: fused-free GQA with QK-norm,
             RoPE at absolute positions cache_pos.., K/V appended to a cache,
             causal (bottom-right) attention over the cache prefix.
Weights are passed as a dict keyed by the module's parameter names.
"""
from __future__ import annotations

import torch

from . import ops


def _w(p, name):
    return p[name].detach().cpu()


def _lin(x, p, name, bias=None):
    b = _w(p, bias) if bias is not None and bias in p else None
    return ops.linear_act(x, _w(p, name), b, "none")


def _rope_bshd(t, cos, sin):
    return ops.rope(t.transpose(1, 2), cos, sin).transpose(1, 2)


def _heads(t, B, S, H, D):
    return t.reshape(B, S, H, D)


def mha(x, p, cos, sin, n_heads, qknorm=True, window_size=None):
    """MultiHeadAttention / SlidingWindowAttention forward; cos/sin [S, D]."""
    B, S, E = x.shape
    D = E // n_heads
    q = _heads(_lin(x, p, "Wq.weight"), B, S, n_heads, D)
    k = _heads(_lin(x, p, "Wk.weight"), B, S, n_heads, D)
    v = _heads(_lin(x, p, "Wv.weight"), B, S, n_heads, D)
    if qknorm:
        q = ops.rmsnorm(q, _w(p, "q_norm.weight"), 1e-6)
        k = ops.rmsnorm(k, _w(p, "k_norm.weight"), 1e-6)
    q, k = _rope_bshd(q, cos, sin), _rope_bshd(k, cos, sin)
    window = (window_size - 1, 0) if window_size is not None else (-1, -1)
    o = ops.attention(q, k, v, causal=True, window=window)
    return _lin(o.reshape(B, S, E), p, "out_projection.weight", "out_projection.bias")


def mqa(x, p, cos, sin, n_q_heads, qk_norm=True):
    B, S, E = x.shape
    D = E // n_q_heads
    q = _heads(_lin(x, p, "Wq.weight"), B, S, n_q_heads, D)
    k = _heads(_lin(x, p, "Wk.weight"), B, S, 1, D)
    v = _heads(_lin(x, p, "Wv.weight"), B, S, 1, D)
    if qk_norm:
        q = ops.rmsnorm(q, _w(p, "q_norm.weight"), 1e-6)
        k = ops.rmsnorm(k, _w(p, "k_norm.weight"), 1e-6)
    q, k = _rope_bshd(q, cos, sin), _rope_bshd(k, cos, sin)
    o = ops.attention(q, k, v, causal=True)
    return _lin(o.reshape(B, S, E), p, "out_projection.weight")


def cross(x, y, p, n_heads, prefix_kv=None):
    """CrossAttention forward. prefix_kv: optional (k, v) [B, Sp, H, D]
    already in the cache; returns (out, (k_all, v_all))."""
    B, Sq, E = x.shape
    D = E // n_heads
    q = _heads(_lin(x, p, "Wq.weight"), B, Sq, n_heads, D)
    k = _lin(y, p, "Wk.weight").reshape(B, -1, n_heads, D)
    v = _lin(y, p, "Wv.weight").reshape(B, -1, n_heads, D)
    if prefix_kv is not None:
        k = torch.cat([prefix_kv[0], k], dim=1)
        v = torch.cat([prefix_kv[1], v], dim=1)
    o = ops.attention(q, k, v, causal=False)
    return _lin(o.reshape(B, Sq, E), p, "out_projection.weight", "out_projection.bias"), (k, v)


class GQAOracle:
    """GroupedQueryAttention.forward with an optional cache (gqa.py:70-131)."""

    def __init__(self, p, n_heads, n_kv_heads, head_dim, qk_norm=True):
        self.p, self.H, self.Hk, self.D, self.qk_norm = p, n_heads, n_kv_heads, head_dim, qk_norm
        self.k = self.v = None

    def forward(self, x, cos, sin, cache_pos=None):
        """cos/sin: full tables [ctx, D]; cache_pos None = no cache (positions
        0..S-1, gqa.py:111-113), else positions cache_pos.. and the cache."""
        B, S, _ = x.shape
        q = _heads(_lin(x, self.p, "Wq.weight"), B, S, self.H, self.D)
        k = _heads(_lin(x, self.p, "Wk.weight"), B, S, self.Hk, self.D)
        v = _heads(_lin(x, self.p, "Wv.weight"), B, S, self.Hk, self.D)
        if self.qk_norm:
            q = ops.rmsnorm(q, _w(self.p, "q_norm.weight"), 1e-6)
            k = ops.rmsnorm(k, _w(self.p, "k_norm.weight"), 1e-6)
        start = 0 if cache_pos is None else cache_pos
        pos = slice(start, start + S)
        q, k = _rope_bshd(q, cos[pos], sin[pos]), _rope_bshd(k, cos[pos], sin[pos])
        if cache_pos is not None:
            if cache_pos == 0 or self.k is None:
                self.k, self.v = k, v
            else:
                self.k = torch.cat([self.k[:, :cache_pos], k], 1)
                self.v = torch.cat([self.v[:, :cache_pos], v], 1)
            k, v = self.k, self.v
        o = ops.attention(q, k, v, causal=True)
        return _lin(o.reshape(B, S, self.H * self.D), self.p, "out_projection.weight")
