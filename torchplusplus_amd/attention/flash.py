"""In-package replacement for the third-party `flash_attn.flash_attn_func`
that the reference imports at torchpp/attention/gqa.py:4 (and swa/mha/mqa/ca).

Same calling convention: q [B, Sq, Hq, D], k/v [B, Sk, Hkv, D] (last dim
contiguous, other strides free), Hq % Hkv == 0 (GQA/MQA natively, no
repeat_interleave), causal aligned bottom-right, window_size=(left, right)
with -1 = unbounded, softmax_scale default 1/sqrt(D).
"""
from __future__ import annotations

import torch

from torchplusplus_amd._native import ext as _ext

_C = _ext()


def flash_attn_func(q, k, v, dropout_p: float = 0.0, softmax_scale=None, causal: bool = False,
                    window_size=(-1, -1), **unused):
    if dropout_p:
        raise NotImplementedError("dropout is not supported (inference kernel)")
    if unused.get("return_attn_probs"):
        raise NotImplementedError("return_attn_probs is not supported")
    left, right = window_size
    return _C.flash_attn_func(q, k, v, causal, int(left), int(right),
                              float(softmax_scale) if softmax_scale else 0.0)


def decode_attention(q, k_cache, v_cache, seqlens=None, softmax_scale=None, window_left: int = -1,
                     out=None):
    """One query per sequence, q [B, 1, Hq, D], against the first seqlens[b]
    positions of caches [B, Hkv, Lmax, D] (split-KV kernel)."""
    return _C.attn_decode(q, k_cache, v_cache, seqlens,
                          float(softmax_scale) if softmax_scale else 0.0, int(window_left), out)
