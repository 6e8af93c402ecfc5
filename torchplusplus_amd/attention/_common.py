"""Shared pieces of the non-GQA attention modules."""
from __future__ import annotations

import torch

from torchplusplus_amd._native import ext as _ext

_C = _ext()


def head_rmsnorm(x: torch.Tensor, norm) -> torch.Tensor:
    """nn.RMSNorm over head_dim on [B, S, H, D] through the fused kernel."""
    if norm is None:
        return x
    eps = norm.eps if norm.eps is not None else 1e-6
    return _C.rmsnormFused(x, norm.weight, eps)


def rope_bshd(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """rope_apply on a [B, S, H, D] tensor: the kernel works on [B, H, S, D]."""
    xt = x.transpose(1, 2).contiguous()
    _C.rope_apply_(xt, cos, sin)
    return xt.transpose(1, 2)
