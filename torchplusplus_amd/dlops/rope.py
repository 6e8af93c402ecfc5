"""Rotary embedding ops (reference: torchpp/dlops/rope.py:6-54).

rope_apply / qkrope_apply keep the reference signatures and return new
tensors; `rope_apply_` is the in-place variant. The kernels accept fp16 and
bf16 inputs with fp16, bf16 or fp32 cos/sin tables, and qkrope_apply allows
fewer K heads than Q heads (GQA).
"""
from __future__ import annotations

import torch

from torchplusplus_amd._native import ext as _ext

_C = _ext()


def rope_apply(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE of x [B, H, S, D] with tables [S, D] (rope.py:6-21)."""
    return _C.rope_apply_cuda(x, cos, sin)


def rope_apply_(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """In-place rope_apply; returns x."""
    return _C.rope_apply_(x, cos, sin)


def qkrope_apply(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """RoPE of q [B, Hq, S, D] and k [B, Hk, S, D] in one launch (rope.py:24-41)."""
    return _C.qkrope_apply_cuda(q, k, cos, sin)


def compute_rope_params(head_dim, theta_base, context_length, device="cuda",
                        dtype=torch.float32, out_dtype=torch.float16):
    """cos/sin tables [context_length, head_dim] (rope.py:43-54): angles
    pos * theta^(-2j/D) in `dtype`, duplicated over both halves, cast to
    `out_dtype` (fp16 in the reference)."""
    assert head_dim % 2 == 0, "head dim must be divisible by 2"
    j = torch.arange(0, head_dim, 2, device=device, dtype=dtype)
    inv_freq = 1.0 / (theta_base ** (j / head_dim))
    pos = torch.arange(context_length, device=device, dtype=dtype)
    ang = torch.outer(pos, inv_freq)
    ang = torch.cat([ang, ang], dim=1)
    return ang.cos().to(out_dtype).contiguous(), ang.sin().to(out_dtype).contiguous()
