"""Normalisation modules (reference: torchpp/dlops/normalization.py:7-77).

RmsNormFused / LayerNormFused keep the reference constructor signature
(normalize_dim_shape, eps=1e-6, dtype=float16, device="cuda") and call the
gfx950 kernels through the torch extension. bf16 is accepted as well.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from torchplusplus_amd._native import ext as _ext

_C = _ext()


class LayerNormFused(nn.Module):
    """y = (x - mean) * rsqrt(var + eps) * weight over the last dim, no bias
    (reference normalization.py:7-27 -> layernormFused.applyLayernorm)."""

    def __init__(
        self,
        normalize_dim_shape: int,
        eps: float = 1e-6,
        dtype: torch.dtype = torch.float16,
        device: torch.device = torch.device("cuda"),
    ):
        super().__init__()
        self.shape = normalize_dim_shape
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(self.shape, dtype=dtype, device=device))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _C.applyLayernorm(x, self.weight, self.eps)


class RmsNormFused(nn.Module):
    """y = x * rsqrt(mean(x^2) + eps) * weight over the last dim
    (reference normalization.py:30-50 -> rmsnormFused.rmsnormFused)."""

    def __init__(
        self,
        normalize_dim_shape: int,
        eps: float = 1e-6,
        dtype: torch.dtype = torch.float16,
        device: torch.device = torch.device("cuda"),
    ):
        super().__init__()
        self.shape = normalize_dim_shape
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(self.shape, dtype=dtype, device=device))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _C.rmsnormFused(x, self.weight, self.eps)

    def forward_add(self, x: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
        """Fused `residual += x; return self(residual)` (one pass over HBM)."""
        return _C.add_rmsnorm(x, residual, self.weight, self.eps)


class LayerNorm4D(nn.Module):
    """Per-channel-last LayerNorm over dims (2, 3) of a 4-D tensor with a
    learned affine (reference normalization.py:58-77; plain torch there too)."""

    def __init__(self, num_features: int):
        super().__init__()
        self.gamma = nn.Parameter(torch.ones(1, 1, 1, num_features))
        self.beta = nn.Parameter(torch.zeros(1, 1, 1, num_features))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        var, mean = torch.var_mean(x, dim=(2, 3), keepdim=True, correction=0)
        return (x - mean) * torch.rsqrt(var + 1e-6) * self.gamma + self.beta
