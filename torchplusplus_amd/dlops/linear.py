"""Linear layers (reference: torchpp/dlops/linear.py:8-145).

LinearGELU / LinearSILU keep the reference constructor (in_features,
out_features) and randn weight init (linear.py:20-22), and run the fused
MFMA GEMM + activation epilogue. Extras: `dtype`/`device`/`bias` keyword
arguments, N-D inputs, and a GEMV path for decode (<= 16 rows).
"""
from __future__ import annotations

import torch
import torch.nn as nn

from torchplusplus_amd._native import ext as _ext

_C = _ext()

ACT_NONE, ACT_GELU, ACT_SILU, ACT_RELU = 0, 1, 2, 3
GEMV_MAX_ROWS = 16


def linear(x: torch.Tensor, weight: torch.Tensor, bias=None, act: int = ACT_NONE) -> torch.Tensor:
    """act(x @ weight^T + bias) on the gfx950 kernels: the split-K GEMV for
    decode-sized inputs (<= 16 rows), the MFMA GEMM otherwise."""
    rows = x.numel() // x.shape[-1]
    if rows <= GEMV_MAX_ROWS:
        return _C.gemv(x, weight, bias, act)
    return _C.linear(x, weight, bias, act)


def swiglu(x: torch.Tensor, w_gu: torch.Tensor) -> torch.Tensor:
    """silu(x Wg^T) * (x Wu^T) from a [gate|up] weight interleaved in blocks
    of 32 rows (see interleave_gate_up)."""
    rows = x.numel() // x.shape[-1]
    if rows <= GEMV_MAX_ROWS:
        return _C.gemv_swiglu(x, w_gu)
    return _C.linear_swiglu(x, w_gu)


def interleave_gate_up(w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """[I, K] gate and up weights -> [2I, K] with rows 64j..64j+31 = gate rows
    32j.. and rows 64j+32..64j+63 = up rows 32j.. (I % 32 == 0)."""
    i, k = w_gate.shape
    assert w_up.shape == (i, k) and i % 32 == 0
    return torch.stack([w_gate.reshape(i // 32, 32, k), w_up.reshape(i // 32, 32, k)], 1).reshape(2 * i, k).contiguous()


class _LinearAct(nn.Module):
    ACT = ACT_NONE

    def __init__(self, in_features, out_features, bias: bool = False,
                 dtype: torch.dtype = torch.float16, device=None):
        super().__init__()
        self.weight = nn.Parameter(torch.randn(out_features, in_features, dtype=dtype, device=device))
        self.bias = nn.Parameter(torch.zeros(out_features, dtype=dtype, device=device)) if bias else None

    def forward(self, x):
        return linear(x, self.weight, self.bias, self.ACT)


class LinearGELU(_LinearAct):
    """Linear layer with fused GELU (tanh approximation) (linear.py:8-25)."""

    ACT = ACT_GELU


class LinearSILU(_LinearAct):
    """Linear layer with fused SiLU (linear.py:28-45)."""

    ACT = ACT_SILU


class LinearRELU(_LinearAct):
    """Linear layer with fused ReLU (the binding's LinearRelu, binding.cu:112-160)."""

    ACT = ACT_RELU


class Dense(nn.Module):
    """Contraction of `axis` of x with the leading dims of a weight of shape
    in_features + out_features (linear.py:48-101; plain torch there too)."""

    def __init__(self, in_featrues, out_features, axis=(-1,), weight_dtype=torch.float16,
                 device=torch.device("cuda")):
        super().__init__()
        self.in_features = tuple(in_featrues)
        self.out_features = tuple(out_features)
        self.axis = tuple(axis)
        self.weight = nn.Parameter(torch.empty(self.in_features + self.out_features,
                                               dtype=weight_dtype, device=device))
        nn.init.normal_(self.weight, std=0.02)

    def forward(self, x):
        dims = tuple(a % x.ndim for a in self.axis)
        out = torch.tensordot(x.to(self.weight.dtype), self.weight,
                              dims=(dims, tuple(range(len(dims)))))
        return out.to(x.dtype)


class LinearNBFp16(nn.Module):
    """Bias-free fp16 nn.Linear wrapper (linear.py:108-126)."""

    def __init__(self, in_features, out_features):
        super().__init__()
        self.linear = nn.Linear(in_features, out_features, bias=False, dtype=torch.float16)

    def forward(self, x):
        return linear(x, self.linear.weight)


class LinearNBBf16(nn.Module):
    """Bias-free bf16 nn.Linear wrapper (linear.py:129-145)."""

    def __init__(self, in_features, out_features):
        super().__init__()
        self.linear = nn.Linear(in_features, out_features, bias=False, dtype=torch.bfloat16)

    def forward(self, x):
        return linear(x, self.linear.weight)
