"""CPU restatements of the reference kernels (test infrastructure only).

All functions take and return CPU tensors. Inputs in fp16/bf16 are read
exactly (upcast), arithmetic is fp32 unless stated, and the result is rounded
once to the output dtype -- the numerical contract of the reference kernels.
"""
from __future__ import annotations

import math

import numpy as np
import torch

__all__ = [
    "rmsnorm",
    "rmsnorm_stats",
    "add_rmsnorm",
    "layernorm",
    "layernorm_stats",
    "compute_rope_params",
    "rope",
    "rope_fp16_arith",
    "qkrope",
    "activation",
    "linear_act",
    "gemv",
    "hgemv_cpu",
    "attention",
    "attention_fp64_loops",
    "decode_attention",
]


def _f32(t: torch.Tensor) -> torch.Tensor:
    return t.detach().to("cpu", torch.float32)


# ---------------------------------------------------------------------------
# RMSNorm  -- csrc/dlops/rmsnorm/rmsnorm_fp16.cuh:63-114
#   partial += fx*fx + fy*fy (fp32, :68-74); inv_rms = rsqrtf(sum/N + eps) (:95)
#   out = half((x * inv_rms) * w) in fp32 (:103-113)
# ---------------------------------------------------------------------------
def rmsnorm_stats(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    xf = _f32(x)
    n = xf.shape[-1]
    ss = (xf * xf).sum(dim=-1)
    return torch.rsqrt(ss / n + eps).reshape(-1)


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    xf = _f32(x)
    inv = rmsnorm_stats(x, eps).reshape(xf.shape[:-1] + (1,))
    return ((xf * inv) * _f32(w)).to(x.dtype)


def add_rmsnorm(x, residual, w, eps: float = 1e-6):
    """Decoder block entry (examples/LLM/fastqwen3.py:107-116): the residual
    sum `x + x_res` is a tensor op in the model dtype (one rounding), then
    RMSNorm of that sum. Returns (y, new_residual)."""
    h = (_f32(x) + _f32(residual)).to(x.dtype)
    return rmsnorm(h, w, eps), h


# ---------------------------------------------------------------------------
# LayerNorm -- csrc/dlops/layernorm/layernorm_fp16.cuh:72-143
#   mean = sum/N; var = sumsq/N - mean^2 (:113-114, one pass, fp32)
#   rstd = rsqrt(var + eps); out = half(((x - mean) * rstd) * w)  (:118-132)
#   no bias in the reference; `b` is the build's optional extension.
# ---------------------------------------------------------------------------
def layernorm_stats(x: torch.Tensor, eps: float = 1e-6):
    xf = _f32(x)
    n = xf.shape[-1]
    mean = xf.sum(-1) / n
    var = (xf * xf).sum(-1) / n - mean * mean
    return mean.reshape(-1), torch.rsqrt(var + eps).reshape(-1)


def layernorm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6, b=None) -> torch.Tensor:
    xf = _f32(x)
    mean, rstd = layernorm_stats(x, eps)
    shp = xf.shape[:-1] + (1,)
    y = ((xf - mean.reshape(shp)) * rstd.reshape(shp)) * _f32(w)
    if b is not None:
        y = y + _f32(b)
    return y.to(x.dtype)


# ---------------------------------------------------------------------------
# RoPE tables -- torchpp/dlops/rope.py:43-54 (duplicate fastqwen3.py:33-44)
# ---------------------------------------------------------------------------
def compute_rope_params(head_dim, theta_base, context_length, dtype=torch.float32,
                        out_dtype=torch.float16):
    assert head_dim % 2 == 0, "head dim must be divisible by 2"
    ar = torch.arange(0, head_dim, 2, dtype=dtype)
    inv_freq = 1.0 / (theta_base ** (ar / head_dim))
    pos = torch.arange(context_length, dtype=dtype)
    angles = pos[:, None] * inv_freq[None, :]
    angles = torch.cat([angles, angles], dim=1)
    return torch.cos(angles).to(out_dtype), torch.sin(angles).to(out_dtype)


# ---------------------------------------------------------------------------
# rotate-half RoPE -- csrc/dlops/rope/apply_rope.cuh:15-46 and
# examples/TTS/dia/og_model.py:218-230:
#   i <  D/2: out_i = x_i*cos_i - x_{i+D/2}*sin_i
#   i >= D/2: out_i = x_i*cos_i + x_{i-D/2}*sin_i
# x: [B, H, S, D]; cos/sin: [S, D] (row s used for position s).
# ---------------------------------------------------------------------------
def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    xf = _f32(x)
    d = xf.shape[-1]
    h = d // 2
    rot = torch.cat([-xf[..., h:], xf[..., :h]], dim=-1)
    return (xf * _f32(cos) + rot * _f32(sin)).to(x.dtype)


def rope_fp16_arith(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """The reference kernel's exact fp16 arithmetic: every __hmul and the
    __hadd round to fp16 (apply_rope.cuh:43-44)."""
    xh = x.detach().cpu().to(torch.float16).float()
    c = cos.detach().cpu().to(torch.float16).float()
    s = sin.detach().cpu().to(torch.float16).float()
    h = xh.shape[-1] // 2
    rot = torch.cat([-xh[..., h:], xh[..., :h]], dim=-1)
    r16 = lambda t: t.to(torch.float16).float()  # noqa: E731
    return r16(r16(xh * c) + r16(rot * s)).to(torch.float16)


def qkrope(q, k, cos, sin):
    """csrc/dlops/qkrope/qkrope.cuh:20-67: rope on q and k with one table."""
    return rope(q, cos, sin), rope(k, cos, sin)


# ---------------------------------------------------------------------------
# Fused Linear + activation -- csrc/activation/fused_gemm.cuh:74-112 (intended
# behaviour; the committed epilogue reads unconverted registers :79-89):
#   acc = fp32 sum of x*W (tensor-op GEMM, W in nn.Linear [N, K] layout)
#   pre = half(alpha*acc + beta*src) with alpha=1, beta=0 (binding.cu:43)
#   out = half(act(float(pre)))       (activation.cuh:26-67, fp32 math)
# The build's optional bias is added to acc before the first rounding.
# ---------------------------------------------------------------------------
def activation(x: torch.Tensor, act: str) -> torch.Tensor:
    if act == "gelu":  # GeluHalf, tanh approximation (activation.cuh:31-39)
        k_alpha = 0.7978845608028654
        return 0.5 * x * (1.0 + torch.tanh(k_alpha * (x + 0.044715 * x * x * x)))
    if act == "silu":  # SiluHalf (activation.cuh:51-53)
        return x / (1.0 + torch.exp(-x))
    if act == "relu":  # ReluHalf (activation.cuh:63-64)
        return torch.clamp_min(x, 0.0)
    if act in (None, "none"):
        return x
    raise ValueError(act)


def linear_act(x: torch.Tensor, w: torch.Tensor, bias=None, act: str = "none") -> torch.Tensor:
    xf = _f32(x).reshape(-1, x.shape[-1])
    acc = xf @ _f32(w).t()
    if bias is not None:
        acc = acc + _f32(bias)
    pre = acc.to(x.dtype).float()
    out = activation(pre, act).to(x.dtype)
    return out.reshape(x.shape[:-1] + (w.shape[0],))


# ---------------------------------------------------------------------------
# GEMV -- csrc/blas/hgemv/hgemv_kernels.cuh:19-67 (y[m] = sum_k A[m,k]*x[k]);
# the build accumulates exact products in fp32 (x: [B, K], W: [N, K]).
# ---------------------------------------------------------------------------
def gemv(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    return (_f32(x) @ _f32(w).t()).to(x.dtype)


def hgemv_cpu(a: np.ndarray, x: np.ndarray) -> np.ndarray:
    """Restatement of the reference's CPU check hgemvCpu
    (csrc/blas/hgemv/hgemv_bench.cpp:10-24): each product a*x is rounded to
    fp16, accumulated in fp32, and the sum stored as fp16."""
    a16 = a.astype(np.float16)
    x16 = x.astype(np.float16)
    prod = (a16.astype(np.float32) * x16.astype(np.float32)[None, :]).astype(np.float16)
    acc = np.zeros(a.shape[0], dtype=np.float32)
    for k in range(a.shape[1]):  # sequential fp32 accumulation, as the loop at :19-21
        acc += prod[:, k].astype(np.float32)
    return acc.astype(np.float16)


# ---------------------------------------------------------------------------
# Attention -- the flash_attn_func contract used at torchpp/attention/gqa.py:128
# and swa.py:85-89, restated with the eager formula of
# examples/TTS/dia/og_model.py:289-297:
#   S = Q K^T * scale (scale = 1/sqrt(D) unless given), fp32 softmax, O = P V.
#   GQA: query head h reads kv head h // (Hq/Hkv) (= repeat_interleave,
#   gqa.py:120-121).
#   Causal is aligned bottom-right: key j is visible to query i iff
#   j <= i + (Sk - Sq); a window (left, right) keeps
#   i + Sk - Sq - left <= j <= i + Sk - Sq + right (left/right < 0 = unbounded).
#   A query with no visible key gets O = 0.
# Layout: q [B, Sq, Hq, D], k/v [B, Sk, Hkv, D] (flash-attn layout).
# ---------------------------------------------------------------------------
def _mask(sq, sk, causal, window, device="cpu"):
    left, right = window
    if causal:
        right = 0
    i = torch.arange(sq, device=device)[:, None]
    j = torch.arange(sk, device=device)[None, :]
    off = sk - sq
    keep = torch.ones(sq, sk, dtype=torch.bool, device=device)
    if right >= 0:
        keep &= j <= i + off + right
    if left >= 0:
        keep &= j >= i + off - left
    return keep


def attention(q, k, v, causal=False, window=(-1, -1), scale=None, out_dtype=None):
    qf, kf, vf = _f32(q), _f32(k), _f32(v)
    b, sq, hq, d = qf.shape
    sk, hkv = kf.shape[1], kf.shape[2]
    g = hq // hkv
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    kf = kf.repeat_interleave(g, dim=2)
    vf = vf.repeat_interleave(g, dim=2)
    s = torch.einsum("bqhd,bkhd->bhqk", qf, kf) * scale
    keep = _mask(sq, sk, causal, window)
    s = s.masked_fill(~keep, float("-inf"))
    p = torch.softmax(s, dim=-1)
    p = torch.nan_to_num(p, nan=0.0)  # fully-masked rows -> 0
    o = torch.einsum("bhqk,bkhd->bqhd", p, vf)
    return o.to(out_dtype or q.dtype)


def attention_fp64_loops(q, k, v, causal=False, window=(-1, -1), scale=None):
    """Brute force in fp64 with explicit loops (small shapes only)."""
    qd = q.detach().cpu().double().numpy()
    kd = k.detach().cpu().double().numpy()
    vd = v.detach().cpu().double().numpy()
    b, sq, hq, d = qd.shape
    sk, hkv = kd.shape[1], kd.shape[2]
    g = hq // hkv
    sc = 1.0 / math.sqrt(d) if scale is None else scale
    left, right = window
    if causal:
        right = 0
    out = np.zeros((b, sq, hq, d))
    for bi in range(b):
        for h in range(hq):
            hk = h // g
            for i in range(sq):
                scores = []
                for j in range(sk):
                    rel = j - (i + sk - sq)
                    if right >= 0 and rel > right:
                        continue
                    if left >= 0 and rel < -left:
                        continue
                    scores.append((j, sum(qd[bi, i, h, t] * kd[bi, j, hk, t] for t in range(d)) * sc))
                if not scores:
                    continue
                m = max(s for _, s in scores)
                den = sum(math.exp(s - m) for _, s in scores)
                for j, s in scores:
                    out[bi, i, h] += math.exp(s - m) / den * vd[bi, j, hk]
    return torch.from_numpy(out)


def decode_attention(q, k_cache, v_cache, seqlens, scale=None, window_left=-1,
                     out_dtype=None):
    """One query per sequence against its cache prefix [0, L_b):
    q [B, 1, Hq, D]; caches [B, Hkv, Lmax, D] (KVCache layout,
    torchpp/llmops/kvcache.py:39-48 with batch B). Equals `attention` with
    Sq=1, causal, on the prefix."""
    outs = []
    for bi in range(q.shape[0]):
        L = int(seqlens[bi])
        kb = k_cache[bi : bi + 1, :, :L].transpose(1, 2)
        vb = v_cache[bi : bi + 1, :, :L].transpose(1, 2)
        outs.append(attention(q[bi : bi + 1], kb, vb, causal=True,
                              window=(window_left, 0), scale=scale,
                              out_dtype=out_dtype or q.dtype))
    return torch.cat(outs, dim=0)
