"""torchplusplus_amd -- gfx950 (MI355X) implementation of torchpp's
transformer-inference kernel set.

Sub-packages mirror the reference's Python API (/root/reference/torchpp):
  dlops      RmsNormFused, LayerNormFused, rope_apply, qkrope_apply,
             compute_rope_params, LinearGELU, LinearSILU
  attention  GroupedQueryAttention, SlidingWindowAttention, MultiHeadAttention,
             MultiQueryAttention, CrossAttention, flash_attn_func
  llmops     KVCache, LLMInference
The top-level package `torchpp` (repo root) aliases this one, and the
reference's compiled module names (rmsnormFused, layernormFused,
ropeApplyFunction, qkropeApplyFunction, linearActvationFp16) are importable
after `import torchplusplus_amd`.
"""
from __future__ import annotations

import importlib.util
import os
import sys

__version__ = "0.1.0"

_COMPAT_MODULES = (
    "rmsnormFused",
    "layernormFused",
    "ropeApplyFunction",
    "qkropeApplyFunction",
    "linearActvationFp16",
)


class _CompatFinder:
    """Import hook: `import rmsnormFused` -> torchplusplus_amd.compat.rmsnormFused."""

    @classmethod
    def find_spec(cls, name, path=None, target=None):
        if name in _COMPAT_MODULES:
            loc = os.path.join(os.path.dirname(__file__), "compat", name + ".py")
            return importlib.util.spec_from_file_location(name, loc)
        return None


def _install_compat() -> None:
    if _CompatFinder not in sys.meta_path:
        sys.meta_path.append(_CompatFinder)


_install_compat()


def prepare_device(device=None) -> dict:
    """One-time checks of a GPU for the kernels that exchange data inside one
    XCD (the decode attention's in-kernel split merge, the one-launch decode
    FFN): a workgroup placement probe and the CU count. Synchronises the
    device's current stream; call it before capturing a HIP graph (a first
    call of those kernels inside a capture cannot probe and takes their
    two-launch paths). Returns {"xcd_local": bool, "cu_count": int}."""
    import torch

    from torchplusplus_amd._native import ext

    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    xcd, cus = ext().prepare_device(torch.empty(0, device=dev))
    return {"xcd_local": bool(xcd), "cu_count": int(cus)}
