"""C-ABI and binding host logic (CPU only: no kernel is launched)."""
import ctypes
import os
import re

import pytest
import torch

from torchplusplus_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tpp.h")


def declared_symbols():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(tpp_[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    syms = declared_symbols()
    assert len(syms) >= 7
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, f"not exported: {missing}"


def test_version():
    assert _native.lib().tpp_version() >> 16 == 1


def _p(v=256):
    return ctypes.c_void_p(v)  # never dereferenced: validation fails first


def test_null_pointer_is_rejected():
    lib = _native.lib()
    rc = lib.tpp_rmsnorm(None, _p(), _p(), ctypes.c_int64(4), ctypes.c_int64(8),
                         ctypes.c_int64(8), ctypes.c_int64(8), ctypes.c_float(1e-6),
                         ctypes.c_int(0), None)
    assert rc == -1
    assert b"null" in lib.tpp_last_error_string()


def test_bad_dtype_is_rejected():
    lib = _native.lib()
    rc = lib.tpp_rmsnorm(_p(), _p(), _p(), ctypes.c_int64(4), ctypes.c_int64(8),
                         ctypes.c_int64(8), ctypes.c_int64(8), ctypes.c_float(1e-6),
                         ctypes.c_int(7), None)
    assert rc == -2
    assert b"dtype" in lib.tpp_last_error_string()


def test_bad_stride_is_rejected():
    lib = _native.lib()
    rc = lib.tpp_layernorm(_p(), _p(), None, _p(), ctypes.c_int64(4), ctypes.c_int64(8),
                           ctypes.c_int64(4), ctypes.c_int64(8), ctypes.c_float(1e-6),
                           ctypes.c_int(0), None)
    assert rc == -1
    assert b"stride" in lib.tpp_last_error_string()


def test_binding_rejects_cpu_tensors_like_the_reference():
    C = _native.ext()
    x = torch.randn(4, 8).half()
    w = torch.ones(8).half()
    with pytest.raises(RuntimeError, match="input must be CUDA"):
        C.rmsnormFused(x, w, 1e-6)
    with pytest.raises(RuntimeError, match="Input tensor must be on CUDA"):
        C.applyLayernorm(x, w, 1e-6)


def test_compat_module_names_import():
    import torchplusplus_amd  # noqa: F401  (installs the import hook)
    import rmsnormFused
    import layernormFused

    assert callable(rmsnormFused.rmsnormFused)
    assert callable(layernormFused.applyLayernorm)


def test_torchpp_alias_imports_reference_paths():
    """The reference's import paths (fastqwen3.py:7-11, tests/*.py) resolve."""
    from torchpp.dlops.normalization import LayerNormFused, RmsNormFused  # noqa: F401
    from torchpp.dlops.rope import compute_rope_params, qkrope_apply, rope_apply  # noqa: F401
    from torchpp.dlops.fused_linear import LinearSILU  # noqa: F401
    from torchpp.attention.gqa import GroupedQueryAttention  # noqa: F401
    from torchpp.llmops.kvcache import KVCache
    from torchpp.llmops.llm import LLMInference  # noqa: F401
    import torchplusplus_amd.llmops.kvcache as real

    assert KVCache is real.KVCache


def test_gemm_vendor_switch_returns_previous_setting():
    L = _native.lib()
    prev = L.tpp_gemm_vendor(-1)
    try:
        assert L.tpp_gemm_vendor(0) == prev
        assert L.tpp_gemm_vendor(-1) == 0
        assert L.tpp_gemm_vendor(1) == 0
        assert L.tpp_gemm_vendor(7) == 1
        assert L.tpp_gemm_vendor(-1) == 1
    finally:
        L.tpp_gemm_vendor(prev)
    L.tpp_gemm_vendor_runs.restype = ctypes.c_longlong
    assert L.tpp_gemm_vendor_runs() >= 0
