"""Loader for the in-tree native build.

The product path has no CPU fallback: if the gfx950 library or its torch
binding is missing, importing an op raises ImportError naming the build
command, instead of silently running some other implementation.
"""
from __future__ import annotations

import ctypes
import glob
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libtorchpp_hip.so")

_C = None
_LIB = None


def _missing(what: str, err: Exception | None = None) -> ImportError:
    msg = (
        f"torchplusplus_amd: {what} is not built. Run `python -m torchplusplus_amd.build` "
        f"(or __graft_entry__.build()) first."
    )
    if err is not None:
        msg += f" ({type(err).__name__}: {err})"
    return ImportError(msg)


def ext():
    """The torch extension module `torchplusplus_amd._C`."""
    global _C
    if _C is None:
        if not glob.glob(os.path.join(PKG_DIR, "_C*.so")):
            raise _missing("the torch extension _C")
        import torch  # noqa: F401  (loads libtorch before the binding)

        try:
            from . import _C as mod  # type: ignore[attr-defined]
        except ImportError as e:  # pragma: no cover - depends on the build
            raise _missing("the torch extension _C", e) from e
        _C = mod
    return _C


def lib() -> ctypes.CDLL:
    """The C-ABI library libtorchpp_hip.so loaded with ctypes."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise _missing("libtorchpp_hip.so")
        _LIB = ctypes.CDLL(LIB_PATH)
        _LIB.tpp_last_error_string.restype = ctypes.c_char_p
    return _LIB
