"""Drop-in for the compiled module `qkropeApplyFunction`
(reference: csrc/dlops/qkrope/qkrope_binding.cu:94-101)."""
from torchplusplus_amd._native import ext as _ext

qkrope_apply_cuda = _ext().qkrope_apply_cuda
