"""Drop-in for the compiled module `ropeApplyFunction`
(reference: csrc/dlops/rope/rope_binding.cu:69-72)."""
from torchplusplus_amd._native import ext as _ext

rope_apply_cuda = _ext().rope_apply_cuda
