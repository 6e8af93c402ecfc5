"""Drop-in for the compiled module `rmsnormFused`
(reference: csrc/dlops/rmsnorm/rmsnorm_binding.cu:70-73)."""
from torchplusplus_amd._native import ext as _ext

rmsnormFused = _ext().rmsnormFused
