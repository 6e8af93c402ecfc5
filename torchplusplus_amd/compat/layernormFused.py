"""Drop-in for the compiled module `layernormFused`
(reference: csrc/dlops/layernorm/layernorm_binding.cu:45-47)."""
from torchplusplus_amd._native import ext as _ext

applyLayernorm = _ext().applyLayernorm
