"""Drop-in for the compiled module `linearActvationFp16`
(reference: csrc/activation/binding.cu:162-166). Accepts fp16 and bf16 and an
optional bias."""
from torchplusplus_amd._native import ext as _ext

LinearGelu = _ext().LinearGelu
LinearSilu = _ext().LinearSilu
LinearRelu = _ext().LinearRelu
