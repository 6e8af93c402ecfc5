"""Alias module: examples/LLM/fastqwen3.py:7 imports
`torchpp.dlops.fused_linear.LinearSILU`, which the reference never shipped."""
from torchplusplus_amd.dlops.linear import LinearGELU, LinearRELU, LinearSILU  # noqa: F401
