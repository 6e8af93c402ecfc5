"""Attention modules mirroring torchpp.attention (reference:
torchpp/attention/__init__.py:1-6). `QKV` (xattention.py) is an unfinished
helper in the reference and is not provided."""
from torchplusplus_amd.attention.ca import CrossAttention  # noqa: F401
from torchplusplus_amd.attention.flash import decode_attention, flash_attn_func  # noqa: F401
from torchplusplus_amd.attention.gqa import GroupedQueryAttention  # noqa: F401
from torchplusplus_amd.attention.mha import MultiHeadAttention  # noqa: F401
from torchplusplus_amd.attention.mqa import MultiQueryAttention  # noqa: F401
from torchplusplus_amd.attention.swa import SlidingWindowAttention  # noqa: F401
