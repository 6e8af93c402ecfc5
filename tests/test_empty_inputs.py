"""Empty inputs (zero rows, tokens or sequences) through the binding."""
import pytest
import torch

import oracle
from tests.conftest import close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("op", ["rmsnorm", "layernorm", "linear", "linear_silu", "rope",
                                "prefill_sq0", "prefill_b0", "decode_b0"])
def test_empty_inputs_raise_like_the_reference(dev, op):
    """Zero rows / tokens / sequences are rejected with a RuntimeError, as
    the reference rejects them (rmsnorm_binding.cu:43 "invalid shapes"; its
    other kernels fail their zero-block launch), and nothing is launched: the
    C ABI returns before any launch for a zero size and the binding raises
    on its error code. The device stays usable afterwards."""
    from torchplusplus_amd._native import ext
    from torchplusplus_amd.attention.flash import flash_attn_func
    C = ext()
    h = torch.float16
    w = torch.ones(1024, dtype=h, device=dev)
    W = torch.randn(64, 1024, dtype=h, device=dev)
    e = lambda *s: torch.empty(*s, dtype=h, device=dev)
    cos, sin = (t.to(dev) for t in oracle.compute_rope_params(64, 1e4, 16))
    k = torch.randn(2, 5, 2, 128, dtype=h, device=dev)
    calls = {
        "rmsnorm": lambda: C.rmsnormFused(e(0, 1024), w, 1e-6),
        "layernorm": lambda: C.applyLayernorm(e(0, 1024), w, 1e-6, None),
        "linear": lambda: C.linear(e(0, 1024), W, None, 0),
        "linear_silu": lambda: C.LinearSilu(e(0, 1024), W),
        "rope": lambda: C.rope_apply_cuda(e(1, 4, 0, 64), cos[:0], sin[:0]),
        "prefill_sq0": lambda: flash_attn_func(e(2, 0, 4, 128), k, k, causal=True),
        "prefill_b0": lambda: flash_attn_func(e(0, 3, 4, 128), e(0, 3, 2, 128), e(0, 3, 2, 128)),
        "decode_b0": lambda: C.attn_decode(e(0, 1, 4, 128), e(0, 2, 16, 128), e(0, 2, 16, 128),
                                           None, 0.0, -1, None),
    }
    with pytest.raises(RuntimeError):
        calls[op]()
        torch.cuda.synchronize()
    x = torch.randn(4, 1024, dtype=h, device=dev)
    close(C.rmsnormFused(x, w, 1e-6), oracle.rmsnorm(x.cpu(), w.cpu(), 1e-6), what="after empty call")
