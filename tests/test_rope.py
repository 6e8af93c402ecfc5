"""GPU parity: RoPE (rope_apply / qkrope_apply / in-place) vs the CPU oracle."""
import pytest
import torch

import oracle
from tests.conftest import close
from torchplusplus_amd.dlops import rope as R

pytestmark = pytest.mark.gpu


def _x(shape, dtype, seed):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("cs_dtype", [torch.float16, torch.float32, torch.bfloat16])
def test_rope_baseline_config(dev, dtype, cs_dtype):
    """Q [1,16,2048,128], K [1,8,2048,128], theta 1e6."""
    q = _x((1, 16, 2048, 128), dtype, 0)
    k = _x((1, 8, 2048, 128), dtype, 1)
    cos, sin = oracle.compute_rope_params(128, 1e6, 2048, out_dtype=cs_dtype)
    qo, ko = R.qkrope_apply(q.to(dev), k.to(dev), cos.to(dev), sin.to(dev))
    eq, ek = oracle.qkrope(q, k, cos, sin)
    close(qo, eq, what="q")
    close(ko, ek, what="k")


def test_rope_matches_reference_fp16_arith(dev):
    """tests/rope_test.py data (U[0,1), B1 H16 S256 D128, theta 1e6) against the
    reference kernel's own fp16 arithmetic."""
    x = torch.rand(1, 16, 256, 128, generator=torch.Generator().manual_seed(2)).half()
    cos, sin = oracle.compute_rope_params(128, 1e6, 256)
    y = R.rope_apply(x.to(dev), cos.to(dev), sin.to(dev))
    close(y, oracle.rope_fp16_arith(x, cos, sin), what="rope vs fp16 arith")


@pytest.mark.parametrize("d", [64, 128, 96, 6])
def test_rope_head_dims(dev, d):
    """D % 16 == 0 uses the 128-bit path; 96 and 6 exercise the scalar path."""
    x = _x((2, 3, 17, d), torch.bfloat16, 3)
    cos, sin = oracle.compute_rope_params(d, 1e4, 17)
    y = R.rope_apply(x.to(dev), cos.to(dev), sin.to(dev))
    close(y, oracle.rope(x, cos, sin), what=f"rope d={d}")


def test_rope_inplace_and_position_slice(dev):
    """Decode-style use (gqa.py:108-112): the table rows for positions p..p+S."""
    x = _x((4, 8, 3, 128), torch.float16, 4)
    cos, sin = oracle.compute_rope_params(128, 1e6, 4096)
    p = 2049
    xd = x.to(dev)
    ptr = xd.data_ptr()
    out = R.rope_apply_(xd, cos.to(dev)[p:p + 3], sin.to(dev)[p:p + 3])
    assert out.data_ptr() == ptr
    close(xd, oracle.rope(x, cos[p:p + 3], sin[p:p + 3]), what="in place")


def test_rope_compute_params_on_device_matches_oracle(dev):
    cos, sin = R.compute_rope_params(128, 1e6, 2048, device=dev)
    ec, es = oracle.compute_rope_params(128, 1e6, 2048)
    assert (cos.cpu().float() - ec.float()).abs().max() <= 1e-3
    assert (sin.cpu().float() - es.float()).abs().max() <= 1e-3


def test_rope_params_on_device_match_golden_rows(dev):
    """The on-device tables against the committed fp16 bit patterns
    (tests/golden/rope_params_d128_t1e6_s2048.json). The GPU's fp32
    theta**(-2j/D) may differ from the CPU's in the last bits; each fp32 ulp
    of it moves the angle pos * inv_freq by up to ~pos * 2^-22 (sin and cos
    have slope <= 1). The bound allows 4 such ulps plus one fp16 spacing of
    rounding; row 0 (angle 0) must be exact."""
    import json
    import os

    import numpy as np

    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                           "rope_params_d128_t1e6_s2048.json")) as f:
        fx = json.load(f)
    rows = torch.tensor(fx["rows"], dtype=torch.float32)
    cos, sin = R.compute_rope_params(128, 1e6, 2048, device=dev)
    for t, key in [(cos, "cos"), (sin, "sin")]:
        got = t.cpu()[fx["rows"]]
        want = torch.from_numpy(np.array(fx[key + "_rows_u16"], dtype=np.uint16).view(np.float16))
        # fp16 spacing at |want| (2^(e-11) for |want| = m 2^e, m in [0.5, 1))
        ulp = torch.ldexp(torch.ones(want.shape), torch.frexp(want.float().abs().clamp_min(2.0 ** -14)).exponent - 11)
        bound = ulp + rows[:, None] * 2.0 ** -20
        assert ((got.float() - want.float()).abs() <= bound).all(), key
        assert torch.equal(got[0], want[0]), key


def test_rope_rejects_bad_shapes(dev):
    x = torch.zeros(1, 2, 4, 8, dtype=torch.float16, device=dev)
    cos = torch.zeros(5, 8, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="cos_cache shape mismatch"):
        R.rope_apply(x, cos, cos)
    with pytest.raises(RuntimeError, match="must be 4D"):
        R.rope_apply(x[0], cos[:4], cos[:4])
