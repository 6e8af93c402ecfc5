"""GPU parity: fused QK-RMSNorm + RoPE + KV-cache append."""
import pytest
import torch

import oracle
from tests.conftest import close
from torchplusplus_amd._native import ext

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,S,start", [(2, 7, [0, 3]), (8, 1, [2048, 17, 0, 5, 2099, 2100, 1, 2]), (1, 64, [5])])
@pytest.mark.parametrize("norm", [True, False])
def test_qkv_rope_cache(dev, dtype, B, S, start, norm):
    g = torch.Generator().manual_seed(0)
    Hq, Hkv, D, Lmax, ctx = 4, 2, 128, 2100, 4096
    qkv = torch.randn(B, S, (Hq + 2 * Hkv) * D, generator=g).to(dtype)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(dtype)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(dtype)
    cos, sin = oracle.compute_rope_params(D, 1e6, ctx)
    kc = torch.zeros(B, Hkv, Lmax, D, dtype=dtype)
    vc = torch.zeros(B, Hkv, Lmax, D, dtype=dtype)
    kcd, vcd = kc.to(dev), vc.to(dev)
    qo = torch.empty(B, S, Hq, D, dtype=dtype, device=dev)
    pos = torch.tensor(start, dtype=torch.int32)
    ext().qkv_rope_cache(qkv.to(dev), qo, kcd, vcd, qw.to(dev) if norm else None,
                         kw.to(dev) if norm else None, cos.to(dev), sin.to(dev), pos.to(dev), 1e-6)
    # oracle: split heads, RMSNorm over head_dim, rope at absolute positions, scatter
    x = qkv.view(B, S, Hq + 2 * Hkv, D)
    q, k, v = x[:, :, :Hq], x[:, :, Hq:Hq + Hkv], x[:, :, Hq + Hkv:]
    if norm:
        q = oracle.rmsnorm(q, qw, 1e-6)
        k = oracle.rmsnorm(k, kw, 1e-6)
    for b in range(B):
        p0 = start[b]
        sl = slice(p0, p0 + S)
        close(qo[b].cpu(), oracle.rope(q[b].transpose(0, 1), cos[sl], sin[sl]).transpose(0, 1), what="q")
        if p0 + S <= Lmax:
            close(kcd[b, :, sl].cpu(), oracle.rope(k[b].transpose(0, 1), cos[sl], sin[sl]), what="k cache")
            assert torch.equal(vcd[b, :, sl].cpu(), v[b].transpose(0, 1)), "v cache must be a copy"
        # nothing outside the written window
        mask = torch.ones(Lmax, dtype=torch.bool)
        mask[p0:p0 + S] = False
        assert bool((kcd[b][:, mask] == 0).all()) and bool((vcd[b][:, mask] == 0).all())
