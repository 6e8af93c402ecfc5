"""GPU parity: RMSNorm / LayerNorm / add+RMSNorm vs the CPU oracle.

Tolerances: fp16/bf16 outputs atol 2e-2 / rtol 1e-2; fp32 statistics 1e-5
relative to an fp64 closed form.
"""
import numpy as np
import pytest
import torch

import oracle
from tests.conftest import close
from torchplusplus_amd.dlops.normalization import LayerNormFused, RmsNormFused
from torchplusplus_amd._native import ext

pytestmark = pytest.mark.gpu

SHAPES = [
    (4096, 1024),   # BASELINE config 1 (wave-per-row, 4 vectors/lane)
    (32 * 128, 512),  # reference tests/rmsnorm_test.py shape
    (777, 128),     # QK-norm width: 4 rows per wave (16-lane DPP rows)
    (5, 4096),      # 16 vectors/lane path
    (3, 1023),      # odd N: generic block-per-row path (reference handles odd N)
    (2, 12288),     # N > 8192: generic path
    (1, 8),
]


def _inputs(m, n, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, n, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(n, generator=g)).to(dtype)
    return x, w


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m,n", SHAPES)
def test_rmsnorm_parity(dev, m, n, dtype):
    x, w = _inputs(m, n, dtype)
    y = ext().rmsnormFused(x.to(dev), w.to(dev), 1e-6)
    close(y, oracle.rmsnorm(x, w, 1e-6), what=f"rmsnorm {m}x{n} {dtype}")


@pytest.mark.parametrize("m,n", [(4096, 1024), (777, 128), (3, 1023)])
def test_rmsnorm_stats_fp32(dev, m, n):
    x, _ = _inputs(m, n, torch.float16, seed=1)
    inv = ext().rmsnorm_stats(x.to(dev), 1e-6).cpu().double().numpy()
    xd = x.double().numpy()
    ref = 1 / np.sqrt((xd * xd).mean(-1) + 1e-6)
    assert np.max(np.abs(inv / ref - 1)) < 1e-5


def test_rmsnorm_module_3d_noncontiguous(dev):
    g = torch.Generator().manual_seed(2)
    x = torch.randn(32, 128, 512, generator=g).half()
    mod = RmsNormFused(512, eps=1e-6, device=dev)
    with torch.no_grad():
        mod.weight.copy_((1 + 0.1 * torch.randn(512, generator=g)).half())
    xt = x.to(dev).transpose(0, 1)  # non-contiguous: made contiguous like the reference
    y = mod(xt)
    assert y.shape == xt.shape
    close(y, oracle.rmsnorm(x.transpose(0, 1), mod.weight.detach().cpu(), 1e-6), what="rmsnorm module")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m,n", [(4096, 1024), (64, 128), (3, 1023)])
def test_add_rmsnorm_parity(dev, m, n, dtype):
    x, w = _inputs(m, n, dtype, seed=3)
    r, _ = _inputs(m, n, dtype, seed=4)
    rd = r.to(dev)
    y = ext().add_rmsnorm(x.to(dev), rd, w.to(dev), 1e-6)
    ey, eh = oracle.add_rmsnorm(x, r, w, 1e-6)
    assert torch.equal(rd.cpu(), eh), "residual sum must be bit-exact"
    close(y, ey, what="add_rmsnorm")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m,n", [(4096, 1024), (32 * 128, 512), (100, 128), (3, 1023), (2, 12288)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_layernorm_parity(dev, m, n, dtype, with_bias):
    x, w = _inputs(m, n, dtype, seed=5)
    x = x + 0.5
    b = (0.1 * torch.randn(n, generator=torch.Generator().manual_seed(6))).to(dtype)
    y = ext().applyLayernorm(x.to(dev), w.to(dev), 1e-6, b.to(dev) if with_bias else None)
    close(y, oracle.layernorm(x, w, 1e-6, b if with_bias else None), what="layernorm")


@pytest.mark.parametrize("m,n", [(4096, 1024), (100, 128), (3, 1023)])
def test_layernorm_stats_fp32(dev, m, n):
    x, _ = _inputs(m, n, torch.float16, seed=7)
    mean, rstd = ext().layernorm_stats(x.to(dev), 1e-6)
    xd = x.double().numpy()
    assert np.max(np.abs(mean.cpu().double().numpy() - xd.mean(-1))) < 1e-5
    assert np.max(np.abs(rstd.cpu().double().numpy() * np.sqrt(xd.var(-1) + 1e-6) - 1)) < 1e-5


def test_layernorm_module_reference_shape(dev):
    g = torch.Generator().manual_seed(8)
    x = torch.randn(32, 128, 512, generator=g).half()
    mod = LayerNormFused(512, eps=1e-6, device=dev)
    y = mod(x.to(dev))
    ln = torch.nn.LayerNorm(512, eps=1e-6)
    with torch.no_grad():
        ln.bias.zero_()
        ref = ln(x.float()).half()
    assert (y.cpu().float() - ref.float()).abs().max() < 1e-2  # tests/layernorm_test.py:34
