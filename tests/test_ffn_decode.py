"""GPU parity of the one-launch decode FFN (tpp_ffn_decode: RMSNorm + SwiGLU
gate/up + down + residual add, the down projection split over the 8 XCDs)
against the oracle composition of the reference block
(examples/LLM/fastqwen3.py:113-116 with the intended SwiGLU) and against the
two-launch GEMV path it replaces."""
import pytest
import torch

import oracle
from tests.conftest import close
from torchplusplus_amd._native import ext
from torchplusplus_amd.dlops.linear import interleave_gate_up

pytestmark = pytest.mark.gpu
C = ext()


def _weights(E, I, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    wg = (0.02 * torch.randn(I, E, generator=g)).to(dtype)
    wu = (0.02 * torch.randn(I, E, generator=g)).to(dtype)
    wd = (0.02 * torch.randn(E, I, generator=g)).to(dtype)
    nw = (1 + 0.1 * torch.randn(E, generator=g)).to(dtype)
    return wg, wu, wd, nw


def _oracle(resid, nw, wg, wu, wd):
    """residual + down(silu(gate(x)) * up(x)), x = RMSNorm(residual) * nw,
    with the eager rounding points (each op's output in the model dtype)."""
    dt = resid.dtype
    x = oracle.rmsnorm(resid, nw, 1e-6)
    gt = oracle.gemv(x, wg).float()
    ut = oracle.gemv(x, wu).float()
    h = (oracle.activation(gt, "silu").to(dt).float() * ut).to(dt)
    d = oracle.gemv(h, wd).float()
    return (resid.float() + d).to(dt)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,I", [(8, 3072), (1, 3072), (3, 3072), (16, 3072), (8, 1024), (5, 4096),
                                 (8, 2048)])
def test_ffn_decode_matches_oracle_and_two_launches(dev, dtype, B, I):
    E = 1024
    wg, wu, wd, nw = _weights(E, I, dtype, seed=B + I)
    resid = torch.randn(B, 1, E, generator=torch.Generator().manual_seed(7)).to(dtype)
    want = _oracle(resid.view(B, E), nw, wg, wu, wd).view(B, 1, E)
    w_gu = interleave_gate_up(wg.to(dev), wu.to(dev))
    r1 = resid.to(dev)
    C.ffn_decode(r1, nw.to(dev), 1e-6, w_gu, wd.to(dev))
    r2 = resid.to(dev)
    h = C.gemv_swiglu(r2, w_gu, nw.to(dev), 1e-6)
    C.gemv_fused(h, wd.to(dev), None, 1e-6, r2)
    torch.cuda.synchronize()
    assert C.ffn_decode_sync_errors(r1) == 0
    close(r1, want, what=f"ffn_decode B={B} I={I}")
    close(r1, r2, atol=1e-2, rtol=1e-2, what="ffn_decode vs gemv_swiglu + down")


def test_ffn_decode_unfused_shape(dev):
    """E != 1024: the entry point takes the two-launch path."""
    B, E, I = 4, 512, 1536
    wg, wu, wd, nw = _weights(E, I, torch.bfloat16, seed=3)
    resid = torch.randn(B, E, generator=torch.Generator().manual_seed(4)).bfloat16()
    r = resid.to(dev)
    C.ffn_decode(r, nw.to(dev), 1e-6, interleave_gate_up(wg.to(dev), wu.to(dev)), wd.to(dev))
    close(r, _oracle(resid, nw, wg, wu, wd), what="ffn_decode unfused")


def test_ffn_decode_graph_replays_over_layers(dev):
    """28 launches over distinct weights captured in one graph (as the decode
    step does), replayed three times with eager work in between: every
    replay equals the eager result (the sync counters are back at zero after
    every launch), and no launch gave up waiting."""
    B, E, I, L = 8, 1024, 3072, 28
    g = torch.Generator(device=dev).manual_seed(11)
    layers = []
    for _ in range(L):
        wg = (0.02 * torch.randn(I, E, generator=g, device=dev)).bfloat16()
        wu = (0.02 * torch.randn(I, E, generator=g, device=dev)).bfloat16()
        wd = (0.02 * torch.randn(E, I, generator=g, device=dev)).bfloat16()
        nw = (1 + 0.1 * torch.randn(E, generator=g, device=dev)).bfloat16()
        layers.append((nw, interleave_gate_up(wg, wu), wd))
    start = torch.randn(B, 1, E, generator=g, device=dev).bfloat16()
    resid = start.clone()

    def run():
        for nw, w_gu, wd in layers:
            C.ffn_decode(resid, nw, 1e-6, w_gu, wd)

    run()
    want = resid.clone()
    resid.copy_(start)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    assert torch.equal(resid, want), "eager runs differ"
    graph = torch.cuda.CUDAGraph()
    resid.copy_(start)
    with torch.cuda.graph(graph):
        run()
    for rep in range(3):
        resid.copy_(start)
        graph.replay()
        _ = torch.randn(1000, device=dev).sum()
        torch.cuda.synchronize()
        assert torch.equal(resid, want), f"replay {rep} differs from eager"
    assert C.ffn_decode_sync_errors(resid) == 0
