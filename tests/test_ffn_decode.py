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


def _capi_ffn(lib, resid, nw, w_gu, wd, ws, stream=None):
    import ctypes

    B, E = resid.numel() // resid.shape[-1], resid.shape[-1]
    I = wd.shape[1]
    rc = lib.tpp_ffn_decode(ctypes.c_void_p(resid.data_ptr()), ctypes.c_void_p(nw.data_ptr()),
                            ctypes.c_float(1e-6), ctypes.c_void_p(w_gu.data_ptr()),
                            ctypes.c_void_p(wd.data_ptr()), ctypes.c_int64(B), ctypes.c_int64(E),
                            ctypes.c_int64(I), ctypes.c_int(1), ctypes.c_void_p(ws.data_ptr()),
                            ctypes.c_size_t(ws.numel()),
                            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, lib.tpp_last_error_string()


@pytest.mark.parametrize("B,I", [(8, 3072), (16, 4096), (1, 1024)])
def test_ffn_decode_runs_one_launch_path(dev, B, I):
    """On a 256-CU device whose placement probe holds, tpp_ffn_decode runs the
    one-launch kernel (not the two GEMVs): only that kernel writes the fp32
    per-XCD partials after the h region of the workspace (the two-GEMV path
    touches h only), so a workspace pre-filled with NaN there must hold 8
    finite partials per output after the call; the residual equals the
    binding's result."""
    import ctypes

    import torchplusplus_amd
    from torchplusplus_amd._native import lib

    info = torchplusplus_amd.prepare_device(dev)
    if info["cu_count"] != 256:
        pytest.skip(f"one-launch FFN needs 256 CUs, device has {info['cu_count']}")
    assert info["xcd_local"], "XCD placement probe failed on a 256-CU device"
    L = lib()
    E = 1024
    f = L.tpp_ffn_decode_workspace_size
    f.restype = ctypes.c_size_t
    need = f(ctypes.c_int64(B), ctypes.c_int64(E), ctypes.c_int64(I))
    h_bytes = (B * I * 2 + 255) // 256 * 256
    assert need == 8192 + h_bytes + 8 * B * E * 4
    ws = torch.full((need,), 0xFF, dtype=torch.uint8, device=dev)
    ws[:8192] = 0  # counters start at zero
    wg, wu, wd, nw = _weights(E, I, torch.bfloat16, seed=31 + B)
    w_gu = interleave_gate_up(wg.to(dev), wu.to(dev))
    resid = torch.randn(B, E, generator=torch.Generator().manual_seed(32)).bfloat16().to(dev)
    r1, r2 = resid.clone(), resid.clone()
    _capi_ffn(L, r1, nw.to(dev), w_gu, wd.to(dev), ws)
    C.ffn_decode(r2, nw.to(dev), 1e-6, w_gu, wd.to(dev))
    torch.cuda.synchronize()
    part = ws[8192 + h_bytes:].view(torch.float32).view(8, B, E)
    assert torch.isfinite(part).all(), "partials not written: the two-GEMV path ran"
    assert torch.equal(r1, r2)
    assert int(ws[:8192].view(torch.int32).abs().sum()) == 0, "counters not back at zero"


def test_ffn_decode_sync_error_flag_read_and_clear(dev):
    """The give-up flag is forced from the host (no kernel is made to wait):
    tpp_ffn_decode_sync_errors reports it once, zeroes the counter region
    (left in an unknown state by a launch that gave up) and the flag, and the
    workspace then gives correct results."""
    import ctypes

    from torchplusplus_amd._native import lib

    L = lib()
    B, E, I = 8, 1024, 3072
    f = L.tpp_ffn_decode_workspace_size
    f.restype = ctypes.c_size_t
    ws = torch.zeros(f(ctypes.c_int64(B), ctypes.c_int64(E), ctypes.c_int64(I)), dtype=torch.uint8,
                     device=dev)
    ctr = ws[:8192].view(torch.int32)
    ctr[0] = 5  # an XCD arrival count left behind
    ctr[(2048 + 7 * 128) // 4] = 3  # a chunk count
    ctr[(2048 + 32 * 128) // 4] = 1  # the flag
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = ctypes.c_int(-1)
    assert L.tpp_ffn_decode_sync_errors(ctypes.c_void_p(ws.data_ptr()), ctypes.byref(out), stream) == 0
    assert out.value == 1
    assert int(ctr.abs().sum()) == 0, "counter region not cleared"
    assert L.tpp_ffn_decode_sync_errors(ctypes.c_void_p(ws.data_ptr()), ctypes.byref(out), stream) == 0
    assert out.value == 0
    wg, wu, wd, nw = _weights(E, I, torch.bfloat16, seed=33)
    resid = torch.randn(B, E, generator=torch.Generator().manual_seed(34)).bfloat16()
    r = resid.to(dev)
    _capi_ffn(L, r, nw.to(dev), interleave_gate_up(wg.to(dev), wu.to(dev)), wd.to(dev), ws)
    close(r, _oracle(resid, nw, wg, wu, wd), what="ffn_decode after the flag was cleared")
    # the binding's check covers its own workspaces and reports nothing here
    assert C.ffn_decode_sync_errors(r) == 0
