"""Device preparation and capture rules of the kernels that exchange data
inside one XCD (decode attention's in-kernel split merge, the one-launch
decode FFN): the placement probe entry point, its refusal during stream
capture, and the refusal to create a counter-holding workspace inside a
capture (its zero fill would only exist once the graph ran)."""
import ctypes

import pytest
import torch

import oracle
import torchplusplus_amd
from tests.conftest import close
from torchplusplus_amd._native import lib
from torchplusplus_amd.attention import decode_attention

pytestmark = pytest.mark.gpu


def test_prepare_device_reports_xcd_placement(dev):
    info = torchplusplus_amd.prepare_device(dev)
    assert info["cu_count"] > 0
    props = torch.cuda.get_device_properties(dev)
    if "gfx950" in getattr(props, "gcnArchName", "") and info["cu_count"] == 256:
        assert info["xcd_local"], "MI355X: workgroups with equal id % 8 must share an XCD"
    assert torchplusplus_amd.prepare_device(dev) == info  # cached, same answer


def test_prepare_device_refused_during_capture(dev):
    torchplusplus_amd.prepare_device(dev)
    L = lib()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    rcs = []
    with torch.cuda.graph(g, stream=s):
        rcs.append(L.tpp_prepare_device(ctypes.c_void_p(s.cuda_stream), None, None))
    assert rcs == [-1]
    assert b"captured" in L.tpp_last_error_string()


def test_decode_workspace_not_created_inside_capture(dev):
    """A decode call whose workspace is larger than the binding holds, made
    inside a capture, is refused with a message (no graph node fills it).
    The shape is about the largest split plan there is (511 pairs, 2 splits
    of G = 8 heads: ~5.3 MB), above every other test's. An eager call
    afterwards still works."""
    f = lib().tpp_attn_decode_workspace_size
    f.restype = ctypes.c_size_t
    B, Hq, Hkv, D, L = 511, 8, 1, 128, 256
    assert f(*(ctypes.c_int64(v) for v in (B, Hq, Hkv, D, L))) > 5_200_000
    gen = torch.Generator().manual_seed(3)
    qd = torch.randn(B, 1, Hq, D, generator=gen).bfloat16().to(dev)
    kd = torch.randn(B, Hkv, L, D, generator=gen).bfloat16().to(dev)
    vd = torch.randn(B, Hkv, L, D, generator=gen).bfloat16().to(dev)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="capture"):
        with torch.cuda.graph(g, stream=s):
            decode_attention(qd, kd, vd)
    torch.cuda.synchronize()
    q, kc, vc = (t[:4].cpu() for t in (qd, kd, vd))
    o = decode_attention(qd[:4], kd[:4], vd[:4])
    close(o, oracle.decode_attention(q, kc, vc, [L] * 4), what="eager decode after the refused capture")
