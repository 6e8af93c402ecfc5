"""tpp_attn_decode_noalloc (no workspace: a static device array) against
tpp_attn_decode (caller workspace), through the C ABI: two calls in a row,
the second with a smaller input and the other merge mode, outputs
bit-identical; a shape whose plan exceeds the static array is rejected
before anything is launched."""
import ctypes

import pytest
import torch

import oracle
from tests.conftest import close
from torchplusplus_amd._native import lib

pytestmark = pytest.mark.gpu

TPP_BF16 = 1


def _s3(*v):
    return (ctypes.c_int64 * 3)(*v)


def _call(name, q, kc, vc, o, lens, ws=None):
    f = getattr(lib(), name)
    B, _, Hq, D = q.shape
    Hkv, Lmax = kc.shape[1], kc.shape[2]
    P = ctypes.c_void_p
    args = [P(q.data_ptr()), P(kc.data_ptr()), P(vc.data_ptr()), P(o.data_ptr()),
            _s3(q.stride(0), q.stride(1), q.stride(2)),
            _s3(kc.stride(0), kc.stride(2), kc.stride(1)),
            _s3(vc.stride(0), vc.stride(2), vc.stride(1)),
            _s3(o.stride(0), o.stride(1), o.stride(2)),
            P(lens.data_ptr()), ctypes.c_int64(B), ctypes.c_int64(Hq), ctypes.c_int64(Hkv),
            ctypes.c_int64(D), ctypes.c_int64(Lmax), ctypes.c_float(0.0), ctypes.c_int(-1),
            ctypes.c_int(TPP_BF16)]
    if ws is not None:
        args += [P(ws.data_ptr()), ctypes.c_size_t(ws.numel() * 4)]
    args.append(P(torch.cuda.current_stream().cuda_stream))
    return f(*args)


def _case(dev, B, Hq, Hkv, D, L, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(B, 1, Hq, D, device=dev, generator=g).bfloat16()
    kc = torch.randn(B, Hkv, L, D, device=dev, generator=g).bfloat16()
    vc = torch.randn(B, Hkv, L, D, device=dev, generator=g).bfloat16()
    lens = torch.randint(1, L + 1, (B,), device=dev, generator=g, dtype=torch.int32)
    lens[0] = L
    return q, kc, vc, lens


def _ws_bytes(B, Hq, Hkv, D, L):
    f = lib().tpp_attn_decode_workspace_size
    f.restype = ctypes.c_size_t
    return f(*(ctypes.c_int64(v) for v in (B, Hq, Hkv, D, L)))


def test_noalloc_decode_matches_workspace_entry(dev):
    # model shape (64 pairs: splits merged in-kernel), then a smaller one
    # (6 pairs: merge kernel); each against the workspace entry point
    for i, (B, Hq, Hkv, D, L) in enumerate([(8, 16, 8, 128, 2058), (3, 8, 2, 64, 500)]):
        q, kc, vc, lens = _case(dev, B, Hq, Hkv, D, L, seed=i)
        ws = torch.zeros((_ws_bytes(B, Hq, Hkv, D, L) + 3) // 4, device=dev)
        o_ref = torch.empty_like(q)
        o_na = torch.full_like(q, float("nan"))
        assert _call("tpp_attn_decode", q, kc, vc, o_ref, lens, ws) == 0, \
            lib().tpp_last_error_string()
        assert _call("tpp_attn_decode_noalloc", q, kc, vc, o_na, lens) == 0, \
            lib().tpp_last_error_string()
        torch.cuda.synchronize()
        assert torch.equal(o_na, o_ref), f"case {i}: noalloc output differs"
        if i == 1:
            close(o_na, oracle.decode_attention(q.cpu(), kc.cpu(), vc.cpu(), lens.cpu().tolist()),
                  what="noalloc vs oracle")


def test_noalloc_rejects_plans_beyond_the_static_array(dev):
    B, Hq, Hkv, D, L = 125, 32, 4, 128, 256
    assert _ws_bytes(B, Hq, Hkv, D, L) > 4 * 1024 * 1024
    q, kc, vc, lens = _case(dev, B, Hq, Hkv, D, L, seed=3)
    o = torch.empty_like(q)
    assert _call("tpp_attn_decode_noalloc", q, kc, vc, o, lens) == -2
    assert b"static" in lib().tpp_last_error_string()
