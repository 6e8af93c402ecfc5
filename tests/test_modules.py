"""GPU parity of the attention modules (MultiHeadAttention,
SlidingWindowAttention, MultiQueryAttention, CrossAttention,
GroupedQueryAttention with and without a KV cache) against the module oracle
(oracle/modules.py), in fp16 and bf16, at the north-star tolerance."""
import math

import pytest
import torch

import oracle
from oracle import modules as om
from tests.conftest import close
from torchplusplus_amd.attention import (CrossAttention, GroupedQueryAttention,
                                         MultiHeadAttention, MultiQueryAttention,
                                         SlidingWindowAttention)
from torchplusplus_amd.llmops.kvcache import KVCache

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16]


def _randomize(mod, seed):
    """Weights ~ N(0, 1/fan_in) (outputs of order 1), norm weights 1 + N(0, 0.1),
    biases N(0, 0.1); returns the CPU state dict the oracle reads."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for n, p in mod.named_parameters():
            if "norm" in n:
                v = 1 + 0.1 * torch.randn(p.shape, generator=g)
            elif n.endswith("bias"):
                v = 0.1 * torch.randn(p.shape, generator=g)
            else:
                v = torch.randn(p.shape, generator=g) / math.sqrt(p.shape[-1])
            p.copy_(v.to(p.dtype))
    return {k: v.detach().cpu() for k, v in mod.state_dict().items()}


def _x(shape, dtype, seed):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)).to(dtype)


def _tables(D, S, dev):
    c, s = oracle.compute_rope_params(D, 1e6, S)
    return c, s, c.to(dev), s.to(dev)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("E,H,S", [(512, 4, 77), (256, 4, 130)])
def test_multi_head_attention(dev, dtype, E, H, S):
    mod = MultiHeadAttention(E, H, dtype=dtype, device=dev)
    p = _randomize(mod, 1)
    x = _x((2, S, E), dtype, 2)
    c, s, cd, sd = _tables(E // H, S, dev)
    with torch.no_grad():
        got = mod(x.to(dev), cd, sd)
    close(got, om.mha(x, p, c, s, H), what="MultiHeadAttention")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("window", [1, 16, 200])  # self only, inside, wider than S
def test_sliding_window_attention(dev, dtype, window):
    E, H, S = 512, 4, 97
    mod = SlidingWindowAttention(window, E, H, dtype=dtype, device=dev)
    p = _randomize(mod, 3)
    x = _x((2, S, E), dtype, 4)
    c, s, cd, sd = _tables(E // H, S, dev)
    with torch.no_grad():
        got = mod(x.to(dev), cd, sd)
    close(got, om.mha(x, p, c, s, H, window_size=window), what=f"SWA window {window}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("qk_norm", [True, False])
def test_multi_query_attention(dev, dtype, qk_norm):
    E, H, S = 512, 4, 70
    mod = MultiQueryAttention(H, E, qk_norm=qk_norm, dtype=dtype, device=dev)
    p = _randomize(mod, 5)
    x = _x((3, S, E), dtype, 6)
    c, s, cd, sd = _tables(E // H, S, dev)
    with torch.no_grad():
        got = mod(x.to(dev), cd, sd)
    close(got, om.mqa(x, p, c, s, H, qk_norm=qk_norm), what="MultiQueryAttention")


@pytest.mark.parametrize("dtype", DTYPES)
def test_cross_attention_with_and_without_cache(dev, dtype):
    E, Cd, H = 512, 384, 4
    mod = CrossAttention(E, Cd, H, dtype=dtype, device=dev)
    p = _randomize(mod, 7)
    x = _x((2, 9, E), dtype, 8)
    y = _x((2, 40, Cd), dtype, 9)
    with torch.no_grad():
        got = mod(x.to(dev), y.to(dev))
        close(got, om.cross(x, y, p, H)[0], what="CrossAttention")
        # the context arrives in two parts through a KVCache
        kv = KVCache(64, H, E // H, dtype=dtype, device=dev)
        mod(x.to(dev), y[:, :25].to(dev), kv)
        got = mod(x.to(dev), y[:, 25:].to(dev), kv)
    _, pre = om.cross(x, y[:, :25], p, H)
    close(got, om.cross(x, y[:, 25:], p, H, prefix_kv=pre)[0], what="CrossAttention + cache")


def _gqa(dev, dtype, seed):
    mod = GroupedQueryAttention(512, 8, 4, head_dim=128, dtype=dtype, device=dev)
    p = _randomize(mod, seed)
    mod.refresh_fused_weights()
    return mod, p


@pytest.mark.parametrize("dtype", DTYPES)
def test_gqa_without_cache(dev, dtype):
    mod, p = _gqa(dev, dtype, 10)
    x = _x((2, 75, 512), dtype, 11)
    c, s, cd, sd = _tables(128, 128, dev)
    with torch.no_grad():
        got = mod(x.to(dev), cd, sd)
    close(got, om.GQAOracle(p, 8, 4, 128).forward(x, c, s), what="GQA without cache")


@pytest.mark.parametrize("dtype", DTYPES)
def test_gqa_cached_prefill_then_decode(dev, dtype):
    """Prefill through the cache, then single-token steps (the fused decode
    kernel: QK-norm + RoPE + append + split-KV attention), each step against
    the oracle's cache; then the same cache serves a smaller batch."""
    mod, p = _gqa(dev, dtype, 12)
    c, s, cd, sd = _tables(128, 128, dev)
    x = _x((4, 40, 512), dtype, 13)
    kv = KVCache(64, 4, 128, dtype=dtype, device=dev, batch_size=4)
    orc = om.GQAOracle(p, 8, 4, 128)
    with torch.no_grad():
        got = mod(x[:, :33].to(dev), cd, sd, kv, 0)
        close(got, orc.forward(x[:, :33], c, s, cache_pos=0), what="GQA cached prefill")
        for t in range(33, 40):
            got = mod(x[:, t:t + 1].to(dev), cd, sd, kv, t)
            close(got, orc.forward(x[:, t:t + 1], c, s, cache_pos=t), what=f"GQA decode {t}")
        # a batch of 2 on the cache allocated for 4
        orc2 = om.GQAOracle(p, 8, 4, 128)
        y = _x((2, 12, 512), dtype, 14)
        got = mod(y[:, :10].to(dev), cd, sd, kv, 0)
        close(got, orc2.forward(y[:, :10], c, s, cache_pos=0), what="GQA prefill, smaller batch")
        for t in range(10, 12):
            got = mod(y[:, t:t + 1].to(dev), cd, sd, kv, t)
            close(got, orc2.forward(y[:, t:t + 1], c, s, cache_pos=t),
                  what=f"GQA decode {t}, smaller batch")


def test_positions_tensor_reuse(dev):
    """The [bs] positions tensor the cached GQA path hands to its kernels is
    reused across layers on one stream, refilled for another value or stream,
    and never cached from inside a graph capture (its fill would only run at
    replay)."""
    from torchplusplus_amd.attention import gqa

    a = gqa._positions(4, 7, dev)
    assert gqa._positions(4, 7, dev) is a and a.tolist() == [7] * 4
    assert gqa._positions(4, 8, dev).tolist() == [8] * 4
    assert gqa._positions(2, 8, dev).tolist() == [8] * 2
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        b = gqa._positions(2, 8, dev)
    s.synchronize()
    c = gqa._positions(2, 8, dev)
    assert b is not c and b.tolist() == c.tolist() == [8] * 2
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        t = gqa._positions(4, 9, dev)
    e = gqa._positions(4, 9, dev)
    assert e is not t and e.tolist() == [9] * 4
    g.replay()
    torch.cuda.synchronize()
    assert t.tolist() == [9] * 4
