"""Pin the attention-module oracle (oracle/modules.py) on the CPU against an
fp64 assembly of torch library routines (F.linear, F.rms_norm,
F.scaled_dot_product_attention with enable_gqa and an explicit bottom-right
mask, RoPE as a complex rotation), plus cache consistency for GQA and
mutation tests that plant one mistake each."""
import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import modules as om

D = 16
CTX = 48


def _params(E, H, Hk, seed, cross_dim=None, bias=True):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: 0.2 * torch.randn(*s, generator=g)  # noqa: E731
    kin = cross_dim or E
    p = {"Wq.weight": r(H * D, E), "Wk.weight": r(Hk * D, kin), "Wv.weight": r(Hk * D, kin),
         "out_projection.weight": r(E, H * D),
         "q_norm.weight": 1 + r(D), "k_norm.weight": 1 + r(D)}
    if bias:
        p["out_projection.bias"] = r(E)
    return p


def _tables(dtype=torch.float64):
    c, s = oracle.compute_rope_params(D, 1e6, CTX)
    return c.to(dtype), s.to(dtype)


def _rope_complex(t, cos, sin, pos0=0):
    """t [B, H, S, D] rotated at positions pos0.. (pairs (i, i+D/2) as complex)."""
    h = t.shape[-1] // 2
    S = t.shape[2]
    z = torch.complex(t[..., :h], t[..., h:]) * torch.complex(cos[pos0:pos0 + S, :h],
                                                              sin[pos0:pos0 + S, :h])
    return torch.cat([z.real, z.imag], dim=-1)


def _mask(sq, sk, left=None):
    i = torch.arange(sq)[:, None] + (sk - sq)
    j = torch.arange(sk)[None, :]
    keep = j <= i
    if left is not None:
        keep &= j >= i - left
    return keep


def lib_self_attn(x, p, H, Hk, qknorm=True, window_size=None, pos0=0, k_prefix=None):
    """fp64 library assembly of an MHA/SWA/MQA/GQA forward; k_prefix = cached
    (k, v) [B, Hk, Sp, D] already rotated."""
    P = {k: v.double() for k, v in p.items()}
    x = x.double()
    B, S, _ = x.shape
    cos, sin = _tables()
    q = F.linear(x, P["Wq.weight"]).view(B, S, H, D).transpose(1, 2)
    k = F.linear(x, P["Wk.weight"]).view(B, S, Hk, D).transpose(1, 2)
    v = F.linear(x, P["Wv.weight"]).view(B, S, Hk, D).transpose(1, 2)
    if qknorm:
        q = F.rms_norm(q, (D,), P["q_norm.weight"], eps=1e-6)
        k = F.rms_norm(k, (D,), P["k_norm.weight"], eps=1e-6)
    q, k = _rope_complex(q, cos, sin, pos0), _rope_complex(k, cos, sin, pos0)
    if k_prefix is not None:
        k = torch.cat([k_prefix[0], k], 2)
        v = torch.cat([k_prefix[1], v], 2)
    left = window_size - 1 if window_size is not None else None
    o = F.scaled_dot_product_attention(q, k, v, attn_mask=_mask(S, k.shape[2], left),
                                       enable_gqa=True)
    out = F.linear(o.transpose(1, 2).reshape(B, S, H * D), P["out_projection.weight"],
                   P.get("out_projection.bias"))
    return out.float(), (k, v)


def lib_cross(x, y, p, H):
    P = {k: v.double() for k, v in p.items()}
    x, y = x.double(), y.double()
    B, Sq, E = x.shape
    q = F.linear(x, P["Wq.weight"]).view(B, Sq, H, D).transpose(1, 2)
    k = F.linear(y, P["Wk.weight"]).view(B, -1, H, D).transpose(1, 2)
    v = F.linear(y, P["Wv.weight"]).view(B, -1, H, D).transpose(1, 2)
    o = F.scaled_dot_product_attention(q, k, v)
    return F.linear(o.transpose(1, 2).reshape(B, Sq, E), P["out_projection.weight"],
                    P["out_projection.bias"]).float()


def _x(B, S, E, seed):
    return torch.randn(B, S, E, generator=torch.Generator().manual_seed(seed))


def _err(a, b):
    return ((a - b).abs().max() / b.abs().max()).item()


def _cos_sin(S=None):
    c, s = oracle.compute_rope_params(D, 1e6, CTX, out_dtype=torch.float16)
    c, s = c.float(), s.float()
    return (c[:S], s[:S]) if S else (c, s)


@pytest.mark.parametrize("window", [None, 5])
def test_mha_swa_oracle_matches_library(window):
    x, p = _x(2, 19, 64, 1), _params(64, 4, 4, 2)
    c, s = _cos_sin(19)
    got = om.mha(x, p, c, s, 4, window_size=window)
    assert _err(got, lib_self_attn(x, p, 4, 4, window_size=window)[0]) < 1e-5


def test_mqa_oracle_matches_library():
    x, p = _x(2, 17, 64, 3), _params(64, 4, 1, 4, bias=False)
    c, s = _cos_sin(17)
    assert _err(om.mqa(x, p, c, s, 4), lib_self_attn(x, p, 4, 1)[0]) < 1e-5


def test_cross_oracle_matches_library():
    x, p = _x(2, 7, 64, 5), _params(64, 4, 4, 6, cross_dim=48)
    y = torch.randn(2, 11, 48, generator=torch.Generator().manual_seed(7))
    assert _err(om.cross(x, y, p, 4)[0], lib_cross(x, y, p, 4)) < 1e-5


def test_cross_oracle_cached_prefix_equals_concatenated_context():
    x, p = _x(2, 7, 64, 8), _params(64, 4, 4, 9, cross_dim=48)
    y = torch.randn(2, 13, 48, generator=torch.Generator().manual_seed(10))
    _, kv = om.cross(x, y[:, :6], p, 4)
    got, _ = om.cross(x, y[:, 6:], p, 4, prefix_kv=kv)
    assert _err(got, lib_cross(x, y, p, 4)) < 1e-5


def test_gqa_oracle_no_cache_and_cached_decode_match_library():
    x, p = _x(2, 21, 64, 11), _params(64, 4, 2, 12, bias=False)
    c, s = _cos_sin()
    want, _ = lib_self_attn(x, p, 4, 2)
    orc = om.GQAOracle(p, 4, 2, D)
    assert _err(orc.forward(x, c, s), want) < 1e-5
    # prefill 15 tokens through the cache, then one token at a time
    outs = [orc.forward(x[:, :15], c, s, cache_pos=0)]
    for t in range(15, 21):
        outs.append(orc.forward(x[:, t:t + 1], c, s, cache_pos=t))
    assert _err(torch.cat(outs, 1), want) < 1e-5


# ---- mutations ---------------------------------------------------------------
def test_mutation_mqa_k_rotated_from_q_is_caught():
    """The reference's mqa.py:81 rotates Q into K; the check must see it."""
    x, p = _x(2, 17, 64, 3), _params(64, 4, 1, 4, bias=False)
    c, s = _cos_sin(17)

    def wrong(x, p, cos, sin, H):
        B, S, E = x.shape
        q = om._heads(om._lin(x, p, "Wq.weight"), B, S, H, D)
        v = om._heads(om._lin(x, p, "Wv.weight"), B, S, 1, D)
        q = oracle.rmsnorm(q, p["q_norm.weight"], 1e-6)
        q = om._rope_bshd(q, cos, sin)
        o = oracle.attention(q, q[:, :, :1], v, causal=True)
        return om._lin(o.reshape(B, S, E), p, "out_projection.weight")

    assert _err(wrong(x, p, c, s, 4), lib_self_attn(x, p, 4, 1)[0]) > 1e-2


def test_mutation_window_off_by_one_is_caught():
    x, p = _x(2, 19, 64, 1), _params(64, 4, 4, 2)
    c, s = _cos_sin(19)
    got = om.mha(x, p, c, s, 4, window_size=6)  # keys [i-5, i] instead of [i-4, i]
    assert _err(got, lib_self_attn(x, p, 4, 4, window_size=5)[0]) > 1e-2


def test_mutation_missing_output_bias_is_caught():
    x, p = _x(2, 19, 64, 1), _params(64, 4, 4, 2)
    c, s = _cos_sin(19)
    q = dict(p)
    q.pop("out_projection.bias")
    assert _err(om.mha(x, q, c, s, 4), lib_self_attn(x, p, 4, 4)[0]) > 1e-2


def test_mutation_decode_positions_from_zero_is_caught():
    x, p = _x(2, 21, 64, 11), _params(64, 4, 2, 12, bias=False)
    c, s = _cos_sin()
    want, _ = lib_self_attn(x, p, 4, 2)

    class Wrong(om.GQAOracle):
        def forward(self, x, cos, sin, cache_pos=None):  # every chunk rotated from 0
            if cache_pos:  # table row cache_pos + i now holds position i
                cos = torch.cat([cos[:cache_pos], cos[:CTX - cache_pos]])
                sin = torch.cat([sin[:cache_pos], sin[:CTX - cache_pos]])
            return super().forward(x, cos, sin, cache_pos)

    orc = Wrong(p, 4, 2, D)
    outs = [orc.forward(x[:, :15], c, s, cache_pos=0)]
    for t in range(15, 21):
        outs.append(orc.forward(x[:, t:t + 1], c, s, cache_pos=t))
    assert _err(torch.cat(outs, 1), want) > 1e-2
