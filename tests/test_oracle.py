"""Pin the CPU oracle before trusting it (CPU only).

Every oracle function is checked against something independent of its own
formula: a torch/numpy library routine, an fp64 closed form, a mathematical
invariant, or brute force on tiny inputs. The `*_mutation_*` tests plant a
plausible mistake in a copy of an oracle function and show the same check
rejects it, so each check has teeth.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle


def gen(seed=0):
    g = torch.Generator().manual_seed(seed)
    return g


# ---------------------------------------------------------------- RMSNorm
def _rms_pin(fn, dtype=torch.float32):
    g = gen(1)
    x = torch.randn(64, 512, generator=g)
    x[3] *= 1e-3  # a row where eps matters (mean(x^2) ~ eps)
    w = 1 + 0.1 * torch.randn(512, generator=g)
    y = fn(x.to(dtype), w.to(dtype), 1e-6).float()
    ref = F.rms_norm(x.double(), (512,), w.double(), eps=1e-6).float()
    return (y - ref).abs().max().item()


def test_rmsnorm_matches_library_routine():
    assert _rms_pin(oracle.rmsnorm) < 1e-5


def test_rmsnorm_mutation_missing_eps_is_caught():
    def wrong(x, w, eps):
        return oracle.rmsnorm(x, w, 0.0)

    assert _rms_pin(wrong) > 1e-2


def test_rmsnorm_mutation_mean_instead_of_rms_is_caught():
    def wrong(x, w, eps):
        xf = x.float()
        return (xf / (xf.abs().mean(-1, keepdim=True) + eps) * w).to(x.dtype)

    assert _rms_pin(wrong) > 1e-2


def test_rmsnorm_stats_fp64_closed_form():
    g = gen(2)
    x = torch.randn(128, 1024, generator=g).half()
    inv = oracle.rmsnorm_stats(x, 1e-6).double()
    xd = x.double().numpy()
    ref = 1.0 / np.sqrt((xd * xd).mean(-1) + 1e-6)
    assert np.max(np.abs(inv.numpy() / ref - 1)) < 1e-5


def test_rmsnorm_invariants():
    g = gen(3)
    x = torch.randn(16, 256, generator=g)
    ones = torch.ones(256)
    y = oracle.rmsnorm(x, ones, 0.0)
    # unit weight -> output RMS is exactly 1
    assert torch.allclose((y * y).mean(-1), torch.ones(16), atol=1e-5)
    # scale invariance
    assert torch.allclose(oracle.rmsnorm(7.5 * x, ones, 0.0), y, atol=1e-5)


def test_rmsnorm_reference_test_shape_fp16():
    """tests/rmsnorm_test.py:15-33 compares against nn.RMSNorm(eps=1e-6).half()
    at [32,128,512] with max abs diff < 1e-2."""
    g = gen(4)
    x = torch.randn(32, 128, 512, generator=g).half()
    w = torch.ones(512).half()
    ref = torch.nn.RMSNorm(512, eps=1e-6)(x.float()).half()
    assert (oracle.rmsnorm(x, w, 1e-6).float() - ref.float()).abs().max() < 1e-2


def test_add_rmsnorm_is_sum_then_norm():
    g = gen(5)
    x = torch.randn(8, 256, generator=g).bfloat16()
    r = torch.randn(8, 256, generator=g).bfloat16()
    w = torch.randn(256, generator=g).bfloat16()
    y, h = oracle.add_rmsnorm(x, r, w, 1e-6)
    assert torch.equal(h, x + r)  # torch's own bf16 add: one rounding
    assert torch.equal(y, oracle.rmsnorm(x + r, w, 1e-6))


# ---------------------------------------------------------------- LayerNorm
def _ln_pin(fn):
    g = gen(6)
    x = torch.randn(64, 512, generator=g) * 2 + 0.5
    w = 1 + 0.1 * torch.randn(512, generator=g)
    b = 0.1 * torch.randn(512, generator=g)
    y = fn(x, w, 1e-6, b)
    ref = F.layer_norm(x.double(), (512,), w.double(), b.double(), eps=1e-6).float()
    return (y - ref).abs().max().item()


def test_layernorm_matches_library_routine():
    assert _ln_pin(oracle.layernorm) < 1e-4


def test_layernorm_mutation_rms_instead_of_centered_is_caught():
    def wrong(x, w, eps, b):
        return oracle.rmsnorm(x, w, eps) + b

    assert _ln_pin(wrong) > 1e-2


def test_layernorm_stats_fp64():
    g = gen(7)
    x = torch.randn(64, 1024, generator=g).half()
    mean, rstd = oracle.layernorm_stats(x, 1e-6)
    xd = x.double().numpy()
    m = xd.mean(-1)
    r = 1 / np.sqrt(xd.var(-1) + 1e-6)
    assert np.max(np.abs(mean.double().numpy() - m)) < 1e-5
    assert np.max(np.abs(rstd.double().numpy() / r - 1)) < 1e-5


def test_layernorm_reference_test_shape_fp16():
    """tests/layernorm_test.py:15-34: vs nn.LayerNorm with zero bias, < 1e-2."""
    g = gen(8)
    x = torch.randn(32, 128, 512, generator=g).half()
    ln = torch.nn.LayerNorm(512, eps=1e-6)
    with torch.no_grad():
        ln.bias.zero_()
        ref = ln(x.float()).half()
    assert (oracle.layernorm(x, torch.ones(512).half(), 1e-6).float() - ref.float()).abs().max() < 1e-2


# ---------------------------------------------------------------- RoPE
def _rope_complex_fp64(x, pos, theta, d):
    """RoPE as complex rotation of the pair (x_j, x_{j+D/2}) by pos*theta^(-2j/D)."""
    xd = x.double()
    h = d // 2
    z = torch.complex(xd[..., :h], xd[..., h:])
    j = torch.arange(h, dtype=torch.float64)
    ang = pos[:, None].double() * theta ** (-2 * j / d)
    zr = z * torch.polar(torch.ones_like(ang), ang)
    return torch.cat([zr.real, zr.imag], dim=-1)


def test_rope_params_fp64_closed_form():
    cos, sin = oracle.compute_rope_params(128, 1e6, 2048)
    assert cos.dtype == torch.float16 and cos.shape == (2048, 128)
    j = torch.arange(64, dtype=torch.float64)
    ang = torch.arange(2048, dtype=torch.float64)[:, None] * 1e6 ** (-2 * j / 128)
    ang = torch.cat([ang, ang], 1)
    # fp32 angle error (|ang| <= 2047 rad, ~1.2e-4 abs) + fp16 rounding (4.9e-4)
    assert (cos.double() - torch.cos(ang)).abs().max() < 1e-3
    assert (sin.double() - torch.sin(ang)).abs().max() < 1e-3
    assert torch.all(cos[0] == 1) and torch.all(sin[0] == 0)


def _rope_fixture():
    import json
    import os

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "rope_params_d128_t1e6_s2048.json")
    with open(path) as f:
        return json.load(f)


def test_rope_params_match_golden_fixture():
    """The committed fp16 bit pattern of the D=128, theta=1e6, 2048-position
    tables (tests/golden/make_rope_params.py): the oracle and the package's
    own compute_rope_params on the CPU reproduce it bit for bit."""
    import hashlib

    from torchplusplus_amd.dlops import rope as R

    fx = _rope_fixture()
    rows = fx["rows"]
    for name, (cos, sin) in [("oracle", oracle.compute_rope_params(128, 1e6, 2048)),
                             ("package", R.compute_rope_params(128, 1e6, 2048, device="cpu"))]:
        for t, key in [(cos, "cos"), (sin, "sin")]:
            bits = t.contiguous().numpy().view(np.uint16)
            assert hashlib.sha256(bits.astype("<u2").tobytes()).hexdigest() == fx["sha256_" + key], (name, key)
            assert bits[rows].tolist() == fx[key + "_rows_u16"], (name, key)


def test_rope_matches_complex_rotation():
    g = gen(9)
    d = 128
    x = torch.randn(2, 3, 64, d, generator=g)
    cos, sin = oracle.compute_rope_params(d, 1e4, 64, out_dtype=torch.float32)
    y = oracle.rope(x, cos, sin)
    ref = _rope_complex_fp64(x, torch.arange(64), 1e4, d).float()
    assert (y - ref).abs().max() < 1e-4


def test_rope_mutation_swapped_sign_is_caught():
    g = gen(10)
    d = 64
    x = torch.randn(1, 2, 16, d, generator=g)
    cos, sin = oracle.compute_rope_params(d, 1e4, 16, out_dtype=torch.float32)
    wrong = oracle.rope(x, cos, -sin)  # rotate the wrong way
    ref = _rope_complex_fp64(x, torch.arange(16), 1e4, d).float()
    assert (wrong - ref).abs().max() > 1e-1


def test_rope_invariants():
    g = gen(11)
    d = 64
    x = torch.randn(1, 1, 1, d, generator=g).double()
    cos, sin = oracle.compute_rope_params(d, 1e4, 50, dtype=torch.float64, out_dtype=torch.float64)
    # position 0 is the identity
    assert torch.allclose(oracle.rope(x, cos[:1], sin[:1]).double(), x)
    # rotating by 20 then 30 equals rotating by 50 (pair norms preserved)
    y = oracle.rope(oracle.rope(x, cos[20:21], sin[20:21]), cos[30:31], sin[30:31])
    cos50, sin50 = oracle.compute_rope_params(d, 1e4, 51, dtype=torch.float64, out_dtype=torch.float64)
    assert torch.allclose(y, oracle.rope(x, cos50[50:51], sin50[50:51]), atol=1e-12)
    pn = lambda t: t[..., :32] ** 2 + t[..., 32:] ** 2  # noqa: E731
    assert torch.allclose(pn(y), pn(x), atol=1e-12)


def test_rope_reference_fp16_arith_within_tolerance():
    """The reference rounds every product and sum to fp16 (apply_rope.cuh:43-44);
    the build computes in fp32 and rounds once. Both agree within fp16 tolerance."""
    g = gen(12)
    x = torch.rand(1, 16, 256, 128, generator=g).half()  # tests/rope_test.py:36 data
    cos, sin = oracle.compute_rope_params(128, 1e6, 256)
    a = oracle.rope(x, cos, sin).float()
    b = oracle.rope_fp16_arith(x, cos, sin).float()
    assert torch.allclose(a, b, atol=2e-3, rtol=1e-2)


# ---------------------------------------------------------------- activations / linear
@pytest.mark.parametrize("act,fn", [
    ("gelu", lambda t: F.gelu(t, approximate="tanh")),
    ("silu", F.silu),
    ("relu", F.relu),
])
def test_activation_matches_library(act, fn):
    x = torch.linspace(-8, 8, 1001, dtype=torch.float64)
    assert (oracle.activation(x, act) - fn(x)).abs().max() < 1e-12


def test_linear_act_brute_force_fp64():
    g = gen(13)
    x = torch.randn(5, 48, generator=g).half()
    w = torch.randn(7, 48, generator=g).half()
    b = torch.randn(7, generator=g).half()
    y = oracle.linear_act(x, w, b, "silu").double()
    xd, wd, bd = x.double().tolist(), w.double().tolist(), b.double().tolist()
    for i in range(5):
        for n in range(7):
            acc = sum(xd[i][k] * wd[n][k] for k in range(48)) + bd[n]
            pre = float(torch.tensor(acc).half())
            ref = pre / (1 + math.exp(-pre))
            assert abs(y[i, n].item() - ref) <= 2e-3 * max(1.0, abs(ref))


def test_linear_act_mutation_transposed_weight_is_caught():
    g = gen(14)
    x = torch.randn(16, 16, generator=g)
    w = torch.randn(16, 16, generator=g)
    ref = torch.from_numpy(x.double().numpy() @ w.double().numpy().T).float()
    assert (oracle.linear_act(x, w) - ref).abs().max() < 1e-4
    assert (oracle.linear_act(x, w.t().contiguous()) - ref).abs().max() > 1e-1


# ---------------------------------------------------------------- GEMV
def test_gemv_matches_numpy_fp64():
    g = gen(15)
    x = torch.randn(4, 1024, generator=g).half()
    w = (0.02 * torch.randn(3072, 1024, generator=g)).half()
    ref = x.double().numpy() @ w.double().numpy().T
    assert np.max(np.abs(oracle.gemv(x, w).double().numpy() - ref)) < 2e-3


def test_hgemv_cpu_known_answer_and_agreement():
    a = np.ones((8, 2048), np.float16)
    x = np.ones(2048, np.float16)
    assert np.all(oracle.hgemv_cpu(a, x) == 2048)
    rng = np.random.default_rng(0)
    a = (0.02 * rng.standard_normal((64, 1024))).astype(np.float16)
    x = rng.standard_normal(1024).astype(np.float16)
    ref = oracle.gemv(torch.from_numpy(x)[None], torch.from_numpy(a))[0].float().numpy()
    assert np.max(np.abs(oracle.hgemv_cpu(a, x).astype(np.float32) - ref)) < 2e-2


# ---------------------------------------------------------------- attention
@pytest.mark.parametrize("causal", [False, True])
def test_attention_matches_sdpa(causal):
    g = gen(16)
    q = torch.randn(2, 64, 8, 32, generator=g)
    k = torch.randn(2, 64, 2, 32, generator=g)
    v = torch.randn(2, 64, 2, 32, generator=g)
    o = oracle.attention(q, k, v, causal=causal)
    ref = F.scaled_dot_product_attention(
        q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), is_causal=causal, enable_gqa=True
    ).transpose(1, 2)
    assert (o - ref).abs().max() < 1e-5


@pytest.mark.parametrize("sq,sk,causal,window", [
    (7, 7, True, (-1, -1)),
    (3, 9, True, (-1, -1)),     # bottom-right causal alignment
    (9, 9, True, (3, 0)),       # sliding window (w-1, 0) as swa.py:88
    (5, 8, False, (2, 1)),
    (6, 4, True, (-1, -1)),     # Sq > Sk: the first rows see nothing -> 0
])
def test_attention_brute_force_fp64(sq, sk, causal, window):
    g = gen(17)
    q = torch.randn(1, sq, 4, 8, generator=g)
    k = torch.randn(1, sk, 2, 8, generator=g)
    v = torch.randn(1, sk, 2, 8, generator=g)
    o = oracle.attention(q, k, v, causal=causal, window=window)
    ref = oracle.attention_fp64_loops(q, k, v, causal=causal, window=window)
    assert (o.double() - ref).abs().max() < 1e-5


def test_attention_mutation_top_left_causal_is_caught():
    g = gen(18)
    q = torch.randn(1, 3, 2, 8, generator=g)
    k = torch.randn(1, 9, 2, 8, generator=g)
    v = torch.randn(1, 9, 2, 8, generator=g)
    ref = oracle.attention_fp64_loops(q, k, v, causal=True)
    wrong = F.scaled_dot_product_attention(  # top-left aligned mask
        q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), is_causal=True
    ).transpose(1, 2)
    assert (wrong.double() - ref).abs().max() > 1e-2


def test_attention_special_cases():
    g = gen(19)
    q = torch.randn(1, 5, 2, 16, generator=g)
    k = torch.randn(1, 5, 1, 16, generator=g)
    row = torch.randn(16, generator=g)
    v = row.expand(1, 5, 1, 16).contiguous()
    # uniform V -> every output row equals that V row
    assert torch.allclose(oracle.attention(q, k, v, causal=True), row.expand(1, 5, 2, 16), atol=1e-6)
    # a single visible key -> O = V of that key
    v2 = torch.randn(1, 5, 1, 16, generator=g)
    o = oracle.attention(q, k, v2, causal=True)
    assert torch.allclose(o[0, 0, 0], v2[0, 0, 0], atol=1e-6)


def test_decode_attention_equals_prefix_attention():
    g = gen(20)
    b, hq, hkv, d, lmax = 3, 4, 2, 16, 12
    q = torch.randn(b, 1, hq, d, generator=g)
    kc = torch.randn(b, hkv, lmax, d, generator=g)
    vc = torch.randn(b, hkv, lmax, d, generator=g)
    lens = [12, 5, 1]
    o = oracle.decode_attention(q, kc, vc, lens)
    for bi, L in enumerate(lens):
        ref = oracle.attention_fp64_loops(q[bi:bi + 1], kc[bi:bi + 1, :, :L].transpose(1, 2),
                                          vc[bi:bi + 1, :, :L].transpose(1, 2), causal=True)
        assert (o[bi:bi + 1].double() - ref).abs().max() < 1e-5
