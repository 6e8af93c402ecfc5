"""The fused projection weights follow their source parameters, as the
reference's modules read nn.Linear weights on every call
(torchpp/attention/gqa.py:82-84, examples/LLM/fastqwen3.py:71-78).

CPU: after a forward-time build of the fused Q/K/V and gate/up weights, a
load_state_dict (plain and under inference mode), an in-place edit and a
replaced Parameter each give the fused weights of a fresh module built from
the new parameters. GPU: forward -> load_state_dict(new) -> forward equals a
fresh module built from `new`, for GroupedQueryAttention, FFN and FastQwen3.
"""
import copy

import pytest
import torch

from torchplusplus_amd.attention import GroupedQueryAttention
from torchplusplus_amd.dlops.linear import interleave_gate_up
from torchplusplus_amd.fastqwen3 import FFN, FastQwen3, QwenConfig

TINY = QwenConfig(vocab_size=300, context_length=128, embed_dim=128, n_heads=4, n_layers=2,
                  head_dim=64, n_kv_heads=2, hidden_dim=256, dtype=torch.bfloat16)


def _rand_state(mod, seed):
    g = torch.Generator().manual_seed(seed)
    return {k: torch.randn(v.shape, generator=g).to(v.dtype) for k, v in mod.state_dict().items()}


def _gqa(dev="cpu"):
    return GroupedQueryAttention(128, 4, 2, head_dim=64, dtype=torch.bfloat16, device=dev)


def _want_qkv(sd):
    return torch.cat([sd["Wq.weight"], sd["Wk.weight"], sd["Wv.weight"]], 0)


def test_gqa_fused_weight_follows_load_state_dict():
    m = _gqa()
    old = m.fused_qkv_weight().clone()
    new = _rand_state(m, 1)
    m.load_state_dict(new)
    got = m.fused_qkv_weight()
    assert not torch.equal(got, old)
    assert torch.equal(got, _want_qkv(new))
    fresh = _gqa()
    fresh.load_state_dict(new)
    assert torch.equal(fresh.fused_qkv_weight(), got)


def test_gqa_fused_weight_follows_inference_mode_load_and_edits():
    with torch.inference_mode():  # inference tensors: no version counter
        m = _gqa()
        m.fused_qkv_weight()
        new = _rand_state(m, 2)
        m.load_state_dict(new)
        assert torch.equal(m.fused_qkv_weight(), _want_qkv(new))
    m = _gqa()
    buf = m.fused_qkv_weight()
    ptr = buf.data_ptr()
    with torch.no_grad():
        m.Wk.weight.mul_(2)  # in-place edit
    assert torch.equal(m.fused_qkv_weight(), torch.cat([m.Wq.weight, m.Wk.weight, m.Wv.weight]))
    assert m.fused_qkv_weight().data_ptr() == ptr  # rebuilt in place (graphs keep their address)
    m.Wv.weight = torch.nn.Parameter(torch.ones_like(m.Wv.weight))  # replaced parameter
    assert torch.equal(m.fused_qkv_weight()[-m.Wv.weight.shape[0]:], m.Wv.weight)


def test_ffn_interleaved_weight_follows_load_state_dict():
    f = FFN(128, 256, dtype=torch.bfloat16)
    f.w_gu()
    new = _rand_state(f, 3)
    f.load_state_dict(new)
    assert torch.equal(f.w_gu(), interleave_gate_up(new["fused_linear_layer1.weight"],
                                                    new["linear_layerP.weight"]))


def test_model_load_state_dict_reaches_every_block_and_copies():
    m = FastQwen3(TINY)
    m.refresh_fused_weights()
    new = _rand_state(m, 4)
    c = copy.deepcopy(m)
    m.load_state_dict(new)
    for i, blk in enumerate(m.transformer_blocs):
        p = f"transformer_blocs.{i}."
        assert torch.equal(blk.attn.fused_qkv_weight(),
                           torch.cat([new[p + "attn.Wq.weight"], new[p + "attn.Wk.weight"],
                                      new[p + "attn.Wv.weight"]]))
        assert torch.equal(blk.ffn.w_gu(), interleave_gate_up(new[p + "ffn.fused_linear_layer1.weight"],
                                                              new[p + "ffn.linear_layerP.weight"]))
    # the copy made before the load keeps its own weights
    for a, b in zip(c.transformer_blocs, m.transformer_blocs):
        assert not torch.equal(a.attn.fused_qkv_weight(), b.attn.fused_qkv_weight())
        assert torch.equal(a.attn.fused_qkv_weight(),
                           torch.cat([a.attn.Wq.weight, a.attn.Wk.weight, a.attn.Wv.weight]))


@pytest.mark.gpu
@torch.inference_mode()
def test_forward_load_forward_matches_fresh_modules(dev):
    from oracle import compute_rope_params

    g = torch.Generator().manual_seed(5)
    cos, sin = (t.to(dev) for t in compute_rope_params(64, 1e6, 64))
    x = (0.5 * torch.randn(2, 24, 128, generator=g)).bfloat16().to(dev)
    x1 = x[:, :1].contiguous()  # decode-sized input (GEMV path)

    def scaled(sd, s):
        return {k: (v.float() * s).to(v.dtype) if "norm" not in k else v for k, v in sd.items()}

    a = _gqa(dev)
    new = scaled(_rand_state(a, 6), 0.1)
    a(x, cos, sin)
    a(x1, cos, sin)
    a.load_state_dict(new)
    fresh = _gqa(dev)
    fresh.load_state_dict(new)
    assert torch.equal(a(x, cos, sin), fresh(x, cos, sin))
    assert torch.equal(a(x1, cos, sin), fresh(x1, cos, sin))

    f = FFN(128, 256, dtype=torch.bfloat16, device=dev)
    new = scaled(_rand_state(f, 7), 0.1)
    f(x), f(x1)
    f.load_state_dict(new)
    ff = FFN(128, 256, dtype=torch.bfloat16, device=dev)
    ff.load_state_dict(new)
    assert torch.equal(f(x), ff(x)) and torch.equal(f(x1), ff(x1))

    m = FastQwen3(TINY, device=dev).eval()
    m.init_weights(std=0.05, generator=torch.Generator(device=dev).manual_seed(8))
    ids = torch.randint(0, TINY.vocab_size, (2, 12), generator=g).to(dev)
    m.generate_greedy(ids, 4)
    new = {k: v.clone() for k, v in m.state_dict().items()}
    with torch.no_grad():
        for k in new:
            if "norm" not in k:
                new[k].normal_(0.0, 0.05, generator=torch.Generator(device=dev).manual_seed(9))
    m.load_state_dict(new)
    fresh = FastQwen3(TINY, device=dev).eval()
    fresh.load_state_dict(new)
    assert torch.equal(m(ids), fresh(ids))
    assert torch.equal(m.generate_greedy(ids, 4), fresh.generate_greedy(ids, 4))
