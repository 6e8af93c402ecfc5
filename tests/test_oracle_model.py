"""Pin the model oracle (oracle/qwen3.py) on the CPU.

The per-op oracle is pinned in test_oracle.py; these checks pin how the model
oracle composes the ops (block order, residual placement, QK-norm before
RoPE, decode positions and cache append, SwiGLU order, final norm) against
things that do not share its code:
  * an fp64 assembly of torch library routines (F.rms_norm, F.linear,
    F.scaled_dot_product_attention(is_causal, enable_gqa), F.silu, RoPE as a
    complex rotation of (x_i, x_{i+D/2}) pairs) of the reference block
    (examples/LLM/fastqwen3.py:107-116, 187-188; torchpp/attention/gqa.py:80-131);
  * cache consistency: prefill S tokens then decode one token at a time
    through the oracle's cache gives the logits of one full forward;
  * causality: changing token t+1 leaves the logits at positions <= t alone.
The mutation tests plant one plausible mistake per stage in a subclass of the
oracle and show that these checks reject it.
"""
from types import SimpleNamespace

import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle.qwen3 import Qwen3Oracle

CFG = SimpleNamespace(vocab_size=97, embed_dim=64, n_heads=4, n_kv_heads=2, head_dim=16,
                      hidden_dim=96, n_layers=2, qk_norm=True, rope_base=1e6,
                      dtype=torch.float32)
CTX = 64


def make_state(cfg, seed=0):
    """A FastQwen3 state dict (parameter names of fastqwen3.py:50-149) with
    random weights, including non-trivial norm weights."""
    g = torch.Generator().manual_seed(seed)
    E, H, Hk, D, I = cfg.embed_dim, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.hidden_dim
    rnd = lambda *s: 0.2 * torch.randn(*s, generator=g)  # noqa: E731
    nrm = lambda n: 1 + 0.2 * torch.randn(n, generator=g)  # noqa: E731
    st = {"tok_embed.weight": torch.randn(cfg.vocab_size, E, generator=g),
          "final_rmsnorm.weight": nrm(E), "out_head.weight": rnd(cfg.vocab_size, E)}
    for i in range(cfg.n_layers):
        p = f"transformer_blocs.{i}."
        st.update({p + "rms_norm1.weight": nrm(E), p + "rms_norm2.weight": nrm(E),
                   p + "attn.Wq.weight": rnd(H * D, E), p + "attn.Wk.weight": rnd(Hk * D, E),
                   p + "attn.Wv.weight": rnd(Hk * D, E), p + "attn.out_projection.weight": rnd(E, H * D),
                   p + "attn.q_norm.weight": nrm(D), p + "attn.k_norm.weight": nrm(D),
                   p + "ffn.fused_linear_layer1.weight": rnd(I, E),
                   p + "ffn.linear_layerP.weight": rnd(I, E),
                   p + "ffn.linear_layer2.weight": rnd(E, I)})
    return st


def _rope_complex(t, cos, sin):
    """t [B, H, S, D]: multiply each pair (t_i, t_{i+D/2}) as a complex number
    by cos + i sin of its position (the rotate-half RoPE written as a complex
    rotation; the tables are the same fp16 tables the model uses)."""
    h = t.shape[-1] // 2
    z = torch.complex(t[..., :h], t[..., h:])
    rot = torch.complex(cos[: t.shape[2], :h], sin[: t.shape[2], :h])
    zr = z * rot
    return torch.cat([zr.real, zr.imag], dim=-1)


def library_forward(state, cfg, ids, dtype=torch.float64):
    """Whole-sequence logits from torch library routines (no oracle code)."""
    W = {k: v.to(dtype) for k, v in state.items()}
    cos, sin = (t.to(dtype) for t in oracle.compute_rope_params(cfg.head_dim, cfg.rope_base, CTX))
    B, S = ids.shape
    E, H, Hk, D = cfg.embed_dim, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    x = F.embedding(ids, W["tok_embed.weight"])
    for i in range(cfg.n_layers):
        p = f"transformer_blocs.{i}."
        h = F.rms_norm(x, (E,), W[p + "rms_norm1.weight"], eps=1e-6)
        q = F.linear(h, W[p + "attn.Wq.weight"]).view(B, S, H, D).transpose(1, 2)
        k = F.linear(h, W[p + "attn.Wk.weight"]).view(B, S, Hk, D).transpose(1, 2)
        v = F.linear(h, W[p + "attn.Wv.weight"]).view(B, S, Hk, D).transpose(1, 2)
        q = _rope_complex(F.rms_norm(q, (D,), W[p + "attn.q_norm.weight"], eps=1e-6), cos, sin)
        k = _rope_complex(F.rms_norm(k, (D,), W[p + "attn.k_norm.weight"], eps=1e-6), cos, sin)
        o = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
        x = x + F.linear(o.transpose(1, 2).reshape(B, S, H * D), W[p + "attn.out_projection.weight"])
        h = F.rms_norm(x, (E,), W[p + "rms_norm2.weight"], eps=1e-6)
        gate = F.silu(F.linear(h, W[p + "ffn.fused_linear_layer1.weight"]))
        x = x + F.linear(gate * F.linear(h, W[p + "ffn.linear_layerP.weight"]),
                         W[p + "ffn.linear_layer2.weight"])
    x = F.rms_norm(x, (E,), W["final_rmsnorm.weight"], eps=1e-6)
    return F.linear(x, W["out_head.weight"]).float()


def _rel(a, b):
    return ((a - b).abs().max() / b.abs().max()).item()


def _incremental(orc, ids, S):
    """Prefill ids[:, :S], then one token per call, then a two-token chunk."""
    T = ids.shape[1]
    outs = [orc.forward(ids[:, :S], 0)]
    pos = S
    while pos < T - 2:
        outs.append(orc.forward(ids[:, pos:pos + 1], pos))
        pos += 1
    outs.append(orc.forward(ids[:, pos:T], pos))
    return torch.cat(outs, dim=1)


IDS = torch.randint(0, CFG.vocab_size, (3, 23), generator=torch.Generator().manual_seed(1))


def _pin_errors(cls, state=None):
    """(prefill error vs the library, incremental-decode error vs the
    library) for an oracle class, relative to the largest logit."""
    state = state or make_state(CFG)
    lib = library_forward(state, CFG, IDS)
    full = cls(state, CFG, CTX).forward(IDS, 0)
    inc = _incremental(cls(state, CFG, CTX), IDS, 15)
    return _rel(full, lib), _rel(inc, lib)


def test_model_oracle_matches_library_assembly():
    e_full, e_inc = _pin_errors(Qwen3Oracle)
    assert e_full < 1e-5, e_full
    assert e_inc < 1e-5, e_inc


def test_model_oracle_decode_through_cache_equals_full_forward():
    st = make_state(CFG, seed=3)
    full = Qwen3Oracle(st, CFG, CTX).forward(IDS, 0)
    inc = _incremental(Qwen3Oracle(st, CFG, CTX), IDS, 9)
    assert _rel(inc, full) < 1e-5


def test_model_oracle_is_causal():
    st = make_state(CFG, seed=4)
    a = Qwen3Oracle(st, CFG, CTX).forward(IDS, 0)
    for t in (0, 7, 21):
        ids = IDS.clone()
        ids[:, t + 1] = (ids[:, t + 1] + 1) % CFG.vocab_size
        b = Qwen3Oracle(st, CFG, CTX).forward(ids, 0)
        assert torch.allclose(a[:, : t + 1], b[:, : t + 1], atol=1e-6, rtol=0), t
        assert not torch.allclose(a[:, t + 1], b[:, t + 1], atol=1e-3)


def test_model_oracle_bf16_flow_close_to_library():
    """With bf16 rounding at every op boundary the oracle stays within the
    model-level tolerance of the exact fp64 assembly."""
    cfg = SimpleNamespace(**{**vars(CFG), "dtype": torch.bfloat16})
    st = {k: v.bfloat16().float() for k, v in make_state(CFG, seed=5).items()}
    lib = library_forward(st, cfg, IDS)
    got = Qwen3Oracle(st, cfg, CTX).forward(IDS, 0)
    rel = ((got - lib).norm() / lib.norm()).item()
    assert rel < 2e-2, rel


# ---- mutations: each must be rejected by the pins above ---------------------
class _DecodeOffByOne(Qwen3Oracle):
    def _positions(self, start, S):  # decode tokens rotated one position late
        return slice(start + 1, start + 1 + S) if start else slice(0, S)


class _NormAfterRope(Qwen3Oracle):
    def _qk(self, i, q, k, start):
        p = f"transformer_blocs.{i}.attn."
        pos = self._positions(start, q.shape[1])
        q, k = self._rope(q, pos).float(), self._rope(k, pos).float()
        return self._norm(q, p + "q_norm.weight"), self._norm(k, p + "k_norm.weight")


class _DroppedAttnResidual(Qwen3Oracle):
    def _block(self, i, x, start):
        p = f"transformer_blocs.{i}."
        x = self._attn(i, self._norm(x, p + "rms_norm1.weight"), start)
        f = self._ffn(i, self._norm(x, p + "rms_norm2.weight"))
        return x + f


class _SiluOnUp(Qwen3Oracle):
    def _ffn(self, i, h):
        p = f"transformer_blocs.{i}.ffn."
        g = self._lin(h, p + "fused_linear_layer1.weight")
        u = oracle.activation(self._lin(h, p + "linear_layerP.weight"), "silu")
        return self._lin(g * u, p + "linear_layer2.weight")


class _NoFinalNorm(Qwen3Oracle):
    def _head(self, x):
        return x @ self.w["out_head.weight"].t()


class _CacheOverwritten(Qwen3Oracle):
    def _attn(self, i, h, start):  # decode attends to the new token only
        self.k[i] = self.v[i] = None
        return super()._attn(i, h, 0)


class _NormBeforeResidualSum(Qwen3Oracle):
    def _block(self, i, x, start):  # ffn norm reads the pre-attention stream
        p = f"transformer_blocs.{i}."
        a = self._attn(i, self._norm(x, p + "rms_norm1.weight"), start)
        f = self._ffn(i, self._norm(x, p + "rms_norm2.weight"))
        return x + a + f


@pytest.mark.parametrize("mutant", [_DecodeOffByOne, _NormAfterRope, _DroppedAttnResidual,
                                    _SiluOnUp, _NoFinalNorm, _CacheOverwritten,
                                    _NormBeforeResidualSum])
def test_model_oracle_mutation_is_caught(mutant):
    e_full, e_inc = _pin_errors(mutant)
    assert max(e_full, e_inc) > 1e-2, (mutant.__name__, e_full, e_inc)
