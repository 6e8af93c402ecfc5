"""CPU restatement of the FastQwen3 forward (test infrastructure only).

Follows examples/LLM/fastqwen3.py:81-189 with the reference's eager data flow:
every op computes in fp32 from the model-dtype inputs and rounds its output
to the model dtype, as the eager PyTorch modules would:
  block: x = x + attn(rms_norm1(x)); x = x + ffn(rms_norm2(x))   (:107-116)
  attn (torchpp/attention/gqa.py:80-131): q/k/v projections, QK-RMSNorm over
       head_dim, rotate-half RoPE at the absolute positions, causal GQA
       attention over the cache prefix, output projection
  ffn: linear_layer2(silu(fused_linear_layer1(x)) * linear_layerP(x)) -- the
       SwiGLU the reference intends (its committed shapes at :71-73 cannot run)
  logits = out_head(final_rmsnorm(x))                              (:187-188)
It reads the weights of a torchplusplus_amd FastQwen3 through its state dict.
"""
from __future__ import annotations

import torch

from . import ops


def _r(t: torch.Tensor, dtype) -> torch.Tensor:
    return t.to(dtype).float()


class Qwen3Oracle:
    def __init__(self, state: dict, cfg, rope_context: int):
        self.cfg = cfg
        self.dt = cfg.dtype
        self.w = {k: v.detach().cpu().float() for k, v in state.items()}
        self.cos, self.sin = ops.compute_rope_params(cfg.head_dim, cfg.rope_base, rope_context)
        self.k = [None] * cfg.n_layers
        self.v = [None] * cfg.n_layers

    def _lin(self, x, name):
        return _r(x @ self.w[name].t(), self.dt)

    def _norm(self, x, name):
        return ops.rmsnorm(x.to(self.dt), self.w[name].to(self.dt), 1e-6).float()

    def forward(self, ids: torch.Tensor, start: int) -> torch.Tensor:
        """Logits [B, S, V] (fp32) for `ids` placed at positions start..;
        keeps K/V for later calls (start must equal the cached length)."""
        c = self.cfg
        B, S = ids.shape
        x = _r(self.w["tok_embed.weight"][ids], self.dt)
        pos = slice(start, start + S)
        for i in range(c.n_layers):
            p = f"transformer_blocs.{i}."
            h = self._norm(x, p + "rms_norm1.weight")
            q = self._lin(h, p + "attn.Wq.weight").view(B, S, c.n_heads, c.head_dim)
            k = self._lin(h, p + "attn.Wk.weight").view(B, S, c.n_kv_heads, c.head_dim)
            v = self._lin(h, p + "attn.Wv.weight").view(B, S, c.n_kv_heads, c.head_dim)
            if c.qk_norm:
                q = self._norm(q, p + "attn.q_norm.weight")
                k = self._norm(k, p + "attn.k_norm.weight")
            q = ops.rope(q.to(self.dt).transpose(1, 2), self.cos[pos], self.sin[pos]).transpose(1, 2)
            k = ops.rope(k.to(self.dt).transpose(1, 2), self.cos[pos], self.sin[pos]).transpose(1, 2)
            v = v.to(self.dt)
            if start == 0:
                self.k[i], self.v[i] = k, v
            else:
                self.k[i] = torch.cat([self.k[i], k], 1)
                self.v[i] = torch.cat([self.v[i], v], 1)
            o = ops.attention(q, self.k[i], self.v[i], causal=True).float()
            a = self._lin(o.reshape(B, S, -1), p + "attn.out_projection.weight")
            x = _r(x + a, self.dt)
            h = self._norm(x, p + "rms_norm2.weight")
            g = self._lin(h, p + "ffn.fused_linear_layer1.weight")
            g = _r(ops.activation(g, "silu"), self.dt)
            u = self._lin(h, p + "ffn.linear_layerP.weight")
            f = self._lin(_r(g * u, self.dt), p + "ffn.linear_layer2.weight")
            x = _r(x + f, self.dt)
        h = self._norm(x, "final_rmsnorm.weight")
        return h @ self.w["out_head.weight"].t()

    def seed_cache(self, batch: int, length: int, generator: torch.Generator):
        """Fill every layer's K/V with `length` random positions (synthetic
        decode context: a decode step costs the same whatever the values)."""
        c = self.cfg
        shape = (batch, length, c.n_kv_heads, c.head_dim)
        for i in range(c.n_layers):
            self.k[i] = torch.randn(shape, generator=generator).to(self.dt)
            self.v[i] = torch.randn(shape, generator=generator).to(self.dt)
