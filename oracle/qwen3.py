"""CPU restatement of the FastQwen3 forward (test infrastructure only).

Follows examples/LLM/fastqwen3.py:81-189 with the reference's eager data flow:
every op computes in fp32 from the model-dtype inputs and rounds its output
to the model dtype, as the eager PyTorch modules would:
  block: x = x + attn(rms_norm1(x)); x = x + ffn(rms_norm2(x))   (:107-116)
  attn (torchpp/attention/gqa.py:80-131): q/k/v projections, QK-RMSNorm over
       head_dim (:90-94), rotate-half RoPE at the absolute positions
       cache_pos.. (:106-113), K/V appended to the cache (:115-116), causal
       GQA attention over the cache prefix (:118-128), output projection
  ffn: linear_layer2(silu(fused_linear_layer1(x)) * linear_layerP(x)) -- the
       SwiGLU the reference intends (its committed shapes at :71-73 cannot run)
  logits = out_head(final_rmsnorm(x))                              (:187-188)
It reads the weights of a torchplusplus_amd FastQwen3 through its state dict.
With cfg.dtype = float32 no rounding happens at all (the form the CPU pin
tests compare against an fp64 assembly of torch library routines).

Each stage is its own method so a test can plant a mistake in one stage of a
copy (a subclass) and show that the pins reject it.
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

    # ---- one op each --------------------------------------------------------
    def _lin(self, x, name):
        return _r(x @ self.w[name].t(), self.dt)

    def _norm(self, x, name):
        return ops.rmsnorm(x.to(self.dt), self.w[name].to(self.dt), 1e-6).float()

    def _positions(self, start: int, S: int) -> slice:
        """Rows of the RoPE tables for tokens placed at start.. (gqa.py:106-110)."""
        return slice(start, start + S)

    def _rope(self, t, pos: slice):
        """t [B, S, H, D] -> rotate-half RoPE with table rows `pos`."""
        return ops.rope(t.to(self.dt).transpose(1, 2), self.cos[pos], self.sin[pos]).transpose(1, 2)

    # ---- stages -------------------------------------------------------------
    def _qk(self, i, q, k, start):
        """QK-RMSNorm over head_dim, then RoPE (gqa.py:90-113)."""
        p = f"transformer_blocs.{i}.attn."
        if self.cfg.qk_norm:
            q = self._norm(q, p + "q_norm.weight")
            k = self._norm(k, p + "k_norm.weight")
        pos = self._positions(start, q.shape[1])
        return self._rope(q, pos), self._rope(k, pos)

    def _attn(self, i, h, start):
        c = self.cfg
        B, S = h.shape[:2]
        p = f"transformer_blocs.{i}.attn."
        q = self._lin(h, p + "Wq.weight").view(B, S, c.n_heads, c.head_dim)
        k = self._lin(h, p + "Wk.weight").view(B, S, c.n_kv_heads, c.head_dim)
        v = self._lin(h, p + "Wv.weight").view(B, S, c.n_kv_heads, c.head_dim)
        q, k = self._qk(i, q, k, start)
        v = v.to(self.dt)
        if start == 0:
            self.k[i], self.v[i] = k, v
        else:  # KVCache.update appends at cache_len (kvcache.py:50-108)
            self.k[i] = torch.cat([self.k[i], k], 1)
            self.v[i] = torch.cat([self.v[i], v], 1)
        o = ops.attention(q, self.k[i], self.v[i], causal=True).float()
        return self._lin(o.reshape(B, S, -1), p + "out_projection.weight")

    def _ffn(self, i, h):
        p = f"transformer_blocs.{i}.ffn."
        g = self._lin(h, p + "fused_linear_layer1.weight")
        g = _r(ops.activation(g, "silu"), self.dt)
        u = self._lin(h, p + "linear_layerP.weight")
        return self._lin(_r(g * u, self.dt), p + "linear_layer2.weight")

    def _block(self, i, x, start):
        """fastqwen3.py:107-116."""
        p = f"transformer_blocs.{i}."
        a = self._attn(i, self._norm(x, p + "rms_norm1.weight"), start)
        x = _r(x + a, self.dt)
        f = self._ffn(i, self._norm(x, p + "rms_norm2.weight"))
        return _r(x + f, self.dt)

    def _head(self, x):
        """fastqwen3.py:187-188."""
        return self._norm(x, "final_rmsnorm.weight") @ self.w["out_head.weight"].t()

    def forward(self, ids: torch.Tensor, start: int) -> torch.Tensor:
        """Logits [B, S, V] (fp32) for `ids` placed at positions start..;
        keeps K/V for later calls (start must equal the cached length)."""
        x = _r(self.w["tok_embed.weight"][ids], self.dt)
        for i in range(self.cfg.n_layers):
            x = self._block(i, x, start)
        return self._head(x)

    def seed_cache(self, batch: int, length: int, generator: torch.Generator):
        """Fill every layer's K/V with `length` random positions (synthetic
        decode context: a decode step costs the same whatever the values)."""
        c = self.cfg
        shape = (batch, length, c.n_kv_heads, c.head_dim)
        for i in range(c.n_layers):
            self.k[i] = torch.randn(shape, generator=generator).to(self.dt)
            self.v[i] = torch.randn(shape, generator=generator).to(self.dt)
