"""FastQwen3: Qwen3-0.6B-architecture decoder on the gfx950 kernels
(reference: examples/LLM/fastqwen3.py:15-189).

Module tree and names follow the reference (tok_embed, transformer_blocs[i].
{attn, rms_norm1, rms_norm2, ffn.{fused_linear_layer1, linear_layerP,
linear_layer2}}, final_rmsnorm, out_head), with the FFN computing the SwiGLU
it intends, down(silu(gate(x)) * up(x)) (the committed FFN feeds the
3072-wide SiLU output into a 1024-input layer, fastqwen3.py:71-73).

Execution:
  * forward_impl keeps the residual stream in one buffer. For prefill it
    fuses each residual add into the next RMSNorm; for <= 16 tokens
    (decode) each RMSNorm is fused into the GEMV that reads it, each
    residual add into the kernel that writes it, the QK-norm + RoPE +
    KV-append of the new token, the output projection and its residual add
    into the decode attention kernel, and the whole FFN half (RMSNorm,
    SwiGLU gate/up, down, residual add) into one launch, so a layer is 3
    kernels: QKV GEMV, split-KV attention + o_proj, FFN.
  * GreedyDecoder captures one whole decode step (28 layers, lm_head,
    argmax, position advance) into a HIP graph and replays it per token, so
    the token loop issues one launch per token and never synchronises.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from torchplusplus_amd import prepare_device
from torchplusplus_amd._native import ext as _ext
from torchplusplus_amd.attention.gqa import GroupedQueryAttention
from torchplusplus_amd.dlops.derived import DerivedWeight, attach
from torchplusplus_amd.dlops.linear import (GEMV_MAX_ROWS, LinearSILU, interleave_gate_up,
                                             linear, swiglu)
from torchplusplus_amd.dlops.normalization import RmsNormFused
from torchplusplus_amd.dlops.rope import compute_rope_params
from torchplusplus_amd.llmops.kvcache import KVCache
from torchplusplus_amd.llmops.llm import LLMInference

_C = _ext()


def check_decode_errors(like: torch.Tensor) -> None:
    """Raise if a one-launch decode kernel on `like`'s device (the decode FFN,
    the decode attention with the output projection) gave up waiting for its
    workgroups since the last check (they need all 256 resident at once; the
    output is then wrong). Clears the flags and the workspace counters.
    Synchronises the current stream."""
    bad = [n for n, f in (("ffn_decode", _C.ffn_decode_sync_errors),
                          ("attn_decode_oproj", _C.attn_decode_sync_errors)) if f(like)]
    if bad:
        raise RuntimeError(
            f"{', '.join(bad)}: a one-launch decode kernel gave up waiting for its 256 workgroups "
            "(not all were resident at once, e.g. other work held CUs), so tokens decoded since "
            "the last check are wrong; the workspaces were reset, decode again")


@dataclass
class QwenConfig:
    """Qwen3-0.6B shape (fastqwen3.py:15-27); bf16 by default."""

    vocab_size: int = 151936
    context_length: int = 32768
    embed_dim: int = 1024
    n_heads: int = 16
    n_layers: int = 28
    head_dim: int = 128
    n_kv_heads: int = 8
    hidden_dim: int = 3072
    qk_norm: bool = True
    rope_base: float = 1e6
    dtype: torch.dtype = torch.bfloat16


@dataclass
class QwenConfig_float16(QwenConfig):  # noqa: N801  (reference name)
    dtype: torch.dtype = torch.float16


class FFN(nn.Module):
    """SwiGLU FFN: linear_layer2(silu(fused_linear_layer1(x)) * linear_layerP(x)).
    Runs as one fused gate/up kernel plus the down projection. The gate/up
    weights are interleaved on first use and again whenever either changes
    (load_state_dict, in-place edits)."""

    def __init__(self, in_dim: int, hidden_dim: int, dtype=torch.float16, device=None):
        super().__init__()
        self.fused_linear_layer1 = LinearSILU(in_dim, hidden_dim, dtype=dtype, device=device)
        self.linear_layerP = nn.Linear(in_dim, hidden_dim, bias=False, dtype=dtype, device=device)
        self.linear_layer2 = nn.Linear(hidden_dim, in_dim, bias=False, dtype=dtype, device=device)
        self._w_gu = attach(self, DerivedWeight(interleave_gate_up))

    def refresh_fused_weights(self):
        """Force a rebuild of the interleaved gate/up weight."""
        self._w_gu.invalidate()
        self.w_gu()

    def w_gu(self) -> torch.Tensor:
        return self._w_gu.get(self.fused_linear_layer1.weight, self.linear_layerP.weight)

    def forward(self, x):
        return linear(swiglu(x, self.w_gu()), self.linear_layer2.weight)


class Transformer(nn.Module):
    """Decoder block (fastqwen3.py:81-118)."""

    def __init__(self, cfg: QwenConfig, device=None):
        super().__init__()
        self.attn = GroupedQueryAttention(d_in=cfg.embed_dim, num_heads=cfg.n_heads,
                                          head_dim=cfg.head_dim, n_kv_heads=cfg.n_kv_heads,
                                          qk_norm=cfg.qk_norm, dtype=cfg.dtype, device=device)
        self.rms_norm1 = RmsNormFused(cfg.embed_dim, eps=1e-6, dtype=cfg.dtype, device=device)
        self.rms_norm2 = RmsNormFused(cfg.embed_dim, eps=1e-6, dtype=cfg.dtype, device=device)
        self.ffn = FFN(cfg.embed_dim, cfg.hidden_dim, dtype=cfg.dtype, device=device)

    def forward(self, x, cos, sin, kv_cache: Optional[KVCache] = None,
                cache_position: Optional[int] = None):
        x = x + self.attn(self.rms_norm1(x), cos, sin, kv_cache, cache_position)
        return x + self.ffn(self.rms_norm2(x))


class FastQwen3(LLMInference):
    def __init__(self, cfg: QwenConfig, device=None, rope_context: Optional[int] = None):
        super().__init__()
        self.cfg = cfg
        dev = device
        self.tok_embed = nn.Embedding(cfg.vocab_size, cfg.embed_dim, dtype=cfg.dtype, device=dev)
        self.transformer_blocs = nn.ModuleList([Transformer(cfg, dev) for _ in range(cfg.n_layers)])
        self.final_rmsnorm = RmsNormFused(cfg.embed_dim, dtype=cfg.dtype, device=dev)
        self.out_head = nn.Linear(cfg.embed_dim, cfg.vocab_size, bias=False, dtype=cfg.dtype,
                                  device=dev)
        ctx = rope_context or cfg.context_length
        cos, sin = compute_rope_params(self.get_head_dim(), cfg.rope_base, ctx,
                                       device=dev if dev is not None else "cpu")
        self.register_buffer("cos", cos, persistent=False)
        self.register_buffer("sin", sin, persistent=False)

    @torch.no_grad()
    def init_weights(self, std: float = 0.02, generator: Optional[torch.Generator] = None):
        """Random init used by the benchmark: linear/embedding weights
        ~N(0, std), norm weights 1; refreshes the fused weights."""
        for mod in self.modules():
            if isinstance(mod, (nn.Linear, nn.Embedding, LinearSILU)):
                mod.weight.normal_(0.0, std, generator=generator)
            elif isinstance(mod, (nn.RMSNorm, RmsNormFused)):
                mod.weight.fill_(1.0)
        self.refresh_fused_weights()

    def refresh_fused_weights(self):
        for blk in self.transformer_blocs:
            blk.attn.refresh_fused_weights()
            blk.ffn.refresh_fused_weights()

    def check_device_errors(self):
        if self.out_head.weight.is_cuda:
            check_decode_errors(self.out_head.weight)

    def get_num_layers(self) -> int:
        return self.cfg.n_layers

    def get_kv_heads(self) -> int:
        return self.cfg.n_kv_heads

    def get_head_dim(self) -> int:
        return self.cfg.head_dim if self.cfg.head_dim is not None else self.cfg.embed_dim // self.cfg.n_heads

    def get_dtype(self) -> torch.dtype:
        return self.cfg.dtype

    def forward_impl(self, input_ids: torch.Tensor, kv_caches: Optional[List[KVCache]] = None,
                     cache_position: Optional[int] = None, last_only: bool = False) -> torch.Tensor:
        blocks = self.transformer_blocs
        resid = F.embedding(input_ids, self.tok_embed.weight)  # residual stream, updated in place
        if input_ids.numel() <= GEMV_MAX_ROWS:
            return self._forward_small(resid, kv_caches, cache_position)
        h = blocks[0].rms_norm1(resid)
        for i, blk in enumerate(blocks):
            kv = kv_caches[i] if kv_caches is not None else None
            a = blk.attn(h, self.cos, self.sin, kv, cache_position)
            h = blk.rms_norm2.forward_add(a, resid)
            f = blk.ffn(h)
            nxt = blocks[i + 1].rms_norm1 if i + 1 < len(blocks) else self.final_rmsnorm
            h = nxt.forward_add(f, resid)
        if last_only:
            h = h[:, -1:, :].contiguous()
        return linear(h, self.out_head.weight)

    def _forward_small(self, resid, kv_caches, cache_position):
        """<= 16 tokens (decode): every RMSNorm is fused into the GEMV that
        consumes it and every residual add into the GEMV that produces it."""
        for i, blk in enumerate(self.transformer_blocs):
            at, n1, n2 = blk.attn, blk.rms_norm1, blk.rms_norm2
            kv = kv_caches[i] if kv_caches is not None else None
            qkv = _C.gemv_fused(resid, at.fused_qkv_weight(), n1.weight, n1.eps)
            if kv is not None and resid.shape[1] == 1:
                at.attend_oproj(qkv, self.cos, self.sin, kv, cache_position, resid)
            else:
                o = at.attend(qkv, self.cos, self.sin, kv, cache_position)
                _C.gemv_fused(o, at.out_projection.weight, None, 1e-6, resid)
            _C.ffn_decode(resid, n2.weight, n2.eps, blk.ffn.w_gu(), blk.ffn.linear_layer2.weight)
        return _C.gemv_fused(resid, self.out_head.weight, self.final_rmsnorm.weight,
                             self.final_rmsnorm.eps)

    @torch.inference_mode()
    def generate_greedy(self, input_ids: torch.Tensor, max_new_token: int,
                        use_graph: bool = True) -> torch.Tensor:
        """Greedy generation: prefill, then one captured decode graph per token."""
        bsz, seq_len = input_ids.shape
        self.setup_kv_cache(seq_len + max_new_token, bsz)
        self.reset_kv_cache()
        logits = self.forward_impl(input_ids, self.kv_cache_array, 0, last_only=True)
        first = _C.argmax_rows(logits[:, -1, :].contiguous())
        dec = GreedyDecoder(self, bsz)
        toks = dec.run(first, seq_len, max_new_token - 1, use_graph=use_graph)
        return torch.cat([input_ids, first.view(bsz, 1), toks], dim=1)


class GreedyDecoder:
    """One greedy decode step for every sequence of the batch, on static
    buffers so it can be captured in a HIP graph:
      resid [B, 1, E] (embedding of the current token) -> 28 blocks (GEMV
      projections, fused QK-norm/RoPE/KV append at `positions`, split-KV
      attention over `seqlens` keys) -> lm_head GEMV + argmax -> ids, and the
      next token's embedding gathered into resid; positions, seqlens += 1."""

    def __init__(self, model: FastQwen3, batch_size: int):
        self.m = model
        self.B = batch_size
        dev = model.out_head.weight.device
        emb = model.tok_embed.weight
        self.ids = torch.zeros(batch_size, 1, dtype=torch.long, device=dev)
        self.resid = torch.zeros(batch_size, 1, emb.shape[1], dtype=emb.dtype, device=dev)
        self.positions = torch.zeros(batch_size, dtype=torch.int32, device=dev)
        self.seqlens = torch.zeros(batch_size, dtype=torch.int32, device=dev)
        self.graph = None
        self.caches = model.kv_cache_array
        assert self.caches is not None, "setup_kv_cache() first"

    def step(self):
        m, B, resid = self.m, self.B, self.resid
        for i, blk in enumerate(m.transformer_blocs):
            at, n1, n2 = blk.attn, blk.rms_norm1, blk.rms_norm2
            kc, vc = self.caches[i].k_cache[:B], self.caches[i].v_cache[:B]
            qkv = _C.gemv_fused(resid, at.fused_qkv_weight(), n1.weight, n1.eps)
            at.decode_oproj(qkv, m.cos, m.sin, kc, vc, self.seqlens, resid)
            _C.ffn_decode(resid, n2.weight, n2.eps, blk.ffn.w_gu(), blk.ffn.linear_layer2.weight)
        fn = m.final_rmsnorm
        _C.greedy_step(resid, m.out_head.weight, fn.weight, fn.eps, m.tok_embed.weight,
                       self.ids, resid, self.positions, self.seqlens)

    def prepare(self, first_tokens: torch.Tensor, position: int):
        self.ids.copy_(first_tokens.view(self.B, 1))
        self.resid.copy_(F.embedding(self.ids, self.m.tok_embed.weight))
        self.positions.fill_(position)
        self.seqlens.fill_(position + 1)
        for c in self.caches:
            c.cache_len = max(c.cache_len, position)

    def capture(self):
        """Run the device checks, warm up once on a side stream (creating the
        kernels' workspaces outside the capture), restore the state, then
        capture."""
        prepare_device(self.ids.device)
        saved = (self.ids.clone(), self.resid.clone(), self.positions.clone(),
                 self.seqlens.clone())
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.step()
        torch.cuda.current_stream().wait_stream(s)
        self.ids.copy_(saved[0])
        self.resid.copy_(saved[1])
        self.positions.copy_(saved[2])
        self.seqlens.copy_(saved[3])
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.step()

    def replay(self):
        if self.graph is not None:
            self.graph.replay()
        else:
            self.step()

    def run(self, first_tokens: torch.Tensor, position: int, n_steps: int,
            use_graph: bool = True) -> torch.Tensor:
        """Decode n_steps tokens after `first_tokens` sits at `position`;
        returns [B, n_steps]."""
        out = torch.empty(self.B, n_steps, dtype=torch.long, device=self.ids.device)
        self.prepare(first_tokens, position)
        if use_graph and self.graph is None and n_steps > 0:
            self.capture()
        for t in range(n_steps):
            self.replay()
            out[:, t] = self.ids[:, 0]
        for c in self.caches:
            c.cache_len = position + n_steps
        if n_steps > 0:
            check_decode_errors(self.ids)
        return out
