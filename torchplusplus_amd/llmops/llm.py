"""LLM inference base class (reference: torchpp/llmops/llm.py:9-326).

Same abstract interface (forward_impl, get_num_layers, get_kv_heads,
get_head_dim, get_dtype), cache management, samplers and generate(). Fixes:
batch > 1 works (the reference's _should_stop calls token.item(),
llm.py:212), the stop check only synchronises with the device when there is
something to check (eos or stop tokens), top-p filtering is the standard
nucleus rule (llm.py:135-137 index with `... : -1`), get_cache_info reads the
caches that exist (llm.py:291 reads a missing attribute), and the prefill in
generate() computes logits for the last position only (the only ones used).
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Callable, List, Optional

import torch
import torch.nn as nn

from torchplusplus_amd.llmops.kvcache import KVCache


class LLMInference(nn.Module, ABC):
    def __init__(self):
        super().__init__()
        self.kv_cache_array: Optional[List[KVCache]] = None

    @abstractmethod
    def forward_impl(self, input_ids: torch.Tensor, kv_caches: Optional[List[KVCache]] = None,
                     cache_position: Optional[int] = None, last_only: bool = False) -> torch.Tensor:
        """Logits [B, S, vocab] (or [B, 1, vocab] with last_only)."""

    @abstractmethod
    def get_num_layers(self) -> int: ...

    @abstractmethod
    def get_kv_heads(self) -> int: ...

    @abstractmethod
    def get_head_dim(self) -> int: ...

    @abstractmethod
    def get_dtype(self) -> torch.dtype: ...

    def _device(self):
        return next(self.parameters()).device

    def setup_kv_cache(self, max_seq_len: int, batch_size: Optional[int] = None):
        """One KVCache per layer (llm.py:52-71). Reuses existing caches when
        they are large enough, so repeated generate() calls do not reallocate."""
        if self.kv_cache_array is not None and all(
                c.max_seq_len >= max_seq_len for c in self.kv_cache_array) and (
                batch_size is None or all(c.batch_size >= batch_size for c in self.kv_cache_array)):
            return
        dev = self._device()
        self.kv_cache_array = [
            KVCache(max_seq_len, self.get_kv_heads(), self.get_head_dim(), self.get_dtype(), dev,
                    batch_size)
            for _ in range(self.get_num_layers())
        ]

    def reset_kv_cache(self):
        if self.kv_cache_array:
            for c in self.kv_cache_array:
                c.reset()

    def clear_kv_cache(self):
        """Drop the caches and free their memory (llm.py:79-88)."""
        self.kv_cache_array = None
        torch.cuda.empty_cache()

    def forward(self, input_ids: torch.Tensor, use_cache: bool = False,
                cache_position: Optional[int] = None) -> torch.Tensor:
        if use_cache and self.kv_cache_array is None:
            raise ValueError(
                "KV cache is not initialized , call setup_kv_cache() or use normal nn.Module")
        return self.forward_impl(input_ids, self.kv_cache_array if use_cache else None,
                                 cache_position)

    # ---- samplers (llm.py:114-186) -------------------------------------------
    def sample_top_p(self, logits, top_p: float = 0.9, temp: float = 1.0,
                     filter_value: float = -float("inf")):
        logits = logits.float() / temp
        if top_p < 1.0:
            sorted_logits, sorted_idx = torch.sort(logits, descending=True, dim=-1)
            cum = torch.cumsum(torch.softmax(sorted_logits, dim=-1), dim=-1)
            remove = cum > top_p
            remove[..., 1:] = remove[..., :-1].clone()  # keep the token that crosses top_p
            remove[..., 0] = False
            logits = logits.masked_fill(remove.scatter(-1, sorted_idx, remove), filter_value)
        return torch.multinomial(torch.softmax(logits, dim=-1), num_samples=1)

    def sample_top_k(self, logits, top_k: int = 50, temp: float = 1.0,
                     filter_value: float = -float("inf")):
        logits = logits.float() / temp
        top_k = min(top_k, logits.size(-1))
        values, idx = torch.topk(logits, top_k)
        filtered = torch.full_like(logits, filter_value).scatter_(-1, idx, values)
        return torch.multinomial(torch.softmax(filtered, dim=-1), num_samples=1)

    def sample_greedy(self, logits):
        return torch.argmax(logits, dim=-1, keepdim=True)

    def _sample_token(self, logits, temperature, top_p, top_k, strategy):
        if strategy == "greedy":
            return self.sample_greedy(logits)
        if strategy == "top_k" and top_k is not None:
            return self.sample_top_k(logits, top_k, temperature)
        if strategy == "top_p":
            return self.sample_top_p(logits, top_p, temperature)
        raise ValueError(f"Unknown sampling strategy: {strategy}")

    def check_device_errors(self):
        """Raise if the device reported a failed launch during the last
        generation (models with kernels that can detect one override this;
        called once at the end of generate(), where it synchronises)."""

    def _should_stop(self, token, stop_token_ids: List[int], eos_token_id: Optional[int]) -> bool:
        """True when every sequence of the batch produced EOS or a stop token."""
        ids = list(stop_token_ids) + ([eos_token_id] if eos_token_id is not None else [])
        if not ids:
            return False  # nothing to check: no device synchronisation
        stop = torch.zeros_like(token, dtype=torch.bool)
        for t in ids:
            stop |= token == t
        return bool(stop.all())

    @torch.inference_mode()
    def generate(self, input_ids: torch.Tensor, max_new_token: int = 100, temp: float = 1.0,
                 top_p: float = 0.9, top_k: Optional[int] = None,
                 sampling_strategy: str = "top_p", stop_token_ids: Optional[List[int]] = None,
                 eos_token_id: Optional[int] = None, stream: bool = False,
                 stream_callback: Optional[Callable[[torch.Tensor], None]] = None):
        """Prefill then token-by-token decode (llm.py:225-286)."""
        batch_size, seq_len = input_ids.shape
        self.setup_kv_cache(seq_len + max_new_token, batch_size)
        self.reset_kv_cache()
        stop_token_ids = stop_token_ids or []

        logits = self.forward_impl(input_ids, self.kv_cache_array, 0, last_only=True)
        next_token = self._sample_token(logits[:, -1, :], temp, top_p, top_k, sampling_strategy)
        if stream and stream_callback:
            stream_callback(next_token)
        generated = [next_token]
        if not self._should_stop(next_token, stop_token_ids, eos_token_id):
            for i in range(max_new_token - 1):
                logits = self.forward_impl(next_token, self.kv_cache_array, seq_len + i)
                next_token = self._sample_token(logits[:, -1, :], temp, top_p, top_k,
                                                sampling_strategy)
                if stream and stream_callback:
                    stream_callback(next_token)
                generated.append(next_token)
                if self._should_stop(next_token, stop_token_ids, eos_token_id):
                    break
        self.check_device_errors()
        return torch.cat([input_ids] + generated, dim=1)

    def get_cache_info(self) -> dict:
        if not self.kv_cache_array:
            return {"initialized": False}
        c = self.kv_cache_array[0]
        return {"initialized": True, "num_layers": len(self.kv_cache_array),
                "cache_length": c.cache_len, "max_seq_len": c.max_seq_len,
                "n_kv_heads": c.n_kv_heads, "head_dim": c.head_dim}

    def estimate_memory_usage(self, max_seq_len: int, batch_size: int = 1) -> dict:
        elt = torch.empty((), dtype=self.get_dtype()).element_size()
        per_layer = 2 * batch_size * self.get_kv_heads() * max_seq_len * self.get_head_dim() * elt
        total = per_layer * self.get_num_layers()
        return {"total_bytes": total, "total_mb": total / 1024 ** 2, "total_gb": total / 1024 ** 3,
                "per_layer_mb": per_layer / 1024 ** 2, "num_layers": self.get_num_layers()}
