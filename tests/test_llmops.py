"""Host logic of the LLM runtime on the CPU: KVCache bookkeeping and the
generate() loop of LLMInference with a tiny CPU model (no kernels)."""
import pytest
import torch

from torchplusplus_amd.llmops.kvcache import KVCache
from torchplusplus_amd.llmops.llm import LLMInference


def test_kvcache_append_and_prefix_views():
    c = KVCache(max_seq_len=10, n_kv_heads=2, head_dim=4, dtype=torch.float32, device="cpu")
    k = torch.randn(3, 2, 4, 4)
    v = torch.randn(3, 2, 4, 4)
    kc, vc = c.update(k, v)
    assert c.cache_len == 4 and kc.shape == (3, 2, 4, 4) and torch.equal(kc, k)
    k2 = torch.randn(3, 2, 1, 4)
    kc, vc = c.update(k2, k2)
    assert c.cache_len == 5 and torch.equal(kc[:, :, 4:], k2) and torch.equal(kc[:, :, :4], k)
    assert kc.data_ptr() == c.k_cache.data_ptr()  # a view, no copy
    kc, _ = c.update(k2 * 2, k2, index=7)
    assert c.cache_len == 8 and torch.equal(kc[:, :, 7:8], k2 * 2)
    c.reset()
    assert c.cache_len == 0 and float(c.k_cache.abs().sum()) == 0


def test_kvcache_overflow_raises():
    c = KVCache(max_seq_len=4, n_kv_heads=1, head_dim=2, dtype=torch.float32, device="cpu")
    c.update(torch.zeros(1, 1, 3, 2), torch.zeros(1, 1, 3, 2))
    with pytest.raises(ValueError, match="overflow"):
        c.update(torch.zeros(1, 1, 2, 2), torch.zeros(1, 1, 2, 2))


class TinyLM(LLMInference):
    """Deterministic CPU model: next-token logits favour (last_id + 1) % V."""

    V = 11

    def __init__(self):
        super().__init__()
        self.p = torch.nn.Parameter(torch.zeros(1))
        self.calls = []

    def forward_impl(self, input_ids, kv_caches=None, cache_position=None, last_only=False):
        self.calls.append((tuple(input_ids.shape), cache_position))
        if kv_caches is not None:
            for c in kv_caches:
                z = torch.zeros(input_ids.shape[0], 1, input_ids.shape[1], 2)
                c.update(z, z)
        logits = torch.nn.functional.one_hot((input_ids + 1) % self.V, self.V).float() * 5
        return logits[:, -1:] if last_only else logits

    def get_num_layers(self):
        return 2

    def get_kv_heads(self):
        return 1

    def get_head_dim(self):
        return 2

    def get_dtype(self):
        return torch.float32


def test_generate_greedy_batch_and_positions():
    m = TinyLM()
    ids = torch.tensor([[1, 2, 3], [5, 6, 7]])
    out = m.generate(ids, max_new_token=4, sampling_strategy="greedy")
    assert out.tolist() == [[1, 2, 3, 4, 5, 6, 7], [5, 6, 7, 8, 9, 10, 0]]
    assert [c[1] for c in m.calls] == [0, 3, 4, 5]
    assert m.kv_cache_array[0].cache_len == 6
    assert m.get_cache_info()["cache_length"] == 6


def test_generate_stops_when_all_sequences_hit_eos():
    m = TinyLM()
    ids = torch.tensor([[1], [1]])
    out = m.generate(ids, max_new_token=10, sampling_strategy="greedy", eos_token_id=4)
    assert out.shape[1] == 1 + 3  # tokens 2, 3, 4 then stop


def test_samplers_respect_filters():
    m = TinyLM()
    torch.manual_seed(0)
    logits = torch.tensor([[0.0, 10.0, 9.0, -5.0]])
    for _ in range(20):
        assert m.sample_top_k(logits, top_k=2).item() in (1, 2)
        assert m.sample_top_p(logits, top_p=0.5).item() == 1
    assert m.sample_greedy(logits).item() == 1
    with pytest.raises(ValueError):
        m._sample_token(logits, 1.0, 0.9, None, "beam")


def test_use_cache_without_setup_raises_and_memory_estimate():
    m = TinyLM()
    with pytest.raises(ValueError, match="setup_kv_cache"):
        m(torch.tensor([[1]]), use_cache=True, cache_position=0)
    est = m.estimate_memory_usage(max_seq_len=100, batch_size=2)
    assert est["total_bytes"] == 2 * 2 * 2 * 1 * 100 * 2 * 4
    assert m.get_cache_info() == {"initialized": False}
