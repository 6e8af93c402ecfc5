"""BASELINE config 5 at its full shape: the random-init Qwen3-0.6B-architecture
decoder (28 layers, hidden 1024, 16/8 heads, head_dim 128, SwiGLU 3072,
vocab 151936, bf16, weights ~N(0, 0.02), norms 1).

  * batch 8, prefill 2048 random ids: finite logits; graph greedy decode ==
    eager greedy decode token for token over 9 steps; the first generated
    token is the argmax of the prefill's last logits.
  * against the CPU model oracle through all 28 layers: the last-position
    logits of a 256-token prefill of one sequence and 2 teacher-forced
    decode steps after it (tolerance as in test_model.py).
"""
import pytest
import torch

from oracle.qwen3 import Qwen3Oracle
from tests.test_model import model_close
from torchplusplus_amd.fastqwen3 import FastQwen3, QwenConfig

pytestmark = pytest.mark.gpu

CFG = QwenConfig()
ROPE_CTX = 4096


@pytest.fixture(scope="module")
def model(dev):
    m = FastQwen3(CFG, device=dev, rope_context=ROPE_CTX).eval()
    m.init_weights(std=0.02, generator=torch.Generator(device=dev).manual_seed(0))
    return m


@torch.inference_mode()
def test_config5_prefill_and_greedy_decode(dev, model):
    B, S, N = 8, 2048, 9
    ids = torch.randint(0, CFG.vocab_size, (B, S), generator=torch.Generator().manual_seed(1)).to(dev)
    graph = model.generate_greedy(ids, N, use_graph=True)
    eager = model.generate_greedy(ids, N, use_graph=False)
    assert graph.shape == (B, S + N)
    assert torch.equal(graph, eager), "graph and eager greedy decode differ"
    model.setup_kv_cache(S + N, B)
    model.reset_kv_cache()
    logits = model.forward_impl(ids, model.kv_cache_array, 0, last_only=True)
    assert torch.isfinite(logits.float()).all()
    assert torch.equal(graph[:, S], logits[:, -1].float().argmax(-1))


@torch.inference_mode()
def test_config5_against_oracle(dev, model):
    S = 256
    ids = torch.randint(0, CFG.vocab_size, (1, S + 2), generator=torch.Generator().manual_seed(2))
    model.setup_kv_cache(S + 2, 1)
    model.reset_kv_cache()
    orc = Qwen3Oracle(model.state_dict(), CFG, ROPE_CTX)
    got = model.forward(ids[:, :S].to(dev), use_cache=True, cache_position=0)
    exp = orc.forward(ids[:, :S], 0)
    model_close(got[:, -1], exp[:, -1], "config 5 prefill, last position")
    for t in range(2):
        got = model.forward(ids[:, S + t:S + t + 1].to(dev), use_cache=True, cache_position=S + t)
        exp = orc.forward(ids[:, S + t:S + t + 1], S + t)
        model_close(got, exp, f"config 5 decode step {t}")
