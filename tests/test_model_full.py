"""BASELINE config 5 at its full shape: the random-init Qwen3-0.6B-architecture
decoder (28 layers, hidden 1024, 16/8 heads, head_dim 128, SwiGLU 3072,
vocab 151936, bf16, weights ~N(0, 0.02), norms 1).

  * batch 8, prefill 2048 random ids: finite logits; graph greedy decode ==
    eager greedy decode token for token over 9 steps; the first generated
    token is the argmax of the prefill's last logits.
  * against the CPU model oracle through all 28 layers: the last-position
    logits of a 256-token prefill of one sequence and 2 teacher-forced
    decode steps after it.

Tolerance through 28 layers: bf16 rounding at every op boundary makes the
eager bf16 computation itself drift from the exact one; with these weights
the bf16 oracle's logits differ from the same oracle run in fp32 by ~1.4%
(relative Frobenius), so a GPU result may differ from the bf16 oracle by as
much. The check is therefore two-sided: per logit within atol 6e-2 / rtol
2e-2 of the bf16 oracle, and the GPU's relative error against the fp32
oracle at most 1.25x the bf16 oracle's own plus 2e-3 (as close to the exact
result as the eager bf16 reference is).
"""
import pytest
import torch

from oracle.qwen3 import Qwen3Oracle
from tests.conftest import close
from tests.test_model import MODEL_ATOL, MODEL_RTOL
from torchplusplus_amd.fastqwen3 import FastQwen3, QwenConfig, QwenConfig_float16

pytestmark = pytest.mark.gpu

CFG = QwenConfig()
ROPE_CTX = 4096


@pytest.fixture(scope="module")
def model(dev):
    m = FastQwen3(CFG, device=dev, rope_context=ROPE_CTX).eval()
    m.init_weights(std=0.02, generator=torch.Generator(device=dev).manual_seed(0))
    return m


def _prefill_and_greedy_decode(dev, model, cfg):
    B, S, N = 8, 2048, 9
    ids = torch.randint(0, cfg.vocab_size, (B, S), generator=torch.Generator().manual_seed(1)).to(dev)
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
def test_config5_prefill_and_greedy_decode(dev, model):
    _prefill_and_greedy_decode(dev, model, CFG)


@torch.inference_mode()
def test_config5_fp16_prefill_and_greedy_decode(dev):
    """The same at the reference's own dtype (QwenConfig_float16,
    examples/LLM/fastqwen3.py:15-27)."""
    cfg = QwenConfig_float16()
    m = FastQwen3(cfg, device=dev, rope_context=ROPE_CTX).eval()
    m.init_weights(std=0.02, generator=torch.Generator(device=dev).manual_seed(0))
    _prefill_and_greedy_decode(dev, m, cfg)
    del m
    torch.cuda.empty_cache()


def _rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return ((a - b).norm() / b.norm()).item()


def _check(got, exp16, exp32, what):
    close(got, exp16, atol=MODEL_ATOL, rtol=MODEL_RTOL, what=what)
    e_gpu, e_orc = _rel(got, exp32), _rel(exp16, exp32)
    assert e_gpu <= 1.25 * e_orc + 2e-3, \
        f"{what}: error vs fp32 {e_gpu:.4f}, bf16 oracle's own {e_orc:.4f}"


@torch.inference_mode()
def test_config5_against_oracle(dev, model):
    S = 256
    ids = torch.randint(0, CFG.vocab_size, (1, S + 2), generator=torch.Generator().manual_seed(2))
    model.setup_kv_cache(S + 2, 1)
    model.reset_kv_cache()
    orc16 = Qwen3Oracle(model.state_dict(), CFG, ROPE_CTX)
    cfg32 = QwenConfig(dtype=torch.float32)
    orc32 = Qwen3Oracle({}, cfg32, ROPE_CTX)
    orc32.w = orc16.w  # the same (bf16-valued) weights, no rounding anywhere
    got = model.forward(ids[:, :S].to(dev), use_cache=True, cache_position=0)
    _check(got[:, -1], orc16.forward(ids[:, :S], 0)[:, -1], orc32.forward(ids[:, :S], 0)[:, -1],
           "config 5 prefill, last position")
    for t in range(2):
        step = ids[:, S + t:S + t + 1]
        got = model.forward(step.to(dev), use_cache=True, cache_position=S + t)
        _check(got, orc16.forward(step, S + t), orc32.forward(step, S + t),
               f"config 5 decode step {t}")


@torch.inference_mode()
def test_config5_batch8_against_oracle(dev, model):
    """The benchmark's batch (8 sequences) through all 28 layers against the
    CPU oracle: last-position prefill logits of a 256-token prefix and 2
    teacher-forced decode steps, which run the decode kernels the benchmark
    times (the folded attention + output projection with 4 splits per
    sequence, the one-launch FFN) on every sequence; same two-sided check."""
    B, S = 8, 256
    ids = torch.randint(0, CFG.vocab_size, (B, S + 2), generator=torch.Generator().manual_seed(3))
    model.setup_kv_cache(S + 2, B)
    model.reset_kv_cache()
    orc16 = Qwen3Oracle(model.state_dict(), CFG, ROPE_CTX)
    orc32 = Qwen3Oracle({}, QwenConfig(dtype=torch.float32), ROPE_CTX)
    orc32.w = orc16.w
    got = model.forward(ids[:, :S].to(dev), use_cache=True, cache_position=0)
    _check(got[:, -1], orc16.forward(ids[:, :S], 0)[:, -1], orc32.forward(ids[:, :S], 0)[:, -1],
           "config 5 batch 8 prefill, last position")
    for t in range(2):
        step = ids[:, S + t:S + t + 1]
        got = model.forward(step.to(dev), use_cache=True, cache_position=S + t)
        _check(got, orc16.forward(step, S + t), orc32.forward(step, S + t),
               f"config 5 batch 8 decode step {t}")
