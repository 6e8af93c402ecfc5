"""Benchmark: Qwen3-0.6B-shape greedy decode on one MI355X.

Workload: random-init Qwen3-0.6B-architecture
decoder (28 layers, hidden 1024, 16/8 heads, head_dim 128, SwiGLU 3072,
vocab 151936, bf16, weights ~N(0, 0.02)), batch 8, prefill 2048 random token
ids, then greedy decode. A step is one decode token for all 8 sequences (one
replay of the captured decode graph); `value` = 8 * steps / time of the K
timed steps at cache positions 2048..2048+K-1.

Also printed in the same JSON line:
  roofline      the dominant decode kernel (split-KV attention, HBM-bound):
                algorithmic bytes per launch / average launch time measured
                with HIP events on the stream it runs on
  kernels       every decode/prefill kernel at its model shape, same method
  prefill       time and tok/s of the 2048 x 8 prefill
  cpu_baseline  the CPU oracle (PyTorch restatement of the reference model)
                decoding on this host's cores, bounded sample
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense bf16
METRIC = "Qwen3-0.6B-shape decode tok/s; per-kernel HBM GB/s & MFMA % of MI355X peak"
BATCH, PREFILL = 8, 2048


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def event_time_us(fn, iters: int, reps: int = 5) -> float:
    """Average GPU time per call of fn(): `iters` calls are captured into one
    HIP graph (so back-to-back kernels are timed, not Python launch
    overhead), the graph is replayed `reps` times between HIP events recorded
    on the stream the kernels run on (torch's current stream)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm-up: allocations and lazily built fused weights
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(iters):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st.record()
    for _ in range(reps):
        graph.replay()
    en.record()
    torch.cuda.synchronize()
    return st.elapsed_time(en) * 1e3 / (reps * iters)


def hbm_entry(name, us, nbytes):
    gbs = nbytes / us / 1e3
    return {"kernel": name, "us": round(us, 3), "bound": "hbm", "bytes": int(nbytes),
            "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}


def mfma_entry(name, us, flops):
    tf = flops / us / 1e6
    return {"kernel": name, "us": round(us, 3), "bound": "mfma", "flops": int(flops),
            "TFLOP/s": round(tf, 1), "frac": round(tf / MFMA_PEAK_TFLOPS, 4)}


def oproj_bytes(B, H, Hkv, D, E, L):
    """Algorithmic HBM bytes of one decode attention + o_proj launch at cache
    length L: the L-1 cached K/V rows of every (sequence, KV head), the new
    token's qkv row, its K/V rows written to the cache, the projection weight,
    the residual read and written, the attention output written."""
    return (2 * B * Hkv * (L - 1) * D * 2 + B * (H + 2 * Hkv) * D * 2 + 2 * B * Hkv * D * 2
            + E * H * D * 2 + 2 * B * E * 2 + B * H * D * 2)


def measure_kernels(model, dec, cfg, L):
    """Per-kernel timings at the decode (cache length L) and prefill shapes.
    Each launch cycles over the 28 layers' weights / caches, so the bytes come
    from HBM (2.1 GB of caches, 1.2 GB of weights >> the 256 MB MALL)."""
    from torchplusplus_amd._native import ext

    C = ext()
    B, E, H, Hkv, D, I, V = BATCH, cfg.embed_dim, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.hidden_dim, cfg.vocab_size
    dev = model.out_head.weight.device
    dt = cfg.dtype
    blocks = model.transformer_blocs
    caches = model.kv_cache_array
    nl = len(blocks)
    g = torch.Generator(device=dev).manual_seed(1)
    x1 = torch.randn(B, 1, E, generator=g, device=dev).to(dt)
    out = []
    it = {"i": 0}

    def cyc():
        it["i"] = (it["i"] + 1) % nl
        return it["i"]

    # decode attention at cache length L
    q = torch.randn(B, 1, H, D, generator=g, device=dev).to(dt)
    seq = torch.full((B,), L, dtype=torch.int32, device=dev)
    o = torch.empty_like(q)

    def attn():
        c = caches[cyc()]
        C.attn_decode(q, c.k_cache, c.v_cache, seq, 0.0, -1, o)

    us = event_time_us(attn, nl)
    out.append(hbm_entry("attn_decode_kernel (splits merged in-kernel) B8 16/8 d128 L%d" % L, us,
                         2 * B * Hkv * L * D * 2 + 2 * B * H * D * 2))

    # the decode step's attention launch: QK-norm + RoPE + K/V append of the
    # new token, attention over L keys, output projection + residual add
    qkv1 = (0.5 * torch.randn(B, 1, (H + 2 * Hkv) * D, generator=g, device=dev)).to(dt)
    reso = torch.randn(B, 1, E, generator=g, device=dev).to(dt)

    def attn_op():
        i = cyc()
        c, at = caches[i], blocks[i].attn
        C.attn_decode_oproj(qkv1, at.q_norm.weight, at.k_norm.weight, model.cos, model.sin, 1e-6,
                            c.k_cache, c.v_cache, seq, at.out_projection.weight, reso)

    attn_us = event_time_us(attn_op, nl)
    attn_bytes = oproj_bytes(B, H, Hkv, D, E, L)
    out.append(hbm_entry("attn_decode_kernel<oproj> (attention + o_proj + residual, one launch) "
                         "B8 16/8 d128 L%d, W_o [1024x2048]" % L, attn_us, attn_bytes))

    def gemv_entry(name, wget, n, k, xin, fn=None):
        def run():
            w = wget(blocks[cyc()])
            (fn or (lambda a, b: C.gemv(a, b, None, 0)))(xin, w)
        t = event_time_us(run, nl)
        out.append(hbm_entry(name, t, (n * k + B * k + B * n) * 2))

    nw = blocks[0].rms_norm1.weight
    gemv_entry("gemv qkv +rmsnorm [8x1024]x[4096x1024]^T", lambda b: b.attn.fused_qkv_weight(), 4096, E,
               x1, lambda a, b: C.gemv_fused(a, b, nw, 1e-6))
    xo = torch.randn(B, 1, H * D, generator=g, device=dev).to(dt)
    res = torch.randn(B, 1, E, generator=g, device=dev).to(dt)
    gemv_entry("gemv o_proj +residual [8x2048]x[1024x2048]^T (two-launch path, not in the step)",
               lambda b: b.attn.out_projection.weight, E, H * D, xo,
               lambda a, b: C.gemv_fused(a, b, None, 1e-6, res))
    # the decode step's FFN half: RMSNorm + gate/up SwiGLU + down + residual in
    # one launch (weights of all 28 layers in turn, residual updated in place)
    resf = torch.randn(B, 1, E, generator=g, device=dev).to(dt)

    def ffn():
        blk = blocks[cyc()]
        C.ffn_decode(resf, nw, 1e-6, blk.ffn.w_gu(), blk.ffn.linear_layer2.weight)

    t = event_time_us(ffn, nl)
    out.append(hbm_entry("ffn_decode (RMSNorm + gate/up SwiGLU + down + residual, one launch) "
                         "[8x1024], I 3072", t, (3 * I * E + 2 * B * E) * 2))
    wout = model.out_head.weight
    fw = model.final_rmsnorm.weight
    t = event_time_us(lambda: C.gemv_argmax(x1, wout, fw, 1e-6, False), 8)
    out.append(hbm_entry("gemv_argmax lm_head +rmsnorm [8x1024]x[151936x1024]^T (+partials)", t,
                         (V * E + B * E) * 2))
    # prefill shapes. QK-norm + RoPE + KV append of the prefill (the decode
    # graph does this inside the attention kernel's prologue instead)
    M = BATCH * PREFILL
    qkv = torch.randn(B, PREFILL, (H + 2 * Hkv) * D, generator=g, device=dev).to(dt)
    qo = torch.empty(B, PREFILL, H, D, dtype=dt, device=dev)
    pos = torch.zeros(B, dtype=torch.int32, device=dev)
    a0 = blocks[0].attn

    def rope():
        c = caches[cyc()]
        C.qkv_rope_cache(qkv, qo, c.k_cache, c.v_cache, a0.q_norm.weight, a0.k_norm.weight,
                         model.cos, model.sin, pos, 1e-6)

    t = event_time_us(rope, nl)
    out.append(hbm_entry("qkv_rope_cache (prefill) [8x2048 tokens, 16+8+8 heads]", t,
                         2 * M * (H + 2 * Hkv) * D * 2 + 2 * PREFILL * D * 2))
    del qkv, qo
    xp = torch.randn(M, E, generator=g, device=dev).to(dt)
    # plain prefill projections: as dispatched (hipBLASLt from one 256x256
    # tile per CU up) and on the hand-written MFMA kernel (dispatch off)
    from torchplusplus_amd._native import lib
    xo_p = torch.randn(M, H * D, generator=g, device=dev).to(dt)
    xd_p = torch.randn(M, I, generator=g, device=dev).to(dt)
    plain = (("gemm qkv [16384x1024]x[4096x1024]^T", xp, lambda b: b.attn.fused_qkv_weight(), 4096, E),
             ("gemm o_proj [16384x2048]x[1024x2048]^T", xo_p, lambda b: b.attn.out_projection.weight, E, H * D),
             ("gemm down [16384x3072]x[1024x3072]^T", xd_p, lambda b: b.ffn.linear_layer2.weight, E, I))
    for vendor, tag in ((1, "hipBLASLt (dispatched)"), (0, "MFMA kernel")):
        prev = lib().tpp_gemm_vendor(vendor)
        try:
            for name, xin, wget, n, k in plain:
                t = event_time_us(lambda: C.linear(xin, wget(blocks[cyc()]), None, 0), nl)
                out.append(mfma_entry(f"{name}, {tag}", t, 2 * M * n * k))
        finally:
            lib().tpp_gemm_vendor(prev)
    del xo_p, xd_p
    t = event_time_us(lambda: C.linear_swiglu(xp, blocks[cyc()].ffn.w_gu()), nl)
    out.append(mfma_entry("gemm swiglu [16384x1024]x[6144x1024]^T", t, 2 * M * 2 * I * E))
    qp = torch.randn(BATCH, PREFILL, H, D, generator=g, device=dev).to(dt)
    kp = torch.randn(BATCH, PREFILL, Hkv, D, generator=g, device=dev).to(dt)
    vp = torch.randn(BATCH, PREFILL, Hkv, D, generator=g, device=dev).to(dt)
    t = event_time_us(lambda: C.flash_attn_func(qp, kp, vp, True, -1, -1, 0.0), 4)
    keys = PREFILL * (PREFILL + 1) // 2
    out.append(mfma_entry("attn_prefill causal B8 S2048 16/8 d128", t, 4 * BATCH * H * D * keys))
    del xp, qp, kp, vp
    return out, attn_us, attn_bytes


def _rotating(make, n):
    """n independent argument sets (make(i)) and a call counter: a graph of n
    launches touches n distinct buffer sets (cold: > 2x the 256 MB MALL when
    n * bytes > 512 MB), or the first set n times (warm)."""
    sets = [make(i) for i in range(n)]
    it = {"i": 0}

    def nxt(cold):
        if not cold:
            return sets[0]
        it["i"] = (it["i"] + 1) % n
        return sets[it["i"]]
    return nxt


def _cold_warm(call, nxt, n):
    keep = []  # outputs stay alive, so each captured launch writes its own buffer
    cold = event_time_us(lambda: keep.append(call(*nxt(True))), n)
    keep.clear()
    warm = event_time_us(lambda: call(*nxt(False)), n)
    return cold, warm


def _cfg_entry(cfg_idx, name, bound, cold, warm, amount):
    e = (hbm_entry if bound == "hbm" else mfma_entry)(name, cold, amount)
    w = (hbm_entry if bound == "hbm" else mfma_entry)(name, warm, amount)
    e["config"] = cfg_idx
    e["us_warm"] = w["us"]
    e["frac_warm"] = w["frac"]
    return e


def _copy_ceiling(e, nbytes, sets, randn):
    """A plain device copy (torch's copy_, one launch) moving the same bytes as
    an HBM-bound entry (half read, half written), timed the same way: what
    one launch of this size reaches (launch floor + HBM round trip)."""
    n = nbytes // 4  # bf16 elements each way
    nxt = _rotating(lambda i: (randn(n, dtype=torch.bfloat16),
                               torch.empty(n, dtype=torch.bfloat16, device="cuda")), sets)
    cold, warm = _cold_warm(lambda a, b: b.copy_(a), nxt, sets)
    e["copy_us"], e["copy_us_warm"] = round(cold, 3), round(warm, 3)
    e["kernel_vs_copy"] = round(cold / e["us"], 4)
    return e


def measure_configs():
    """BASELINE.json configs[0..3] at their stated shapes, dtypes and
    distributions (seeded). HBM-bound ops rotate through >= 512 MB of
    distinct buffers for the cold figure; `us_warm` repeats one buffer set."""
    from torchplusplus_amd._native import ext
    from torchplusplus_amd.dlops.rope import compute_rope_params

    C = ext()
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    out = []

    def randn(*shape, dtype, std=1.0, mean=0.0):
        return (mean + std * torch.randn(*shape, generator=g, device=dev, dtype=torch.float32)).to(dtype)

    # RMSNorm fp16 [4096, 1024]
    M, N = 4096, 1024
    w = randn(N, dtype=torch.float16, std=0.1, mean=1.0)
    nxt = _rotating(lambda i: (randn(M, N, dtype=torch.float16),), 40)
    cold, warm = _cold_warm(lambda x: C.rmsnormFused(x, w, 1e-6), nxt, 40)
    out.append(_copy_ceiling(_cfg_entry(0, "rmsnormFused fp16 [4096x1024]", "hbm", cold, warm,
                                        2 * M * N * 2 + N * 2), 2 * M * N * 2, 40, randn))
    # LayerNorm has no config of its own; same shape
    cold, warm = _cold_warm(lambda x: C.applyLayernorm(x, w, 1e-6), nxt, 40)
    out.append(_cfg_entry(0, "applyLayernorm fp16 [4096x1024]", "hbm", cold, warm, 2 * M * N * 2 + N * 2))
    del nxt

    # RoPE on Q [1,16,2048,128], K [1,8,2048,128] bf16, theta 1e6
    S, D = 2048, 128
    cos, sin = compute_rope_params(D, 1e6, S, device=dev, out_dtype=torch.bfloat16)
    nxt = _rotating(lambda i: (randn(1, 16, S, D, dtype=torch.bfloat16),
                               randn(1, 8, S, D, dtype=torch.bfloat16)), 24)
    rope_bytes = 2 * (16 + 8) * S * D * 2 + 2 * S * D * 2
    cold, warm = _cold_warm(lambda q, k: C.qkrope_apply_cuda(q, k, cos, sin), nxt, 24)
    out.append(_copy_ceiling(_cfg_entry(1, "qkrope_apply Q[1,16,2048,128] K[1,8,2048,128] bf16", "hbm",
                                        cold, warm, rope_bytes), 2 * (16 + 8) * S * D * 2, 24, randn))

    def inplace(q, k):
        C.rope_apply_(q, cos, sin)
        C.rope_apply_(k, cos, sin)
    cold, warm = _cold_warm(inplace, nxt, 24)
    out.append(_cfg_entry(1, "rope_apply_ (in place, 2 launches) Q+K bf16", "hbm", cold, warm, rope_bytes))
    del nxt
    # Linear+SiLU bf16 [2048x1024] @ [1024x3072] + bias
    M, K, N = 2048, 1024, 3072
    nxt = _rotating(lambda i: (randn(M, K, dtype=torch.bfloat16), randn(N, K, dtype=torch.bfloat16, std=0.02),
                               randn(N, dtype=torch.bfloat16, std=0.02)), 24)
    cold, warm = _cold_warm(lambda x, W, b: C.LinearSilu(x, W, b), nxt, 24)
    out.append(_cfg_entry(1, "LinearSilu bf16 [2048x1024]x[3072x1024]^T +bias", "mfma", cold, warm,
                          2 * M * N * K))
    cold, warm = _cold_warm(lambda x, W, b: C.LinearGelu(x, W, b), nxt, 24)
    out.append(_cfg_entry(1, "LinearGelu bf16 [2048x1024]x[3072x1024]^T +bias", "mfma", cold, warm,
                          2 * M * N * K))
    del nxt

    # prefill B4 S2048 16/8 d128 causal, and window 512
    B, S, Hq, Hkv = 4, 2048, 16, 8
    q = randn(B, S, Hq, D, dtype=torch.bfloat16)
    k = randn(B, S, Hkv, D, dtype=torch.bfloat16)
    v = randn(B, S, Hkv, D, dtype=torch.bfloat16)
    t = event_time_us(lambda: C.flash_attn_func(q, k, v, True, -1, -1, 0.0), 8)
    out.append(_cfg_entry(2, "flash_attn causal B4 S2048 16/8 d128", "mfma", t, t,
                          4 * B * Hq * D * (S * (S + 1) // 2)))
    keys = sum(min(i + 1, 512) for i in range(S))
    t = event_time_us(lambda: C.flash_attn_func(q, k, v, True, 511, 0, 0.0), 8)
    out.append(_cfg_entry(2, "flash_attn causal window 512 B4 S2048 16/8 d128", "mfma", t, t,
                          4 * B * Hq * D * keys))
    del q, k, v

    # hgemv fp16 [1x1024]@[1024x3072] and [1x3072]@[3072x1024]
    for (Mo, K) in ((3072, 1024), (1024, 3072)):
        nxt = _rotating(lambda i: (randn(1, K, dtype=torch.float16),
                                   randn(Mo, K, dtype=torch.float16, std=0.02)), 96)
        cold, warm = _cold_warm(lambda x, W: C.gemv(x, W, None, 0), nxt, 96)
        hb = (Mo * K + K + Mo) * 2
        del nxt
        out.append(_copy_ceiling(_cfg_entry(3, f"hgemv fp16 [1x{K}]x[{Mo}x{K}]^T", "hbm", cold, warm,
                                            hb), hb, 96, randn))
    # decode attention B32 16/8 d128, cache 4096, bf16 ~N(0,1)
    B, L = 32, 4096
    kc = randn(B, Hkv, L, D, dtype=torch.bfloat16)
    vc = randn(B, Hkv, L, D, dtype=torch.bfloat16)
    q = randn(B, 1, Hq, D, dtype=torch.bfloat16)
    seq = torch.full((B,), L, dtype=torch.int32, device=dev)
    o = torch.empty_like(q)
    t = event_time_us(lambda: C.attn_decode(q, kc, vc, seq, 0.0, -1, o), 8)
    out.append(_cfg_entry(3, "attn_decode B32 16/8 d128 L4096", "hbm", t, t,
                          2 * B * Hkv * L * D * 2 + 2 * B * Hq * D * 2))
    del kc, vc
    return out


def cpu_config_timings() -> dict:
    """The oracle (PyTorch CPU restatement of each reference op) timed on the
    host cores for every BASELINE config entry: median of 5 calls after two
    warm-ups, same shapes and dtypes (attention on a 1-sequence sample, scaled
    to the config's batch; noted in `cpu_sample`). Returns {entry-name prefix:
    {cpu_us, cpu_cores, cpu_sample}}."""
    import oracle

    torch.set_num_threads(len(os.sched_getaffinity(0)))
    g = torch.Generator().manual_seed(0)

    def rnd(*shape, dtype, std=1.0, mean=0.0):
        return (mean + std * torch.randn(*shape, generator=g)).to(dtype)

    def med_us(fn, reps=5):
        fn()
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        ts.sort()
        return ts[len(ts) // 2] * 1e6

    x = rnd(4096, 1024, dtype=torch.float16)
    w = rnd(1024, dtype=torch.float16, std=0.1, mean=1.0)
    cos, sin = oracle.compute_rope_params(128, 1e6, 2048)
    q1, k1 = rnd(1, 16, 2048, 128, dtype=torch.bfloat16), rnd(1, 8, 2048, 128, dtype=torch.bfloat16)
    xl, wl, bl = (rnd(2048, 1024, dtype=torch.bfloat16), rnd(3072, 1024, dtype=torch.bfloat16, std=0.02),
                  rnd(3072, dtype=torch.bfloat16, std=0.02))
    qa, ka, va = (rnd(1, 2048, 16, 128, dtype=torch.bfloat16), rnd(1, 2048, 8, 128, dtype=torch.bfloat16),
                  rnd(1, 2048, 8, 128, dtype=torch.bfloat16))
    timings = {
        "rmsnormFused": (lambda: oracle.rmsnorm(x, w, 1e-6), 1, "exact config"),
        "applyLayernorm": (lambda: oracle.layernorm(x, w, 1e-6), 1, "exact config"),
        "qkrope_apply": (lambda: oracle.qkrope(q1, k1, cos, sin), 1, "exact config"),
        "rope_apply_": (lambda: oracle.qkrope(q1, k1, cos, sin), 1, "exact config (out of place)"),
        "LinearSilu": (lambda: oracle.linear_act(xl, wl, bl, "silu"), 1, "exact config"),
        "LinearGelu": (lambda: oracle.linear_act(xl, wl, bl, "gelu"), 1, "exact config"),
        "flash_attn causal B4": (lambda: oracle.attention(qa, ka, va, causal=True), 4,
                                 "batch 1 of 4, x4"),
        "flash_attn causal window": (lambda: oracle.attention(qa, ka, va, causal=True, window=(511, 0)), 4,
                                     "batch 1 of 4, x4"),
    }
    for K, N in ((1024, 3072), (3072, 1024)):
        xv, wv = rnd(1, K, dtype=torch.float16), rnd(N, K, dtype=torch.float16, std=0.02)
        timings[f"hgemv fp16 [1x{K}]"] = ((lambda xv=xv, wv=wv: oracle.gemv(xv, wv)), 1, "exact config")
    qd = rnd(1, 1, 16, 128, dtype=torch.bfloat16)
    kc, vc = rnd(1, 8, 4096, 128, dtype=torch.bfloat16), rnd(1, 8, 4096, 128, dtype=torch.bfloat16)
    sl = torch.tensor([4096], dtype=torch.int32)
    timings["attn_decode B32"] = ((lambda: oracle.decode_attention(qd, kc, vc, sl)), 32, "batch 1 of 32, x32")
    cores = len(os.sched_getaffinity(0))
    return {key: {"cpu_us": round(med_us(fn) * scale, 1), "cpu_cores": cores,
                  "cpu_sample": "oracle on the host CPU, " + sample}
            for key, (fn, scale, sample) in timings.items()}


def apply_cpu_configs(configs, table: dict):
    """Attach the CPU timings of cpu_config_timings() to the config entries."""
    for e in configs:
        for key, v in table.items():
            if e["kernel"].startswith(key):
                e.update(v)
                break


def cpu_model_name() -> str:
    """The host CPU's model name (/proc/cpuinfo, as lscpu reports it)."""
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median(ts):
    ts = sorted(ts)
    return ts[len(ts) // 2]


def cpu_baseline(model, cfg, steps: int = 5, warmup: int = 2, full: bool = False, reps: int = 5):
    """The oracle's eager PyTorch decode (fp32 math, bf16 rounding at op
    boundaries) on this host's cores, batch 8.

    Default (bounded sample, ~10-30 s of CPU work so the bench stays within
    minutes): `warmup` decode steps, then `steps` timed decode steps against a
    2048-position cache filled with random K/V (a decode step costs the same
    whatever the cache holds); value = batch / median step time.
    full=True: the complete CPU plan -- per rep a 2048-token batch-8 prefill
    followed by 32 greedy decode steps, `warmup` + `reps` reps, medians of
    the per-rep prefill time and decode step time (several minutes per rep)."""
    from oracle.qwen3 import Qwen3Oracle

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(2)
    base = {"unit": "tok/s", "cores": cores, "kind": "port", "cpu_model": cpu_model_name(),
            "timer": "time.perf_counter"}
    if not full:
        orc = Qwen3Oracle(model.state_dict(), cfg, PREFILL + warmup + steps + 2)
        orc.seed_cache(BATCH, PREFILL, g)
        ids = torch.randint(0, cfg.vocab_size, (BATCH, 1), generator=g)
        ts = []
        for s in range(warmup + steps):
            t0 = time.perf_counter()
            logits = orc.forward(ids, PREFILL + s)
            ids = logits[:, -1].argmax(-1, keepdim=True)
            if s >= warmup:
                ts.append(time.perf_counter() - t0)
        step = _median(ts)
        return {**base, "value": round(BATCH / step, 3), "ms_per_step": round(step * 1e3, 1),
                "sample": f"bounded sample: {warmup} warm-up + {steps} timed greedy decode steps "
                          f"(median), batch {BATCH}, cache {PREFILL} positions of random K/V; "
                          f"oracle/qwen3.py on the host CPU, random-init weights of the model's "
                          f"shape, glibc malloc keeping freed blocks (`malloc`). The full plan "
                          f"(2048-token prefill + 32 steps, median of 5) runs with --cpu-full"}
    n_dec = 32
    pre, dec = [], []
    for r in range(warmup + reps):
        orc = Qwen3Oracle(model.state_dict(), cfg, PREFILL + n_dec + 2)
        ids = torch.randint(0, cfg.vocab_size, (BATCH, PREFILL), generator=g)
        t0 = time.perf_counter()
        logits = orc.forward(ids, 0)
        t1 = time.perf_counter()
        log(f"[bench] cpu full rep {r}: prefill {t1 - t0:.1f} s")
        nxt = logits[:, -1].argmax(-1, keepdim=True)
        for s in range(n_dec):
            logits = orc.forward(nxt, PREFILL + s)
            nxt = logits[:, -1].argmax(-1, keepdim=True)
            if s % 8 == 7:
                log(f"[bench] cpu full rep {r}: {s + 1} decode steps")
        t2 = time.perf_counter()
        log(f"[bench] cpu full rep {r}: prefill {t1 - t0:.1f} s, {n_dec} steps {t2 - t1:.1f} s")
        if r >= warmup:
            pre.append(t1 - t0)
            dec.append((t2 - t1) / n_dec)
    step = _median(dec)
    return {**base, "value": round(BATCH / step, 3), "ms_per_step": round(step * 1e3, 1),
            "prefill_s": round(_median(pre), 2),
            "prefill_tok_per_s": round(BATCH * PREFILL / _median(pre), 1),
            "sample": f"full plan: {warmup} warm-up + {reps} reps (medians) of a {PREFILL}-token "
                      f"batch-{BATCH} prefill then {n_dec} greedy decode steps; oracle/qwen3.py, "
                      f"glibc malloc keeping freed blocks (`malloc`)"}


TRAFFIC_GROUPS = ["attn_oproj", "attn", "gemv_qkv", "gemv_o", "gemv_gu", "gemv_down", "ffn", "lm_head", "rmsnorm",
                  "layernorm", "rope", "hgemv_3072", "hgemv_1024", "copy"]


def traffic_probe(group: str, L: int, launches: int = 16):
    """Counter run (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE) of one
    HBM-bound kernel, `launches` times over distinct buffer sets (so no launch
    finds its bytes in another launch's L2 lines), followed by three plain
    512 MiB device copies whose counter readings calibrate KiB per dispatch
    against known bytes. Groups: the decode attention at the decode-bench
    shape (B 8, 16/8 heads, d 128, cache length L), the four decode GEMVs, the
    fused decode FFN and the lm_head at the model shapes, and BASELINE configs 0/1/3 (RMSNorm,
    LayerNorm, Q+K RoPE, both hgemv shapes); `copy` is the calibration alone.
    Prints the algorithmic bytes per launch."""
    from torchplusplus_amd._native import ext

    C = ext()
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(3)
    B, H, Hkv, D, E, I, V = BATCH, 16, 8, 128, 1024, 3072, 151936

    def rn(*shape, dtype=torch.bfloat16, std=1.0):
        return (std * torch.randn(*shape, generator=g, device=dev)).to(dtype)

    def rot(n, make):
        sets = [make() for _ in range(n)]
        return lambda i: sets[i % n]

    launch, nbytes = None, 0
    if group == "attn_oproj":
        get = rot(8, lambda: (rn(B, Hkv, L, D), rn(B, Hkv, L, D), rn(E, H * D, std=0.02)))
        qkv, seq = rn(B, 1, (H + 2 * Hkv) * D, std=0.5), torch.full((B,), L, dtype=torch.int32, device=dev)
        res, nw = rn(B, 1, E), torch.ones(D, dtype=torch.bfloat16, device=dev)
        from torchplusplus_amd.dlops.rope import compute_rope_params
        cos, sin = compute_rope_params(D, 1e6, L + 1, device=dev)

        def launch(i):
            kc, vc, wo = get(i)
            return C.attn_decode_oproj(qkv, nw, nw, cos, sin, 1e-6, kc, vc, seq, wo, res)
        nbytes = oproj_bytes(B, H, Hkv, D, E, L)
    elif group == "attn":
        get = rot(8, lambda: (rn(B, Hkv, L, D), rn(B, Hkv, L, D)))
        q, seq = rn(B, 1, H, D), torch.full((B,), L, dtype=torch.int32, device=dev)
        o = torch.empty_like(q)
        launch = lambda i: C.attn_decode(q, *get(i), seq, 0.0, -1, o)  # noqa: E731
        nbytes = 2 * B * Hkv * L * D * 2 + 2 * B * H * D * 2
    elif group.startswith("gemv_"):
        nw = torch.ones(E, dtype=torch.bfloat16, device=dev)
        res = rn(B, 1, E)
        n, k, x, call = {
            "gemv_qkv": (4096, E, rn(B, 1, E), lambda x, w: C.gemv_fused(x, w, nw, 1e-6)),
            "gemv_o": (E, H * D, rn(B, 1, H * D), lambda x, w: C.gemv_fused(x, w, None, 1e-6, res)),
            "gemv_gu": (2 * I, E, rn(B, 1, E), lambda x, w: C.gemv_swiglu(x, w, nw, 1e-6)),
            "gemv_down": (E, I, rn(B, 1, I), lambda x, w: C.gemv_fused(x, w, None, 1e-6, res)),
        }[group]
        get = rot(16, lambda: rn(n, k, std=0.02))
        launch = lambda i: call(x, get(i))  # noqa: E731
        nbytes = (n * k + B * k + B * n) * 2
    elif group == "ffn":
        nw = torch.ones(E, dtype=torch.bfloat16, device=dev)
        res = rn(B, 1, E)
        get = rot(16, lambda: (rn(2 * I, E, std=0.02), rn(E, I, std=0.02)))
        launch = lambda i: C.ffn_decode(res, nw, 1e-6, *get(i))  # noqa: E731
        nbytes = (3 * I * E + 2 * B * E) * 2
    elif group == "lm_head":
        get = rot(2, lambda: rn(V, E, std=0.02))
        x, nw = rn(B, 1, E), torch.ones(E, dtype=torch.bfloat16, device=dev)
        launch = lambda i: C.gemv_argmax(x, get(i), nw, 1e-6, False)  # noqa: E731
        nbytes = (V * E + B * E) * 2
    elif group in ("rmsnorm", "layernorm"):
        w = rn(E, dtype=torch.float16, std=0.1) + 1
        get = rot(16, lambda: rn(4096, E, dtype=torch.float16))
        fn = C.rmsnormFused if group == "rmsnorm" else C.applyLayernorm
        launch = lambda i: fn(get(i), w, 1e-6)  # noqa: E731
        nbytes = 2 * 4096 * E * 2 + E * 2
    elif group == "rope":
        from torchplusplus_amd.dlops.rope import compute_rope_params
        cos, sin = compute_rope_params(D, 1e6, 2048, device=dev, out_dtype=torch.bfloat16)
        get = rot(12, lambda: (rn(1, 16, 2048, D), rn(1, 8, 2048, D)))
        launch = lambda i: C.qkrope_apply_cuda(*get(i), cos, sin)  # noqa: E731
        nbytes = 2 * 24 * 2048 * D * 2 + 2 * 2048 * D * 2
    elif group.startswith("hgemv_"):
        n = int(group.split("_")[1])
        k = 4096 - n
        get = rot(48, lambda: (rn(1, k, dtype=torch.float16), rn(n, k, dtype=torch.float16, std=0.02)))
        launch = lambda i: C.gemv(*get(i), None, 0)  # noqa: E731
        nbytes = (n * k + k + n) * 2
    elif group != "copy":
        raise SystemExit(f"unknown traffic group {group}")
    src = torch.randn(256 << 20, generator=g, device=dev).bfloat16()  # 512 MiB
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    keep = []
    if launch is not None:
        for i in range(launches):
            keep.append(launch(i))
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"probe": group, "B": B, "L": L, "launches": launches if launch else 0,
                      "algorithmic_bytes": nbytes, "copy_bytes_each_way": src.numel() * 2}),
          flush=True)


def measured_traffic(cache_len: int):
    """HBM bytes per launch of the roofline kernel from a committed counter
    summary (two rocprofv3 --pmc passes calibrated on a copy of known size)
    measured at this cache length; else None."""
    import glob
    import re
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "attn_decode_oproj_b8_l*_traffic.md"))):
        txt = open(path).read()
        b = re.search(r"^traffic_bytes_per_launch: (\d+)$", txt, re.M)
        L = re.search(r"^traffic_cache_len: (\d+)$", txt, re.M)
        if b and L and int(L.group(1)) == cache_len:
            return int(b.group(1))
    return None


def kernel_probe(name: str, reps: int = 5):
    """Counter runs (rocprofv3 --pmc ...) of one BASELINE config kernel:
    `gemm` = Linear+SiLU [2048x1024]x[3072x1024]^T + bias and the prefill
    qkv GEMM [16384x1024]x[4096x1024]^T, as dispatched (hipBLASLt) and on
    the hand-written persistent kernel; `attn_prefill` = causal flash
    attention B4 S2048 16/8 d128. `reps` launches each, no timing."""
    from torchplusplus_amd._native import ext, lib

    C = ext()
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(5)
    if name == "gemm":
        x = torch.randn(2048, 1024, generator=g, device=dev).bfloat16()
        w = (0.02 * torch.randn(3072, 1024, generator=g, device=dev)).bfloat16()
        b = (0.02 * torch.randn(3072, generator=g, device=dev)).bfloat16()
        xp = torch.randn(16384, 1024, generator=g, device=dev).bfloat16()
        wp = (0.02 * torch.randn(4096, 1024, generator=g, device=dev)).bfloat16()
        for _ in range(reps):
            C.LinearSilu(x, w, b)
        for vendor in (1, 0):
            prev = lib().tpp_gemm_vendor(vendor)
            try:
                for _ in range(reps):
                    C.linear(xp, wp, None, 0)
            finally:
                lib().tpp_gemm_vendor(prev)
    elif name in ("attn_prefill", "attn_prefill_window"):
        q = torch.randn(4, 2048, 16, 128, generator=g, device=dev).bfloat16()
        k = torch.randn(4, 2048, 8, 128, generator=g, device=dev).bfloat16()
        v = torch.randn(4, 2048, 8, 128, generator=g, device=dev).bfloat16()
        left = 511 if name == "attn_prefill_window" else -1
        for _ in range(reps):
            C.flash_attn_func(q, k, v, True, left, -1, 0.0)
    else:
        raise SystemExit(f"unknown probe {name}")
    torch.cuda.synchronize()
    print(json.dumps({"probe": name, "reps": reps}), flush=True)


# glibc malloc settings of the CPU-baseline process: freed blocks stay in the
# process instead of going back to the OS, so the oracle's per-step
# temporaries (tens of MB per layer: the fp32 copies of the K/V cache, the
# appended cache) are not page-faulted afresh on every decode step. Measured
# on the GPU box's 16 cores: 0.63-0.76 s per decode step against 1.45-1.64 s
# with the defaults, same code.
CPU_MALLOC_TUNABLES = "glibc.malloc.mmap_threshold=4294967295:glibc.malloc.trim_threshold=4294967295"


def _under_profiler() -> bool:
    """rocprofv3 runs the program with its tool library preloaded."""
    return "rocprof" in os.environ.get("LD_PRELOAD", "") or any(k.startswith("ROCPROF") for k in os.environ)


def start_cpu_child(args):
    """The CPU baseline runs in a child process with the malloc settings
    above (they are read at process start). It is started before this
    process touches the GPU and waits on its stdin, so it takes no CPU time
    while the GPU is measured; finish_cpu_child() lets it run."""
    env = dict(os.environ)
    env["GLIBC_TUNABLES"] = ":".join(t for t in (env.get("GLIBC_TUNABLES"), CPU_MALLOC_TUNABLES) if t)
    cmd = [sys.executable, os.path.abspath(__file__), "--cpu-baseline-only",
           "--cpu-steps", str(args.cpu_steps), "--cpu-reps", str(args.cpu_reps)]
    if args.cpu_full:
        cmd.append("--cpu-full")
    return subprocess.Popen(cmd, env=env, stdin=subprocess.PIPE, stdout=subprocess.PIPE, text=True)


def finish_cpu_child(child, timeout_s: float):
    """Signal the child, wait for its JSON line (its progress goes to
    stderr). A failed or overrunning child costs the line its CPU figures
    only: None, with the reason logged."""
    try:
        out, _ = child.communicate("go\n", timeout=timeout_s)
    except subprocess.TimeoutExpired:
        child.kill()
        child.communicate()
        log(f"[bench] cpu baseline: no result within {timeout_s:.0f} s, left out")
        return None
    lines = [ln for ln in out.splitlines() if ln.startswith("{")]
    if child.returncode != 0 or not lines:
        log(f"[bench] cpu baseline process failed (exit {child.returncode}), left out")
        return None
    return json.loads(lines[-1])


def cpu_child_main(args):
    """--cpu-baseline-only: wait for the parent's go, then time the oracle on
    a CPU model of the benchmark's shape (random init like the GPU model) and
    every BASELINE config op; print one JSON line."""
    if sys.stdin.readline().strip() != "go":
        return  # the parent ended first
    from torchplusplus_amd.fastqwen3 import FastQwen3, QwenConfig

    cfg = QwenConfig(dtype=torch.bfloat16)
    log("[bench] cpu baseline: building the CPU model")
    with torch.inference_mode():
        model = FastQwen3(cfg, device="cpu").eval()
        model.init_weights(std=0.02, generator=torch.Generator().manual_seed(0))
        cpu = cpu_baseline(model, cfg, args.cpu_steps, full=args.cpu_full, reps=args.cpu_reps)
        del model
        table = cpu_config_timings()
    cpu["malloc"] = os.environ.get("GLIBC_TUNABLES", "")
    print(json.dumps({"cpu_baseline": cpu, "cpu_configs": table}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-steps", type=int, default=5)
    ap.add_argument("--cpu-full", action="store_true",
                    help="CPU baseline as full 2048-token prefill + 32 decode steps, 2 warm-ups, "
                         "median of 5 reps (several minutes per rep)")
    ap.add_argument("--cpu-reps", type=int, default=5)
    ap.add_argument("--cpu-baseline-only", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--traffic-probe", nargs="?", const="attn", choices=TRAFFIC_GROUPS,
                    help="only launch one HBM-bound kernel group + a calibration copy (for "
                         "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE); attn at cache length "
                         "2048 + steps // 2")
    ap.add_argument("--kernel-probe", choices=["gemm", "attn_prefill", "attn_prefill_window"],
                    help="only launch one config's kernels a few times (for rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.cpu_baseline_only:
        cpu_child_main(args)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only; across GPUs the decode path would "
              "shard by KV head (attention) and by columns/rows (projections), which is not "
              "built here. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    if args.kernel_probe:
        torch.cuda.set_device(0)
        with torch.inference_mode():
            kernel_probe(args.kernel_probe)
        return
    if args.traffic_probe:
        torch.cuda.set_device(0)
        with torch.inference_mode():
            traffic_probe(args.traffic_probe, PREFILL + args.steps // 2)
        return

    # the CPU-baseline process is started first, before this one loads the HIP
    # library; not under a profiler, whose preloaded library may have set up
    # the GPU in this process already
    child = None
    if not args.no_cpu_baseline:
        if _under_profiler():
            log("[bench] profiler detected: no CPU baseline in this run")
        else:
            child = start_cpu_child(args)
    from torchplusplus_amd.fastqwen3 import FastQwen3, GreedyDecoder, QwenConfig

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = QwenConfig(dtype=torch.bfloat16)
    K, W = args.steps, args.warmup
    lmax = PREFILL + max(K, W) + 1
    log(f"[bench] building model (28 layers, bf16), kv cache {lmax} positions")
    with torch.inference_mode():
        model = FastQwen3(cfg, device=dev, rope_context=lmax + 1).eval()
        model.init_weights(std=0.02, generator=torch.Generator(device=dev).manual_seed(0))
        ids = torch.randint(0, cfg.vocab_size, (BATCH, PREFILL),
                            generator=torch.Generator().manual_seed(0)).to(dev)
        model.setup_kv_cache(lmax, BATCH)

        # prefill (timed separately; warm once)
        model.reset_kv_cache()
        model.forward_impl(ids, model.kv_cache_array, 0, last_only=True)
        torch.cuda.synchronize()
        model.reset_kv_cache()  # zeroes the caches, as the reference's reset does
        torch.cuda.synchronize()  # ... outside the timed prefill
        t0 = time.perf_counter()
        logits = model.forward_impl(ids, model.kv_cache_array, 0, last_only=True)
        torch.cuda.synchronize()
        prefill_s = time.perf_counter() - t0
        log(f"[bench] prefill {prefill_s * 1e3:.2f} ms")
        first = torch.argmax(logits[:, -1], dim=-1)

        dec = GreedyDecoder(model, BATCH)
        dec.prepare(first, PREFILL)
        dec.capture()
        for _ in range(W):
            dec.replay()
        torch.cuda.synchronize()
        dec.prepare(first, PREFILL)  # timed steps decode positions 2048..2048+K-1
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(K):
            dec.replay()
        torch.cuda.synchronize()
        decode_s = time.perf_counter() - t0
        log(f"[bench] decode {K} steps {decode_s * 1e3:.2f} ms")
        tok_s = BATCH * K / decode_s
        # the one-launch decode kernels flag a bounded wait that gave up (their
        # output is then wrong): such a run measured nothing valid
        model.check_device_errors()

        L = PREFILL + K // 2  # mean cache length over the timed steps
        kernels, attn_us, attn_bytes = measure_kernels(model, dec, cfg, L)
        model.check_device_errors()
        log("[bench] kernel table done")
        configs = measure_configs()
        log("[bench] config table done")

    cpu = None
    if child is not None:
        log("[bench] cpu baseline ...")
        res = finish_cpu_child(child, 3600.0 if args.cpu_full else 900.0)
        if res is not None:
            cpu = res["cpu_baseline"]
            apply_cpu_configs(configs, res["cpu_configs"])
            log("[bench] cpu baseline and config timings done")

    achieved = attn_bytes / attn_us / 1e3
    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(decode_s * 1e3 / K, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init weights ~N(0,0.02), random token ids",
        "config": {"workload": "Qwen3-0.6B-shape greedy decode (28 layers, hidden 1024, 16/8 heads, "
                               "head_dim 128, SwiGLU 3072, vocab 151936), batch 8, prefill 2048",
                   "global_batch": BATCH, "prefill_len": PREFILL, "decode_steps": K,
                   "parallelism": "single GPU"},
        "roofline": {"kernel": "attn_decode_kernel<oproj> (decode attention + o_proj + residual)",
                     "bound": "hbm",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(L),
                     "bytes_per_launch": attn_bytes, "avg_launch_us": round(attn_us, 3),
                     "cache_len": L},
        "prefill": {"ms": round(prefill_s * 1e3, 3), "tok_per_s": round(BATCH * PREFILL / prefill_s, 1)},
        "kernels": kernels,
        "configs": configs,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
