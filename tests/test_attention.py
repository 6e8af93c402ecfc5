"""GPU parity: flash-attention prefill (GQA/MQA/MHA, causal, window) and
split-KV decode vs the CPU oracle (fp32 eager attention)."""
import pytest
import torch

import oracle
from tests.conftest import close
from torchplusplus_amd.attention import decode_attention, flash_attn_func

pytestmark = pytest.mark.gpu


def _qkv(b, sq, sk, hq, hkv, d, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, sq, hq, d, generator=g).to(dtype)
    k = torch.randn(b, sk, hkv, d, generator=g).to(dtype)
    v = torch.randn(b, sk, hkv, d, generator=g).to(dtype)
    return q, k, v


@pytest.mark.parametrize("window", [(-1, -1), (511, 0)])
def test_prefill_baseline_config(dev, window):
    """B4 S2048 16/8 heads D128 causal (+ window 512).
    Every output row is checked: the oracle runs per (batch, KV head) pair
    (its 2 query heads), all 32 pairs."""
    q, k, v = _qkv(4, 2048, 2048, 16, 8, 128, torch.bfloat16)
    o = flash_attn_func(q.to(dev), k.to(dev), v.to(dev), causal=True, window_size=window).cpu()
    for b in range(4):
        for hk in range(8):
            e = oracle.attention(q[b:b + 1, :, 2 * hk:2 * hk + 2], k[b:b + 1, :, hk:hk + 1],
                                 v[b:b + 1, :, hk:hk + 1], causal=True, window=window)
            close(o[b:b + 1, :, 2 * hk:2 * hk + 2], e,
                  what=f"prefill window={window} batch {b} kv head {hk}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("b,sq,sk,hq,hkv,d,causal,window", [
    (2, 200, 200, 4, 2, 128, True, (-1, -1)),    # ragged S (not a tile multiple)
    (1, 256, 256, 8, 1, 128, True, (-1, -1)),    # MQA (4 heads per block)
    (2, 130, 130, 3, 3, 64, False, (-1, -1)),    # MHA, D=64, non-causal
    (1, 5, 300, 4, 2, 128, True, (-1, -1)),      # Sq < Sk: bottom-right causal
    (1, 97, 97, 4, 2, 128, True, (16, 0)),       # small sliding window
    (1, 64, 70, 2, 1, 64, False, (10, 3)),       # two-sided window
    (1, 40, 20, 2, 2, 128, True, (-1, -1)),      # Sq > Sk: early rows see nothing -> 0
    (2, 33, 33, 6, 2, 128, True, (-1, -1)),      # G = 3: one head per block
    (2, 300, 300, 8, 4, 128, True, (100, 0)),    # 8 (batch, head group) pairs: XCD-grouped order
    (1, 200, 260, 16, 8, 64, True, (-1, -1)),    # same with D=64, Sq < Sk, ragged last tile
])
def test_prefill_shapes(dev, dtype, b, sq, sk, hq, hkv, d, causal, window):
    q, k, v = _qkv(b, sq, sk, hq, hkv, d, dtype, seed=1)
    o = flash_attn_func(q.to(dev), k.to(dev), v.to(dev), causal=causal, window_size=window)
    close(o, oracle.attention(q, k, v, causal=causal, window=window), what="prefill")


@pytest.mark.parametrize("b,sq,sk,hq,hkv,d,window", [
    (8, 1500, 1530, 8, 4, 64, (-1, -1)),   # 384 items, pairs split over the XCDs, Sq < Sk
    (8, 1500, 1530, 8, 4, 64, (200, 0)),   # same with a window (items of unequal length)
    (5, 1100, 1100, 12, 4, 64, (-1, -1)),  # 300 items, 60 pairs: round-robin items, G = 3
    (5, 1100, 1100, 12, 4, 64, (300, 0)),
    (4, 2048, 600, 16, 8, 64, (-1, -1)),   # Sq > Sk: items with no visible key between others
])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_persistent_items(dev, dtype, b, sq, sk, hq, hkv, d, window):
    """More work items (query tile x batch x head group) than CUs: each
    workgroup runs several, the next item's q rows and first K / V tiles
    requested during the previous item's epilogue."""
    q, k, v = _qkv(b, sq, sk, hq, hkv, d, dtype, seed=6)
    o = flash_attn_func(q.to(dev), k.to(dev), v.to(dev), causal=True, window_size=window)
    close(o, oracle.attention(q, k, v, causal=True, window=window), what=f"persistent window={window}")


@pytest.mark.parametrize("d", [32, 96])
def test_prefill_generic_head_dims(dev, d):
    q, k, v = _qkv(1, 37, 37, 4, 2, d, torch.bfloat16, seed=2)
    o = flash_attn_func(q.to(dev), k.to(dev), v.to(dev), causal=True)
    close(o, oracle.attention(q, k, v, causal=True), what=f"generic d={d}")


def test_prefill_strided_views_and_scale(dev):
    """[B, H, S, D] tensors transposed to [B, S, H, D] views (gqa.py:123-125)
    run without copies; an explicit softmax_scale is honoured."""
    g = torch.Generator().manual_seed(3)
    qh = torch.randn(2, 4, 100, 128, generator=g).bfloat16()
    kh = torch.randn(2, 2, 100, 128, generator=g).bfloat16()
    vh = torch.randn(2, 2, 100, 128, generator=g).bfloat16()
    o = flash_attn_func(qh.to(dev).transpose(1, 2), kh.to(dev).transpose(1, 2),
                        vh.to(dev).transpose(1, 2), causal=True, softmax_scale=0.05)
    e = oracle.attention(qh.transpose(1, 2), kh.transpose(1, 2), vh.transpose(1, 2), causal=True, scale=0.05)
    close(o, e, what="strided")


def test_prefill_uniform_v_special_case(dev):
    q, k, _ = _qkv(1, 128, 128, 2, 1, 128, torch.bfloat16, seed=4)
    row = torch.randn(128, generator=torch.Generator().manual_seed(5)).bfloat16()
    v = row.expand(1, 128, 1, 128).contiguous()
    o = flash_attn_func(q.to(dev), k.to(dev), v.to(dev), causal=True)
    close(o, row.expand(1, 128, 2, 128), atol=1e-2, rtol=0, what="uniform V")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_baseline_config(dev, dtype):
    """B32, 16/8 heads, D128, cache length 4096; all 32
    sequences against the oracle."""
    g = torch.Generator().manual_seed(6)
    B, Hq, Hkv, D, L = 32, 16, 8, 128, 4096
    q = torch.randn(B, 1, Hq, D, generator=g).to(dtype)
    kc = torch.randn(B, Hkv, L, D, generator=g).to(dtype)
    vc = torch.randn(B, Hkv, L, D, generator=g).to(dtype)
    lens = torch.full((B,), L, dtype=torch.int32)
    o = decode_attention(q.to(dev), kc.to(dev), vc.to(dev), lens.to(dev))
    e = oracle.decode_attention(q, kc, vc, lens.tolist())
    close(o, e, what="decode")


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (8, 1, 128), (4, 4, 64), (6, 2, 128)])
def test_decode_ragged_lengths(dev, hq, hkv, d):
    g = torch.Generator().manual_seed(7)
    B, Lmax = 5, 700
    q = torch.randn(B, 1, hq, d, generator=g).bfloat16()
    kc = torch.randn(B, hkv, Lmax, d, generator=g).bfloat16()
    vc = torch.randn(B, hkv, Lmax, d, generator=g).bfloat16()
    lens = torch.tensor([1, 64, 65, 333, 700], dtype=torch.int32)
    o = decode_attention(q.to(dev), kc.to(dev), vc.to(dev), lens.to(dev))
    close(o, oracle.decode_attention(q, kc, vc, lens.tolist()), what="ragged decode")


def test_decode_shared_workspace_across_shapes(dev):
    """Decode calls of different shapes share one workspace (its arrival
    counters must be back at zero after every call, and no call's partials may
    land on them, whether it merges in-kernel (pairs a multiple of 8) or with
    the merge kernel (5 x 4 pairs)): alternate four shapes twice, each
    against the oracle."""
    g = torch.Generator().manual_seed(11)
    cases = []
    for B, hq, hkv, d, Lmax in [(4, 16, 8, 128, 600), (5, 8, 4, 128, 300), (8, 16, 8, 64, 200),
                                (2, 8, 4, 128, 900)]:
        q = torch.randn(B, 1, hq, d, generator=g).bfloat16()
        kc = torch.randn(B, hkv, Lmax, d, generator=g).bfloat16()
        vc = torch.randn(B, hkv, Lmax, d, generator=g).bfloat16()
        lens = torch.randint(1, Lmax + 1, (B,), generator=g, dtype=torch.int32)
        cases.append((q, kc, vc, lens, oracle.decode_attention(q, kc, vc, lens.tolist())))
    dcases = [(q.to(dev), kc.to(dev), vc.to(dev), lens.to(dev), e) for q, kc, vc, lens, e in cases]
    for rep in range(2):
        for i, (q, kc, vc, lens, e) in enumerate(dcases):
            close(decode_attention(q, kc, vc, lens), e, what=f"decode shape {i} pass {rep}")


def test_decode_shared_workspace_across_streams(dev):
    """Decode calls on two streams share the binding's per-device workspace;
    each call waits for the stream that used it last, so back-to-back calls
    on alternating streams stay correct."""
    g = torch.Generator().manual_seed(12)
    cases = []
    for B, Lmax in [(8, 640), (4, 900)]:
        q = torch.randn(B, 1, 16, 128, generator=g).bfloat16()
        kc = torch.randn(B, 8, Lmax, 128, generator=g).bfloat16()
        vc = torch.randn(B, 8, Lmax, 128, generator=g).bfloat16()
        lens = torch.randint(Lmax // 2, Lmax + 1, (B,), generator=g, dtype=torch.int32)
        cases.append(((q.to(dev), kc.to(dev), vc.to(dev), lens.to(dev)),
                      oracle.decode_attention(q, kc, vc, lens.tolist())))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    outs = []
    for rep in range(3):
        for i, (args, _) in enumerate(cases):
            with torch.cuda.stream(streams[(rep + i) % 2]):
                outs.append((i, rep, decode_attention(*args)))
    torch.cuda.synchronize()
    for i, rep, o in outs:
        close(o, cases[i][1], what=f"stream-alternating decode {i} pass {rep}")


def test_decode_window_and_matches_prefill_path(dev):
    g = torch.Generator().manual_seed(8)
    B, Hq, Hkv, D, L = 3, 4, 2, 128, 300
    q = torch.randn(B, 1, Hq, D, generator=g).bfloat16()
    kc = torch.randn(B, Hkv, L, D, generator=g).bfloat16()
    vc = torch.randn(B, Hkv, L, D, generator=g).bfloat16()
    lens = torch.tensor([300, 150, 7], dtype=torch.int32)
    o = decode_attention(q.to(dev), kc.to(dev), vc.to(dev), lens.to(dev), window_left=63)
    close(o, oracle.decode_attention(q, kc, vc, lens.tolist(), window_left=63), what="windowed decode")
    # the prefill kernel on the same prefix (Sq = 1) agrees with the decode kernel
    p = flash_attn_func(q[:1].to(dev), kc[:1, :, :300].transpose(1, 2).to(dev),
                        vc[:1, :, :300].transpose(1, 2).to(dev), causal=True)
    d0 = decode_attention(q[:1].to(dev), kc[:1].to(dev), vc[:1].to(dev))
    close(p, d0, atol=1e-2, rtol=1e-2, what="decode vs prefill kernel")


@pytest.mark.parametrize("hq,hkv,norm", [(16, 8, True), (8, 1, True), (4, 4, False)])
def test_decode_fused_prologue_matches_unfused(dev, hq, hkv, norm):
    """attn_decode_fused == qkv_rope_cache + attn_decode: same caches (bit-exact)
    and the same attention output, for ragged positions."""
    from torchplusplus_amd._native import ext

    C = ext()
    g = torch.Generator().manual_seed(9)
    B, D, Lmax = 4, 128, 600
    qkv = torch.randn(B, 1, (hq + 2 * hkv) * D, generator=g).bfloat16().to(dev)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(dev) if norm else None
    kw = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(dev) if norm else None
    cos, sin = oracle.compute_rope_params(D, 1e6, 1024)
    cos, sin = cos.to(dev), sin.to(dev)
    kc = torch.randn(B, hkv, Lmax, D, generator=g).bfloat16().to(dev)
    vc = torch.randn(B, hkv, Lmax, D, generator=g).bfloat16().to(dev)
    pos = torch.tensor([0, 5, 299, 599], dtype=torch.int32).to(dev)
    kc2, vc2 = kc.clone(), vc.clone()
    q = torch.empty(B, 1, hq, D, dtype=torch.bfloat16, device=dev)
    C.qkv_rope_cache(qkv, q, kc2, vc2, qw, kw, cos, sin, pos, 1e-6)
    ref = C.attn_decode(q, kc2, vc2, pos + 1, 0.0, -1, None)
    got = C.attn_decode_fused(qkv, qw, kw, cos, sin, 1e-6, kc, vc, pos + 1)
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2), "cache append differs"
    close(got, ref, atol=1e-2, rtol=1e-2, what="fused decode")
    e, k_ref, v_ref = _fused_decode_oracle(qkv.cpu(), hq, hkv, qw, kw, cos.cpu(), sin.cpu(),
                                           kc2.cpu(), vc2.cpu(), pos.cpu())
    close(kc.cpu(), k_ref, what="fused decode: appended K vs oracle")
    assert torch.equal(vc.cpu(), v_ref), "fused decode: appended V differs from the projection"
    close(got, e, what="fused decode vs oracle")


def _fused_decode_oracle(qkv, hq, hkv, qw, kw, cos, sin, k_before, v_before, pos):
    """Independent of the HIP prologue: q and the appended K/V from the oracle
    (QK-RMSNorm over D, RoPE at position pos[b], V as projected;
    torchpp/attention/gqa.py:90-116, kvcache.py:50-108), then decode attention
    over pos[b] + 1 keys. Returns (output, K cache, V cache) on the CPU."""
    B, D = k_before.shape[0], k_before.shape[-1]
    x = qkv.view(B, hq + 2 * hkv, D)
    qh, kh, vh = x[:, :hq], x[:, hq:hq + hkv], x[:, hq + hkv:]
    if qw is not None:
        qh, kh = oracle.rmsnorm(qh, qw.cpu(), 1e-6), oracle.rmsnorm(kh, kw.cpu(), 1e-6)
    pl = pos.long()
    cr, sr = cos[pl][:, None], sin[pl][:, None]  # [B, 1, D]
    qh, kh = oracle.rope(qh[:, :, None], cr[:, :, None], sr[:, :, None])[:, :, 0], \
        oracle.rope(kh[:, :, None], cr[:, :, None], sr[:, :, None])[:, :, 0]
    k_ref, v_ref = k_before.clone(), v_before.clone()
    for b in range(B):
        k_ref[b, :, pl[b]] = kh[b]
        v_ref[b, :, pl[b]] = vh[b]
    return oracle.decode_attention(qh[:, None], k_ref, v_ref, (pl + 1).tolist()), k_ref, v_ref


@pytest.mark.parametrize("lens", [[2049] * 8, [2068] * 8, [2068, 2049, 2060, 1921, 1920, 641, 640, 1]],
                         ids=["L2049", "L2068", "ragged"])
def test_decode_fused_model_shape_split_merge(dev, lens):
    """The roofline kernel at its own shape: the decode step of the benchmark
    (batch 8, 16/8 heads, D 128, a 2069-row cache, cache lengths 2049..2068
    over the driver's 20 steps), where each (batch, KV head) pair's keys are
    split over 4 workgroups of 640 keys (the last split 129-148 keys) merged
    in-kernel by the pair's last workgroup. All 8 sequences and the K/V append
    against the oracle; the ragged case has splits with no key at all."""
    import ctypes

    import torchplusplus_amd
    from torchplusplus_amd._native import ext, lib

    C = ext()
    B, hq, hkv, D, Lmax = 8, 16, 8, 128, 2069
    f = lib().tpp_attn_decode_workspace_size
    f.restype = ctypes.c_size_t
    ws = f(*(ctypes.c_int64(v) for v in (B, hq, hkv, D, Lmax)))
    assert ws == 64 * 1024 + B * hq * 4 * (D + 32) * 4, f"plan is not 4 splits ({ws} B)"
    info = torchplusplus_amd.prepare_device(dev)
    assert info["xcd_local"], "XCD placement probe failed: the split merge would run unfused"
    g = torch.Generator().manual_seed(21)
    qkv = torch.randn(B, 1, (hq + 2 * hkv) * D, generator=g).bfloat16()
    qw = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    kw = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    cos, sin = oracle.compute_rope_params(D, 1e6, Lmax + 1)
    kc = torch.randn(B, hkv, Lmax, D, generator=g).bfloat16()
    vc = torch.randn(B, hkv, Lmax, D, generator=g).bfloat16()
    seqlens = torch.tensor(lens, dtype=torch.int32)
    e, k_ref, v_ref = _fused_decode_oracle(qkv, hq, hkv, qw, kw, cos, sin, kc, vc, seqlens - 1)
    kd, vd = kc.to(dev), vc.to(dev)
    got = C.attn_decode_fused(qkv.to(dev), qw.to(dev), kw.to(dev), cos.to(dev), sin.to(dev), 1e-6,
                              kd, vd, seqlens.to(dev))
    close(kd.cpu(), k_ref, what="model-shape fused decode: appended K")
    assert torch.equal(vd.cpu(), v_ref), "model-shape fused decode: appended V"
    close(got, e, what="model-shape fused decode vs oracle")
    # a second call over the same workspace (its arrival counters back at zero)
    got2 = C.attn_decode_fused(qkv.to(dev), qw.to(dev), kw.to(dev), cos.to(dev), sin.to(dev), 1e-6,
                               kd, vd, seqlens.to(dev))
    assert torch.equal(got, got2), "repeated call differs"


def _oproj_inputs(B, hq, hkv, Lmax, lens, seed, E=1024, D=128, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(B, 1, (hq + 2 * hkv) * D, generator=g).to(dtype)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(dtype)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(dtype)
    cos, sin = oracle.compute_rope_params(D, 1e6, Lmax + 1)
    kc = torch.randn(B, hkv, Lmax, D, generator=g).to(dtype)
    vc = torch.randn(B, hkv, Lmax, D, generator=g).to(dtype)
    w_o = (0.02 * torch.randn(E, hq * D, generator=g)).to(dtype)
    resid = torch.randn(B, 1, E, generator=g).to(dtype)
    return qkv, qw, kw, cos, sin, kc, vc, w_o, resid, torch.tensor(lens, dtype=torch.int32)


def _oproj_oracle(qkv, qw, kw, cos, sin, kc, vc, w_o, resid, seqlens, hq, hkv):
    """The reference block's attention half for one new token: QK-norm, RoPE,
    cache append, attention (torchpp/attention/gqa.py:90-128), the output
    projection and the residual add (examples/LLM/fastqwen3.py:107-111), each
    op's output rounded to the model dtype."""
    o, k_ref, v_ref = _fused_decode_oracle(qkv, hq, hkv, qw, kw, cos, sin, kc, vc, seqlens - 1)
    B = o.shape[0]
    proj = oracle.gemv(o.reshape(B, -1), w_o)
    return o, (resid.float() + proj.float().view(B, 1, -1)).to(resid.dtype), k_ref, v_ref


def _oproj_capi(o, kd, vd, qkv, qw, kw, cos, sin, seqlens, w_o, resid, ws):
    import ctypes

    from torchplusplus_amd._native import lib

    B, hkv, Lmax, D = kd.shape
    hq = o.shape[2]
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    ks = (ctypes.c_int64 * 3)(kd.stride(0), kd.stride(2), kd.stride(1))
    vs = (ctypes.c_int64 * 3)(vd.stride(0), vd.stride(2), vd.stride(1))
    L = lib()
    rc = L.tpp_attn_decode_oproj(
        P(qkv), P(qw), P(kw), P(cos), P(sin), ctypes.c_int64(cos.shape[0]), ctypes.c_int(0),
        ctypes.c_float(1e-6), P(kd), P(vd), P(o), ks, vs, P(seqlens), P(w_o), P(resid),
        ctypes.c_int64(B), ctypes.c_int64(hq), ctypes.c_int64(hkv), ctypes.c_int64(D),
        ctypes.c_int64(Lmax), ctypes.c_int64(w_o.shape[0]), ctypes.c_float(0.0), ctypes.c_int(-1),
        ctypes.c_int(1), P(ws), ctypes.c_size_t(ws.numel()),
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, L.tpp_last_error_string()


@pytest.mark.parametrize("lens", [[2049] * 8, [2068] * 8, [2068, 2049, 2060, 1921, 1920, 641, 640, 1]],
                         ids=["L2049", "L2068", "ragged"])
def test_decode_oproj_model_shape(dev, lens):
    """Decode attention with the output projection and residual add folded in
    (one launch) at the benchmark shape: batch 8, 16/8 heads, a 2069-row
    cache, W_o [1024, 2048]. Attention output, appended K/V and the updated
    residual against the oracle; the same launch through the C ABI on a
    workspace whose partial-projection region starts as NaN must leave it
    finite (the one-launch path ran, not the two-launch fallback) and give
    the binding's residual bit for bit."""
    import ctypes

    import torchplusplus_amd
    from torchplusplus_amd._native import ext, lib

    info = torchplusplus_amd.prepare_device(dev)
    if info["cu_count"] != 256:
        pytest.skip(f"the one-launch path needs 256 CUs, device has {info['cu_count']}")
    assert info["xcd_local"]
    C = ext()
    B, hq, hkv, D, Lmax, E = 8, 16, 8, 128, 2069, 1024
    qkv, qw, kw, cos, sin, kc, vc, w_o, resid, seqlens = _oproj_inputs(B, hq, hkv, Lmax, lens, 22)
    e_o, e_res, k_ref, v_ref = _oproj_oracle(qkv, qw, kw, cos, sin, kc, vc, w_o, resid, seqlens,
                                             hq, hkv)
    dq = [t.to(dev) for t in (qkv, qw, kw, cos, sin, seqlens, w_o)]
    kd, vd, rd = kc.to(dev), vc.to(dev), resid.to(dev)
    o = C.attn_decode_oproj(dq[0], dq[1], dq[2], dq[3], dq[4], 1e-6, kd, vd, dq[5], dq[6], rd)
    close(kd.cpu(), k_ref, what="oproj decode: appended K")
    assert torch.equal(vd.cpu(), v_ref), "oproj decode: appended V"
    close(o, e_o, what="oproj decode: attention output vs oracle")
    close(rd, e_res, what="oproj decode: residual vs oracle")
    assert C.attn_decode_sync_errors(rd) == 0
    # C ABI on a NaN-filled workspace
    f = lib().tpp_attn_decode_oproj_workspace_size
    f.restype = ctypes.c_size_t
    need = f(*(ctypes.c_int64(v) for v in (B, hq, hkv, D, Lmax, E)))
    part_off = 65536 + B * hq * 4 * (D + 32) * 4
    assert need == part_off + 8 * B * E * 4
    ws = torch.full((need,), 0xFF, dtype=torch.uint8, device=dev)
    ws[:65536] = 0
    kd2, vd2, rd2 = kc.to(dev), vc.to(dev), resid.to(dev)
    o2 = torch.empty_like(o)
    _oproj_capi(o2, kd2, vd2, dq[0], dq[1], dq[2], dq[3], dq[4], dq[5], dq[6], rd2, ws)
    torch.cuda.synchronize()
    part = ws[part_off:].view(torch.float32)
    assert torch.isfinite(part).all(), "partial projections not written: the fallback ran"
    assert torch.equal(rd2, rd) and torch.equal(o2, o)
    assert int(ws[:65536].view(torch.int32).abs().sum()) == 0, "counters not back at zero"


@pytest.mark.parametrize("B,hq,dtype", [(1, 16, torch.bfloat16), (2, 16, torch.bfloat16),
                                        (4, 16, torch.bfloat16), (16, 16, torch.bfloat16),
                                        (8, 8, torch.bfloat16), (16, 8, torch.bfloat16),
                                        (8, 16, torch.float16), (1, 8, torch.float16)])
def test_decode_oproj_batches_and_groups(dev, B, hq, dtype):
    """The one-launch path at every batch it takes (32 / B splits per
    sequence; B = 1 leaves most splits without a key), with one query head
    per KV head (G = 1, K slice 128), ragged lengths, bf16 and fp16 (the
    reference's model dtype), vs the oracle."""
    hkv, Lmax = 8, 700
    g = torch.Generator().manual_seed(B * 31 + hq)
    lens = torch.randint(1, Lmax + 1, (B,), generator=g).tolist()
    qkv, qw, kw, cos, sin, kc, vc, w_o, resid, seqlens = _oproj_inputs(B, hq, hkv, Lmax, lens, 23 + B,
                                                                       dtype=dtype)
    e_o, e_res, _, _ = _oproj_oracle(qkv, qw, kw, cos, sin, kc, vc, w_o, resid, seqlens, hq, hkv)
    from torchplusplus_amd._native import ext

    C = ext()
    rd = resid.to(dev)
    o = C.attn_decode_oproj(qkv.to(dev), qw.to(dev), kw.to(dev), cos.to(dev), sin.to(dev), 1e-6,
                            kc.to(dev), vc.to(dev), seqlens.to(dev), w_o.to(dev), rd)
    close(o, e_o, what=f"oproj decode B={B} Hq={hq} {dtype}: attention output")
    close(rd, e_res, what=f"oproj decode B={B} Hq={hq} {dtype}: residual")


def test_decode_oproj_unfolded_shape(dev):
    """Hkv = 4 (not one KV head per XCD): the entry point runs the fused
    decode attention and the projection GEMV; same results vs the oracle."""
    B, hq, hkv, Lmax = 3, 8, 4, 300
    qkv, qw, kw, cos, sin, kc, vc, w_o, resid, seqlens = _oproj_inputs(
        B, hq, hkv, Lmax, [300, 17, 1], 24, E=512)
    e_o, e_res, _, _ = _oproj_oracle(qkv, qw, kw, cos, sin, kc, vc, w_o, resid, seqlens, hq, hkv)
    from torchplusplus_amd._native import ext

    rd = resid.to(dev)
    o = ext().attn_decode_oproj(qkv.to(dev), qw.to(dev), kw.to(dev), cos.to(dev), sin.to(dev),
                                1e-6, kc.to(dev), vc.to(dev), seqlens.to(dev), w_o.to(dev), rd)
    close(o, e_o, what="unfolded oproj decode: attention output")
    close(rd, e_res, what="unfolded oproj decode: residual")


def test_decode_oproj_graph_replays_over_layers(dev):
    """28 launches over distinct caches and weights captured in one graph (as
    the decode step does), replayed three times with eager work in between:
    every replay equals the eager run (counters back at zero after every
    launch), and no launch gave up waiting."""
    from torchplusplus_amd._native import ext

    C = ext()
    B, hq, hkv, D, Lmax, E, NL = 8, 16, 8, 128, 640, 1024, 28
    g = torch.Generator(device=dev).manual_seed(25)
    cos, sin = (t.to(dev) for t in oracle.compute_rope_params(D, 1e6, Lmax + 1))
    layers = []
    for _ in range(NL):
        layers.append(((0.5 * torch.randn(B, 1, (hq + 2 * hkv) * D, generator=g, device=dev)).bfloat16(),
                       torch.randn(B, hkv, Lmax, D, generator=g, device=dev).bfloat16(),
                       torch.randn(B, hkv, Lmax, D, generator=g, device=dev).bfloat16(),
                       (0.02 * torch.randn(E, hq * D, generator=g, device=dev)).bfloat16()))
    seqlens = torch.randint(400, Lmax + 1, (B,), generator=g, device=dev, dtype=torch.int32)
    start = torch.randn(B, 1, E, generator=g, device=dev).bfloat16()
    resid = start.clone()

    def run():
        for qkv, kc, vc, w in layers:
            C.attn_decode_oproj(qkv, None, None, cos, sin, 1e-6, kc, vc, seqlens, w, resid)

    run()
    want = resid.clone()
    resid.copy_(start)
    run()
    assert torch.equal(resid, want), "eager runs differ"
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    resid.copy_(start)
    with torch.cuda.graph(graph, stream=s):
        run()
    for rep in range(3):
        resid.copy_(start)
        graph.replay()
        _ = torch.randn(1000, device=dev).sum()
        torch.cuda.synchronize()
        assert torch.equal(resid, want), f"replay {rep} differs from eager"
    assert C.attn_decode_sync_errors(resid) == 0
