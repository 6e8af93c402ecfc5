"""GPU parity: MFMA GEMM + activation epilogue, decode GEMV, SwiGLU."""
import pytest
import torch

import oracle
from tests.conftest import close
from torchplusplus_amd._native import ext
from torchplusplus_amd.dlops import linear as L

pytestmark = pytest.mark.gpu
ACTS = {"none": 0, "gelu": 1, "silu": 2, "relu": 3}


@pytest.fixture(params=["mfma", "vendor"])
def backend(request):
    """Plain GEMMs with at least one 256x256 tile per CU run on hipBLASLt unless
    the dispatch is switched off: each such test runs once on the MFMA
    kernels and once with the dispatch on. Yields a callable returning how
    many GEMMs hipBLASLt has run so far."""
    import ctypes
    from torchplusplus_amd._native import lib
    lb = lib()
    lb.tpp_gemm_vendor_runs.restype = ctypes.c_longlong
    prev = lb.tpp_gemm_vendor(1 if request.param == "vendor" else 0)
    try:
        yield request.param, lb.tpp_gemm_vendor_runs
    finally:
        lb.tpp_gemm_vendor(prev)


def _expect_backend(backend, runs_before, m, n):
    """The vendor path ran exactly when it was on and the shape has at least
    one 256x256 tile per CU; never with the dispatch off."""
    name, runs = backend
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    wanted = name == "vendor" and ((m + 255) // 256) * ((n + 255) // 256) >= cus
    assert (runs() > runs_before) == wanted, f"{name} backend, {m}x{n}: hipBLASLt runs {runs() - runs_before}"


def _mk(m, n, k, dtype, seed=0, wstd=0.02):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g).to(dtype)
    w = (wstd * torch.randn(n, k, generator=g)).to(dtype)
    b = (wstd * torch.randn(n, generator=g)).to(dtype)
    return x, w, b


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_linear_silu_baseline_config(dev, dtype):
    """BASELINE config 2b: [2048x1024] @ [1024x3072] + bias, SiLU."""
    x, w, b = _mk(2048, 3072, 1024, dtype)
    y = ext().LinearSilu(x.to(dev), w.to(dev), b.to(dev))
    close(y, oracle.linear_act(x, w, b, "silu"), what="linear+silu")


@pytest.mark.parametrize("act", ["none", "gelu", "silu", "relu"])
@pytest.mark.parametrize("m,n,k", [(300, 200, 136), (128, 128, 64), (1, 64, 1024), (257, 3, 8)])
def test_linear_act_shapes(dev, act, m, n, k):
    x, w, b = _mk(m, n, k, torch.bfloat16, seed=1, wstd=0.1)
    y = ext().linear(x.to(dev), w.to(dev), b.to(dev), ACTS[act])
    close(y, oracle.linear_act(x, w, b, act), what=f"linear {act} {m}x{n}x{k}")


@pytest.mark.parametrize("act", ["none", "gelu"])
@pytest.mark.parametrize("m,n", [(1100, 4100), (4096, 1100), (2048, 4096)])
def test_linear_pipelined_path_edges(dev, act, m, n):
    """Large K % 64 == 0 GEMMs (the LDS-DMA ring kernel): ragged M, N not a
    multiple of 8 (element-wise tail stores), and each tile shape."""
    x, w, b = _mk(m, n, 1024, torch.bfloat16, seed=21, wstd=0.05)
    y = ext().linear(x.to(dev), w.to(dev), b.to(dev), ACTS[act])
    close(y, oracle.linear_act(x, w, b, act), what=f"linear {act} {m}x{n}x1024")


@pytest.mark.parametrize("m,n", [(2048, 2048), (2048, 3072), (2048, 4096)])
@pytest.mark.parametrize("k", [64, 128, 192, 256, 320])
def test_linear_ring_depths_short_k(dev, m, n, k):
    """128x128 / 128x192 / 128x256 tiles (5-, 4- and 3-stage DMA rings) with
    fewer K steps than ring stages and every tail of the ring's waits."""
    x, w, b = _mk(m, n, k, torch.bfloat16, seed=25, wstd=0.05)
    y = ext().linear(x.to(dev), w.to(dev), b.to(dev), ACTS["silu"])
    close(y, oracle.linear_act(x, w, b, "silu"), what=f"linear silu {m}x{n}x{k}")


def test_linear_pipelined_strided_output(dev):
    """Output rows with a pitch (a column slice of a wider tensor) and K = 3072."""
    x, w, _ = _mk(2048, 2048, 3072, torch.float16, seed=22, wstd=0.02)
    out = torch.zeros(2048, 2056, dtype=torch.float16, device=dev)
    from torchplusplus_amd._native import lib
    import ctypes
    xd, wd = x.to(dev), w.to(dev)
    rc = lib().tpp_linear_act(ctypes.c_void_p(xd.data_ptr()), ctypes.c_void_p(wd.data_ptr()), None,
                              ctypes.c_void_p(out.data_ptr()), ctypes.c_int64(2048), ctypes.c_int64(2048),
                              ctypes.c_int64(3072), ctypes.c_int64(3072), ctypes.c_int64(2056),
                              ctypes.c_int(0), ctypes.c_int(0),
                              ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    close(out[:, :2048], oracle.linear_act(x, w, None, "none"), what="pitched output")
    assert torch.count_nonzero(out[:, 2048:]) == 0


@pytest.mark.parametrize("m,n,k,dtype", [(5900, 4100, 128, torch.bfloat16), (8900, 2700, 64, torch.float16),
                                         (16384, 2048, 320, torch.bfloat16)])
def test_linear_persistent_path(dev, backend, m, n, k, dtype):
    """256x256-tile launches with more tiles than CUs: on the MFMA kernels one
    workgroup per CU loops over its tiles, the K steps of consecutive tiles in
    one DMA stream (ragged M and N with element-wise tail stores, one K step
    per tile at K = 64, blocks with 1, 2 and 2+ tiles); with the dispatch on,
    hipBLASLt runs the same shapes."""
    x, w, _ = _mk(m, n, k, dtype, seed=23, wstd=0.05)
    before = backend[1]()
    y = ext().linear(x.to(dev), w.to(dev), None, ACTS["none"])
    torch.cuda.synchronize()
    _expect_backend(backend, before, m, n)
    close(y, oracle.linear_act(x, w, None, "none"), what=f"persistent {m}x{n}x{k} {backend[0]}")


def test_persistent_gemm_repeatable(dev, backend):
    """The persistent kernel's first K step of a tile waits only for the DMA
    issued before the previous tile's output stores (vector memory completes
    in issue order): 40 back-to-back launches on the same operands must give
    bit-identical outputs, equal to the oracle's within tolerance. The same
    holds for the hipBLASLt kernel the dispatch picks for this shape."""
    x, w, _ = _mk(16384, 2048, 512, torch.bfloat16, seed=26, wstd=0.05)
    xd, wd = x.to(dev), w.to(dev)
    before = backend[1]()
    ref = ext().linear(xd, wd, None, ACTS["none"])
    outs = [ext().linear(xd, wd, None, ACTS["none"]) for _ in range(40)]
    torch.cuda.synchronize()
    _expect_backend(backend, before, 16384, 2048)
    for i, y in enumerate(outs):
        assert torch.equal(y, ref), f"launch {i} differs"
    close(ref, oracle.linear_act(x, w, None, "none"), what=f"persistent repeat {backend[0]}")


@pytest.mark.parametrize("m,n,k,dtype", [(4352, 4096, 1024, torch.bfloat16), (4100, 4100, 1024, torch.float16),
                                         (16384, 1024, 3072, torch.bfloat16)])
def test_linear_vendor_matches_mfma(dev, m, n, k, dtype):
    """A plain GEMM with at least one 256x256 tile per CU gives the same result
    through hipBLASLt as through the MFMA kernel (both fp32 accumulation, one
    rounding), each within tolerance of the oracle; the prefill down
    projection's shape is the last case."""
    import ctypes
    from torchplusplus_amd._native import lib
    lb = lib()
    lb.tpp_gemm_vendor_runs.restype = ctypes.c_longlong
    x, w, _ = _mk(m, n, k, dtype, seed=31, wstd=0.05)
    xd, wd = x.to(dev), w.to(dev)
    prev = lb.tpp_gemm_vendor(1)
    try:
        r0 = lb.tpp_gemm_vendor_runs()
        y_v = ext().linear(xd, wd, None, ACTS["none"])
        torch.cuda.synchronize()
        assert lb.tpp_gemm_vendor_runs() == r0 + 1, "hipBLASLt did not run"
        lb.tpp_gemm_vendor(0)
        y_m = ext().linear(xd, wd, None, ACTS["none"])
        torch.cuda.synchronize()
        assert lb.tpp_gemm_vendor_runs() == r0 + 1
    finally:
        lb.tpp_gemm_vendor(prev)
    ref = oracle.linear_act(x, w, None, "none")
    close(y_v, ref, what=f"vendor {m}x{n}x{k}")
    close(y_m, ref, what=f"mfma {m}x{n}x{k}")
    # same inputs, two fp32-accumulating kernels: at most one rounding step apart
    close(y_v, y_m, atol=1e-2, rtol=8e-3, what=f"vendor vs mfma {m}x{n}x{k}")


def test_linear_vendor_in_graph(dev):
    """A hipBLASLt GEMM captured into a HIP graph: every replay, with eager
    work and a synchronisation between replays, equals the eager result."""
    import ctypes
    from torchplusplus_amd._native import lib
    lb = lib()
    lb.tpp_gemm_vendor_runs.restype = ctypes.c_longlong
    x, w, _ = _mk(4352, 4096, 1024, torch.bfloat16, seed=33, wstd=0.05)
    xd, wd = x.to(dev), w.to(dev)
    prev = lb.tpp_gemm_vendor(1)
    try:
        y_e = ext().linear(xd, wd, None, ACTS["none"])  # eager: builds the plan
        torch.cuda.synchronize()
        r0 = lb.tpp_gemm_vendor_runs()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            y = ext().linear(xd, wd, None, ACTS["none"])
        assert lb.tpp_gemm_vendor_runs() == r0 + 1, "hipBLASLt was not captured"
        for r in range(4):
            y.fill_(float(r + 1))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, y_e), f"replay {r} differs from the eager result"
    finally:
        lb.tpp_gemm_vendor(prev)
    close(y_e, oracle.linear_act(x, w, None, "none"), what="vendor eager")


def test_linear_vendor_shape_first_met_under_capture(dev):
    """A plain GEMM shape never run eagerly and first met inside a graph
    capture runs on the MFMA kernel (no hipBLASLt plan is made during a
    capture); its replays match the eager result, which then runs on
    hipBLASLt."""
    import ctypes
    from torchplusplus_amd._native import lib
    lb = lib()
    lb.tpp_gemm_vendor_runs.restype = ctypes.c_longlong
    m, n = 4352 + 256, 4096  # a shape no other test uses
    x, w, _ = _mk(m, n, 1024, torch.bfloat16, seed=34, wstd=0.05)
    xd, wd = x.to(dev), w.to(dev)
    prev = lb.tpp_gemm_vendor(1)
    try:
        r0 = lb.tpp_gemm_vendor_runs()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            y = ext().linear(xd, wd, None, ACTS["none"])
        assert lb.tpp_gemm_vendor_runs() == r0, "hipBLASLt planned a shape during capture"
        g.replay()
        torch.cuda.synchronize()
        y_e = ext().linear(xd, wd, None, ACTS["none"])
        torch.cuda.synchronize()
        assert lb.tpp_gemm_vendor_runs() == r0 + 1, "eager call did not run on hipBLASLt"
    finally:
        lb.tpp_gemm_vendor(prev)
    ref = oracle.linear_act(x, w, None, "none")
    close(y, ref, what="captured (MFMA kernel)")
    close(y_e, ref, what="eager (hipBLASLt)")


def test_linear_vendor_pitched_output(dev):
    """hipBLASLt path with an output row pitch (a column slice of a wider
    tensor): the columns past N stay untouched."""
    import ctypes
    from torchplusplus_amd._native import lib
    lb = lib()
    lb.tpp_gemm_vendor_runs.restype = ctypes.c_longlong
    x, w, _ = _mk(4352, 4096, 1024, torch.bfloat16, seed=32, wstd=0.05)
    xd, wd = x.to(dev), w.to(dev)
    out = torch.zeros(4352, 4104, dtype=torch.bfloat16, device=dev)
    prev = lb.tpp_gemm_vendor(1)
    try:
        r0 = lb.tpp_gemm_vendor_runs()
        rc = lb.tpp_linear_act(ctypes.c_void_p(xd.data_ptr()), ctypes.c_void_p(wd.data_ptr()), None,
                               ctypes.c_void_p(out.data_ptr()), ctypes.c_int64(4352), ctypes.c_int64(4096),
                               ctypes.c_int64(1024), ctypes.c_int64(1024), ctypes.c_int64(4104),
                               ctypes.c_int(0), ctypes.c_int(1),
                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert rc == 0
        torch.cuda.synchronize()
        assert lb.tpp_gemm_vendor_runs() == r0 + 1, "hipBLASLt did not run"
    finally:
        lb.tpp_gemm_vendor(prev)
    close(out[:, :4096], oracle.linear_act(x, w, None, "none"), what="vendor pitched output")
    assert torch.count_nonzero(out[:, 4096:]) == 0


@pytest.mark.parametrize("rows,inter,k", [(5200, 2400, 192), (16384, 3072, 128)])
def test_swiglu_persistent_path(dev, rows, inter, k):
    """SwiGLU through the persistent 256x256 kernel: ragged rows and [gate|up]
    pairs past the last full tile."""
    g = torch.Generator().manual_seed(24)
    x = torch.randn(rows, k, generator=g).bfloat16()
    wg = (0.05 * torch.randn(inter, k, generator=g)).bfloat16()
    wu = (0.05 * torch.randn(inter, k, generator=g)).bfloat16()
    y = L.swiglu(x.to(dev), L.interleave_gate_up(wg, wu).to(dev))
    gt = oracle.linear_act(x, wg)
    e = (torch.nn.functional.silu(gt.float()).bfloat16().float() * oracle.linear_act(x, wu).float()).bfloat16()
    close(y, e, what=f"swiglu persistent {rows}x{inter}x{k}")


def test_linear_odd_k_scalar_path(dev):
    x, w, b = _mk(33, 40, 13, torch.float16, seed=2, wstd=0.2)
    y = ext().linear(x.to(dev), w.to(dev), None, ACTS["gelu"])
    close(y, oracle.linear_act(x, w, None, "gelu"), what="odd K")


def test_reference_linear_act_test_shape(dev):
    """tests/linear_act_test.py:5-17: x [32,512], W [256,512] fp16 randn (shape only
    there); checked here against the formula."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(32, 512, generator=g).half()
    w = torch.randn(256, 512, generator=g).half()
    y = ext().LinearSilu(x.to(dev), w.to(dev))
    assert y.shape == (32, 256)
    e = oracle.linear_act(x, w, None, "silu")
    # |acc| ~ sqrt(512) ~ 22: fp16 pre-activation rounding alone is 2^-6 there
    close(y, e, atol=6e-2, rtol=1e-2, what="randn weights")


def test_linear_module_3d_input(dev):
    mod = L.LinearGELU(256, 512, dtype=torch.bfloat16, device=dev)
    with torch.no_grad():
        mod.weight.mul_(0.05)
    x = torch.randn(4, 100, 256, generator=torch.Generator().manual_seed(4)).bfloat16()
    y = mod(x.to(dev))
    assert y.shape == (4, 100, 512)
    close(y, oracle.linear_act(x, mod.weight.detach().cpu(), None, "gelu"), what="3-D")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bsz", [1, 8, 16])
@pytest.mark.parametrize("n,k", [(3072, 1024), (1024, 3072), (4096, 1024), (1000, 200), (24, 2048),
                                 (1003, 4096)])
def test_gemv_parity(dev, dtype, bsz, n, k):
    """[1x1024]@[1024x3072] and [1x3072]@[3072x1024]; plus the
    decode-step shapes at batch 8/16 and ragged sizes (a last row tile past N,
    K shorter than one 256-wide wave batch, K longer than 12 wave batches with
    8-row tiles)."""
    x, w, _ = _mk(bsz, n, k, dtype, seed=5)
    y = ext().gemv(x.to(dev), w.to(dev))
    close(y, oracle.gemv(x, w), what=f"gemv b{bsz} {n}x{k}")


@pytest.mark.parametrize("n,k", [(257, 8), (100, 520), (2049, 4096), (3, 4088), (5000, 1536)])
@pytest.mark.parametrize("epi", ["plain", "gelu", "residual"])
def test_gemv_one_row_input(dev, n, k, epi):
    """Batch 1 (the reference's hgemv): one weight row per wave, 1 to 8
    16-byte chunks per lane, K not a multiple of 512 (the last chunks of a
    row past K), more rows than waves of one block per CU; plain, bias + GeLU
    and residual epilogues."""
    x, w, b = _mk(1, n, k, torch.float16, seed=n + k)
    xd, wd = x.to(dev), w.to(dev)
    if epi == "plain":
        close(ext().gemv(xd, wd), oracle.gemv(x, w), what=f"b1 {n}x{k}")
    elif epi == "gelu":
        close(ext().gemv(xd, wd, b.to(dev), ACTS["gelu"]), oracle.linear_act(x, w, b, "gelu"),
              what=f"b1 gelu {n}x{k}")
    else:
        r = torch.randn(1, n, generator=torch.Generator().manual_seed(k)).half()
        rd = r.to(dev)
        ext().gemv_fused(xd, wd, None, 1e-6, rd)
        close(rd, (r.float() + oracle.gemv(x, w).float()).half(), what=f"b1 residual {n}x{k}")


def test_gemv_repeated_calls_are_deterministic(dev):
    """No cross-block reduction: repeated calls give bit-identical results."""
    x, w, _ = _mk(8, 1024, 3072, torch.bfloat16, seed=6)
    xd, wd = x.to(dev), w.to(dev)
    first = ext().gemv(xd, wd)
    for _ in range(20):
        again = ext().gemv(xd, wd)
    assert torch.equal(first, again)
    close(first, oracle.gemv(x, w), what="repeat")


def test_gemv_bias_act_and_hgemv_cpu_reference(dev):
    import numpy as np

    x, w, b = _mk(1, 512, 1024, torch.float16, seed=7)
    y = ext().gemv(x.to(dev), w.to(dev), b.to(dev), ACTS["silu"])
    close(y, oracle.linear_act(x, w, b, "silu"), what="gemv silu")
    y0 = ext().gemv(x.to(dev), w.to(dev))
    ref = oracle.hgemv_cpu(w.numpy(), x[0].numpy())
    close(y0[0], torch.from_numpy(ref), what="vs hgemvCpu restatement")


@pytest.mark.parametrize("rows", [1, 8, 300, 1100])
def test_swiglu_gemm_and_gemv(dev, rows):
    g = torch.Generator().manual_seed(8)
    I, K = 3072, 1024
    x = torch.randn(rows, K, generator=g).bfloat16()
    wg = (0.02 * torch.randn(I, K, generator=g)).bfloat16()
    wu = (0.02 * torch.randn(I, K, generator=g)).bfloat16()
    wgu = L.interleave_gate_up(wg, wu)
    y = L.swiglu(x.to(dev), wgu.to(dev))
    gt = oracle.linear_act(x, wg)
    e = (torch.nn.functional.silu(gt.float()).bfloat16().float() * oracle.linear_act(x, wu).float()).bfloat16()
    close(y, e, what=f"swiglu rows={rows}")


@pytest.mark.parametrize("bsz", [1, 8])
@pytest.mark.parametrize("n,k", [(4096, 1024), (1024, 3072), (40, 1024)])
def test_gemv_fused_input_rmsnorm(dev, bsz, n, k):
    x, w, _ = _mk(bsz, n, k, torch.bfloat16, seed=9)
    nw = (1 + 0.1 * torch.randn(k, generator=torch.Generator().manual_seed(10))).bfloat16()
    y = ext().gemv_fused(x.to(dev), w.to(dev), nw.to(dev), 1e-6)
    close(y, oracle.linear_act(oracle.rmsnorm(x, nw, 1e-6), w), what="gemv(rmsnorm(x))")


@pytest.mark.parametrize("bsz", [1, 8, 16])
@pytest.mark.parametrize("n,k", [(1024, 2048), (1024, 3072), (1003, 1000), (20000, 512), (1024, 5000)])
def test_gemv_fused_residual_add(dev, bsz, n, k):
    """Residual += x W^T: one tile per workgroup, workgroups looping over
    several tiles (N = 20000: more tiles than workgroups, the next tile's
    residual values requested with its weights), and K slices longer than
    one load batch (K = 5000)."""
    x, w, _ = _mk(bsz, n, k, torch.bfloat16, seed=11)
    r = torch.randn(bsz, n, generator=torch.Generator().manual_seed(12)).bfloat16()
    rd = r.to(dev)
    out = ext().gemv_fused(x.to(dev), w.to(dev), None, 1e-6, rd)
    assert out.data_ptr() == rd.data_ptr()
    e = (r.float() + oracle.linear_act(x, w).float()).bfloat16()
    close(rd, e, what="residual += x W^T")


@pytest.mark.parametrize("bsz", [3, 8])
def test_gemv_fused_norm_and_residual(dev, bsz):
    """Input RMSNorm and residual add in one GEMV (every wave loads the
    residual values there, counted by the input's asm wait)."""
    x, w, _ = _mk(bsz, 4096, 1024, torch.bfloat16, seed=13)
    nw = (1 + 0.1 * torch.randn(1024, generator=torch.Generator().manual_seed(14))).bfloat16()
    r = torch.randn(bsz, 4096, generator=torch.Generator().manual_seed(15)).bfloat16()
    rd = r.to(dev)
    ext().gemv_fused(x.to(dev), w.to(dev), nw.to(dev), 1e-6, rd)
    e = (r.float() + oracle.linear_act(oracle.rmsnorm(x, nw, 1e-6), w).float()).bfloat16()
    close(rd, e, what="residual += rmsnorm(x) W^T")


def test_gemv_swiglu_with_input_norm(dev):
    g = torch.Generator().manual_seed(13)
    I, K = 3072, 1024
    x = torch.randn(8, K, generator=g).bfloat16()
    nw = (1 + 0.1 * torch.randn(K, generator=g)).bfloat16()
    wg = (0.02 * torch.randn(I, K, generator=g)).bfloat16()
    wu = (0.02 * torch.randn(I, K, generator=g)).bfloat16()
    y = ext().gemv_swiglu(x.to(dev), L.interleave_gate_up(wg, wu).to(dev), nw.to(dev), 1e-6)
    h = oracle.rmsnorm(x, nw, 1e-6)
    gt = oracle.linear_act(h, wg)
    e = (torch.nn.functional.silu(gt.float()).bfloat16().float() * oracle.linear_act(h, wu).float()).bfloat16()
    close(y, e, what="swiglu(rmsnorm(x))")


@pytest.mark.parametrize("bsz,n", [(8, 151936), (3, 1000), (1, 17)])
def test_gemv_argmax_lm_head(dev, bsz, n):
    x, w, _ = _mk(bsz, n, 1024, torch.bfloat16, seed=14)
    nw = (1 + 0.1 * torch.randn(1024, generator=torch.Generator().manual_seed(15))).bfloat16()
    idx, logits = ext().gemv_argmax(x.to(dev), w.to(dev), nw.to(dev), 1e-6, True)
    assert torch.equal(idx.cpu(), torch.argmax(logits.cpu().float(), dim=-1))
    close(logits, oracle.linear_act(oracle.rmsnorm(x, nw, 1e-6), w), what="lm_head logits")
    only = ext().gemv_argmax(x.to(dev), w.to(dev), nw.to(dev), 1e-6, False)
    assert len(only) == 1 and torch.equal(only[0], idx)


@pytest.mark.parametrize("bsz,n,k,norm", [(16, 40001, 512, True), (1, 33000, 256, False),
                                           (5, 50000, 768, True), (8, 36000, 1024, False),
                                           (2, 34000, 256, True)])
def test_gemv_wide_path(dev, bsz, n, k, norm):
    """>= 2048 row tiles with K % 256 == 0 run the whole-K-per-wave kernel:
    ragged last tile, every chunk count, with and without the input norm."""
    x, w, _ = _mk(bsz, n, k, torch.bfloat16, seed=23)
    nw = (1 + 0.1 * torch.randn(k, generator=torch.Generator().manual_seed(24))).bfloat16()
    idx, logits = ext().gemv_argmax(x.to(dev), w.to(dev), nw.to(dev) if norm else None, 1e-6, True)
    xin = oracle.rmsnorm(x, nw, 1e-6) if norm else x
    close(logits, oracle.linear_act(xin, w), what=f"wide gemv {bsz}x{n}x{k}")
    assert torch.equal(idx.cpu(), torch.argmax(logits.cpu().float(), dim=-1))
    y = ext().gemv(x.to(dev), w.to(dev))
    close(y, oracle.gemv(x, w), what=f"wide plain gemv {bsz}x{n}x{k}")


@pytest.mark.parametrize("n", [5000, 40000])
def test_greedy_step_tail(dev, n):
    """argmax -> ids, next embedding gathered into the residual row, and the
    position/length advance, in one call (llm.py:181-186, 226-236)."""
    bsz, k = 8, 1024
    x, w, _ = _mk(bsz, n, k, torch.bfloat16, seed=16)
    nw = (1 + 0.1 * torch.randn(k, generator=torch.Generator().manual_seed(17))).bfloat16()
    emb = torch.randn(n, k, generator=torch.Generator().manual_seed(18)).bfloat16()
    # a duplicated, dominant row pair: the first index must win across blocks
    w[3] *= 8
    w[n - 7] = w[3]
    xd, wd, nwd = x.to(dev), w.to(dev), nw.to(dev)
    want, logits = ext().gemv_argmax(xd, wd, nwd, 1e-6, True)
    e = oracle.linear_act(oracle.rmsnorm(x, nw, 1e-6), w)
    close(logits, e, what="lm_head logits")
    assert torch.equal(want.cpu(), torch.argmax(logits.cpu().float(), dim=-1))
    ids = torch.full((bsz, 1), -1, dtype=torch.long, device=dev)
    resid = xd.clone()
    pos = torch.arange(bsz, dtype=torch.int32, device=dev)
    sl = pos + 1
    ext().greedy_step(resid, wd, nwd, 1e-6, emb.to(dev), ids, resid, pos, sl)
    assert torch.equal(ids.view(-1), want)
    assert torch.equal(resid.cpu(), emb[want.cpu()])
    assert pos.cpu().tolist() == list(range(1, bsz + 1))
    assert sl.cpu().tolist() == list(range(2, bsz + 2))


def test_argmax_first_index_on_ties(dev):
    x = torch.zeros(2, 1000).bfloat16()
    x[0, [5, 700]] = 3.0
    x[1, 999] = 1.0
    x[1, 998] = 1.0
    assert ext().argmax_rows(x.to(dev)).cpu().tolist() == [5, 998]
