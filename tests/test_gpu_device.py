"""GPU parity of the device-resident entry points (``*_dev``) at the
benchmark configurations' shapes: bf16 activations, the T1 cache handed from forward to
backward, and full-size size-independent checks.

Outputs are compared with the oracle on sampled rows (every output row is
an independent reduction, so a row sample is exact per row); grad_A and
grad_B are compared in full.
"""
import numpy as np
import pytest

import oracle as O
from gpu_layer import run_layer as _run, say as _say, setup_layer as _setup
from parity import SEED, TOL_BF16, TOL_F32, nerr

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def QD(ctx):
    from qlora_hip import device
    return device


@pytest.mark.parametrize("act", [torch.float32, torch.bfloat16])
def test_prefill_shape_parity(ctx, QD, act):
    # config 3 at a reduced token count (the kernels and tiles are the same)
    N = K = 4096
    r, M, alpha = 64, 512, 16.0
    _say(f"prefill-shape parity act={act}")
    d = _setup(QD, ctx, N, K, r, M, SEED ^ 3, act)
    rows = [0, 1, 127, 128, 255, 300, 511]
    e = _run(QD, ctx, d, N, K, r, M, alpha, rows)
    tol = TOL_F32 if act == torch.float32 else TOL_BF16
    _say(e)
    assert all(v < tol for v in e.values()), e


@pytest.mark.parametrize("N,K,r,M,act", [
    (576, 576, 8, 100, torch.float32),     # C4/C1 class: T1 and Ds on the rank kernel
    (192, 576, 33, 70, torch.bfloat16),    # r past one 32-column block, bf16 X and dY
    (576, 1024, 64, 33, torch.float32),    # r = 64: four 16-column blocks
    (192, 2048, 64, 37, torch.float32),    # the largest K the rank kernel takes
    (640, 320, 1, 40, torch.bfloat16),     # rank 1
    (256, 200, 16, 50, torch.float32),     # K not a multiple of 16 (fp32 weight path)
    (1536, 576, 8, 64, torch.float32),     # Ds over N = 1536
    (256, 2560, 16, 40, torch.float32),    # T1 past K = 2048: the dense bf16 kernel
    (320, 640, 24, 2104, torch.float32),   # grad_A / grad_B past 2048 tokens: dense kernel
    (512, 384, 40, 2300, torch.bfloat16),  # the same with bf16 X and dY, ragged tiles
    (192, 576, 33, 2050, torch.float32),   # r not a multiple of 8: the tile engine
])
def test_rank_gemm_shapes_parity(ctx, QD, N, K, r, M, act):
    _say(f"rank-gemm shapes N={N} K={K} r={r} M={M} act={act}")
    d = _setup(QD, ctx, N, K, r, M, SEED ^ (N * 31 + K), act)
    rows = sorted({0, 1, M // 2, M - 1})
    e = _run(QD, ctx, d, N, K, r, M, 8.0, rows)
    tol = TOL_F32 if act == torch.float32 else TOL_BF16
    _say(e)
    assert all(v < tol for v in e.values()), e


@pytest.mark.parametrize("N,K", [(11008, 4096), (4096, 11008)])
@pytest.mark.parametrize("M", [1, 4, 16])
def test_decode_shape_forward_parity(ctx, QD, N, K, M):
    # config 2: forward only
    _say(f"decode parity N={N} K={K} M={M}")
    r, alpha = 16, 32.0
    d = _setup(QD, ctx, N, K, r, M, SEED ^ 2)
    lora = QD.lora_struct(d["ta"], d["tb"], r, alpha)
    y = torch.empty(M, N, device="cuda:0")
    QD.forward(d["W"], lora, d["tx"], M, y, ctx=ctx)
    torch.cuda.synchronize()
    wd = O.dequantize(O.quantize(d["w"]))
    yo = O.qlora_forward(wd, N, K, d["a"], d["b"], r, alpha, d["x"], M)
    e = nerr(y.cpu().numpy().ravel(), yo, K, d["x"], wd)
    assert e < TOL_F32, e


@pytest.mark.parametrize("act", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M", [1, 2, 7, 16])
def test_decode_path_ragged_rows_t1_and_dtypes(ctx, QD, act, M):
    # batch <= 16 with in_dim % 256 == 0 takes the MFMA decode kernel;
    # N = 300 is not a multiple of its 16-row tile
    N, K, r, alpha = 300, 512, 8, 16.0
    _say(f"decode path M={M} act={act}")
    d = _setup(QD, ctx, N, K, r, M, SEED ^ (M + 77), act)
    lora = QD.lora_struct(d["ta"], d["tb"], r, alpha)
    y = torch.empty(M, N, device="cuda:0")
    t1 = torch.empty(M, r, device="cuda:0")
    QD.forward(d["W"], lora, d["tx"], M, y, t1=t1, ctx=ctx)
    y0 = torch.empty(M, N, device="cuda:0")
    QD.forward(d["W"], None, d["tx"], M, y0, ctx=ctx)
    torch.cuda.synchronize()
    wd = O.dequantize(O.quantize(d["w"]))
    tol = TOL_F32 if act == torch.float32 else TOL_BF16
    yo = O.qlora_forward(wd, N, K, d["a"], d["b"], r, alpha, d["x"], M)
    assert nerr(y.cpu().numpy().ravel(), yo, K, d["x"], wd) < tol
    y0o = O.qlora_forward(wd, N, K, None, None, 0, 0.0, d["x"], M)
    assert nerr(y0.cpu().numpy().ravel(), y0o, K, d["x"], wd) < tol
    t1o = O.matmul_trans_b(d["x"], d["a"], M, K, r)
    assert nerr(t1.cpu().numpy().ravel(), t1o, K, d["x"], d["a"]) < tol


def test_decode_path_f32_scales(ctx, QD):
    N, K, M = 64, 1024, 3
    g = O.Rng(12)
    w, x = g.normal(N * K, 0.02), g.normal(M * K)
    W = QD.DeviceWeight.quantize(torch.from_numpy(w).cuda().view(N, K),
                                 double_quant=False, ctx=ctx)
    y = torch.empty(M, N, device="cuda:0")
    QD.forward(W, None, torch.from_numpy(x).cuda(), M, y, ctx=ctx)
    torch.cuda.synchronize()
    wd = O.dequantize(O.quantize(w, 64, False))
    yo = O.qlora_forward(wd, N, K, None, None, 0, 0.0, x, M)
    assert nerr(y.cpu().numpy().ravel(), yo, K, x, wd) < TOL_F32


def test_smollm_block_projections_and_adam(ctx, QD):
    # config 4: seven projections fwd+bwd at 8x256 tokens, then one
    # PagedAdam step (max_resident_pages=4) over the 14 adapter tensors
    import qlora_hip as QH
    projs = [(576, 576), (192, 576), (192, 576), (576, 576), (1536, 576),
             (1536, 576), (576, 1536)]
    M, r, alpha = 2048, 8, 16.0
    grads_dev, params_dev, params_np = [], [], []
    for i, (N, K) in enumerate(projs):
        d = _setup(QD, ctx, N, K, r, M, SEED ^ (40 + i))
        e = _run(QD, ctx, d, N, K, r, M, alpha, [0, 1000, 2047])
        assert all(v < TOL_F32 for v in e.values()), (i, e)
    # Adam over 14 tensors, device path vs oracle, bit-exact
    g = O.Rng(SEED ^ 99)
    lens = []
    for N, K in projs:
        lens += [r * K, N * r]
    p_np = [g.normal(n, 0.05) for n in lens]
    gr_np = [g.normal(n, 0.01) for n in lens]
    p_dev = [torch.from_numpy(p).cuda() for p in p_np]
    g_dev = [torch.from_numpy(x).cuda() for x in gr_np]
    import ctypes as C
    opt = QH.Adam8bit(lr=1e-3, max_resident_pages=4, ctx=ctx)
    oo = O.Adam8bit(lr=1e-3, max_resident_pages=4)
    cnt = len(lens)
    pp = (C.c_void_p * cnt)(*[t.data_ptr() for t in p_dev])
    gp = (C.c_void_p * cnt)(*[t.data_ptr() for t in g_dev])
    ll = (C.c_size_t * cnt)(*lens)
    st = QH._lib.AdamStats()
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    QH._lib.check(ctx.lib.qh_adam8bit_step_dev(opt.h, pp, gp, ll, cnt, C.byref(st),
                                               stream))
    pages = oo.step(p_np, gr_np)
    torch.cuda.synchronize()
    assert st.pages_streamed == pages == 318
    for t, p in zip(p_dev, p_np):
        assert np.array_equal(t.cpu().numpy().view(np.uint32), p.view(np.uint32))


def test_quantize_70b_layer_bit_exact(ctx, QD):
    # config 5's quantize pass at full size (28672 x 8192), bit-exact
    N, K = 28672, 8192
    _say("quantize 28672x8192")
    gen = torch.Generator(device="cuda").manual_seed(5)
    w = torch.randn(N, K, device="cuda", generator=gen) * 0.02
    W = QD.DeviceWeight.quantize(w, ctx=ctx)
    torch.cuda.synchronize()
    q = O.quantize(w.cpu().numpy().ravel())
    assert np.array_equal(W.codes.cpu().numpy(), q["codes"])
    assert np.array_equal(W.scale_codes.cpu().numpy(), q["scale_codes"])
    assert np.array_equal(W.absmax.cpu().numpy().view(np.uint32),
                          q["absmax"].view(np.uint32))
    # dequantize at full size, bit-exact
    wd = W.dequantize(ctx=ctx).cpu().numpy()
    assert np.array_equal(wd.view(np.uint32), O.dequantize(q).view(np.uint32))


def test_library_owned_weight_handle(ctx, QD):
    """qh_weight_upload keeps a packed weight in HBM; its view drives the
    device entry points like any device qh_qweight."""
    import ctypes as C
    from qlora_hip._lib import QWeight
    from qlora_hip.api import qweight_struct
    N, K, r, M = 256, 512, 8, 40
    g = O.Rng(SEED ^ 0x77)
    w = g.normal(N * K, 0.02)
    q = O.quantize(w)
    q.update(rows=N, cols=K)
    hs = qweight_struct(q)
    h = C.c_void_p()
    QD.check(ctx.lib.qh_weight_upload(ctx.h, C.byref(hs), C.byref(h)))
    try:
        v = QWeight()
        QD.check(ctx.lib.qh_dweight_view(h, C.byref(v)))
        out = torch.empty(N * K, device="cuda:0")
        QD.check(ctx.lib.qh_dequantize_dev(ctx.h, C.byref(v), QD._p(out), None))
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), O.dequantize(q).view(np.uint32))
        a, b = g.uniform(r * K, -0.04, 0.04), g.normal(N * r, 0.01)
        x = g.normal(M * K)
        y = torch.empty(M, N, device="cuda:0")
        lora = QD.lora_struct(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(), r, 16.0)
        QD.forward(None, lora, torch.from_numpy(x).cuda().view(M, K), M, y, ctx=ctx, qw=v)
        torch.cuda.synchronize()
        wd = O.dequantize(q)
        yo = O.qlora_forward(wd, N, K, a, b, r, 16.0, x, M)
        assert nerr(y.cpu().numpy().ravel(), yo, K, x, wd) < TOL_F32
    finally:
        ctx.lib.qh_dweight_destroy(h)


@pytest.mark.parametrize("N,K,M", [(48, 0, 5), (0, 96, 5), (48, 96, 0)])
def test_empty_reductions(ctx, QD, N, K, M):
    """A layer with in_dim, out_dim or batch 0 (qlora.rs:86-165): every
    requested output is written, zeros where the reduction is empty, T1
    computed when out_dim alone is 0."""
    r, alpha = 4, 8.0
    dev = torch.device("cuda:0")
    g = O.Rng(SEED ^ (N + 3 * K + 7 * M))
    a, b = g.uniform(r * K, -0.1, 0.1), g.normal(N * r, 0.01)
    x, dy = g.normal(M * K), g.normal(M * N)
    if N * K:
        w = g.normal(N * K, 0.02)
        W = QD.DeviceWeight.quantize(torch.from_numpy(w).to(dev).view(N, K), ctx=ctx)
        wd = O.dequantize(O.quantize(w))
    else:
        W = QD.DeviceWeight(N, K, 64, torch.empty(0, dtype=torch.uint8, device=dev),
                            scale_codes=torch.empty(0, dtype=torch.uint8, device=dev),
                            absmax=torch.empty(0, device=dev))
        wd = np.zeros(0, np.float32)
    t = lambda v: torch.from_numpy(v).to(dev)  # noqa: E731
    nan = lambda *s: torch.full(s, float("nan"), device=dev)  # noqa: E731
    lora = QD.lora_struct(t(a), t(b), r, alpha)
    y, t1, gx, ga, gb = nan(M, N), nan(M, r), nan(M, K), nan(r, K), nan(N, r)
    QD.forward(W, lora, t(x), M, y, t1=t1, ctx=ctx)
    QD.backward(W, lora, t(x), t(dy), M, gx, ga, gb, ctx=ctx)
    torch.cuda.synchronize()
    yo = O.qlora_forward(wd, N, K, a, b, r, alpha, x, M)
    gxo, gao, gbo = O.qlora_backward(wd, N, K, a, b, r, alpha, x, dy, M)
    t1o = O.matmul_trans_b(x, a, M, K, r)
    for got, want in ((y, yo), (gx, gxo), (ga, gao), (gb, gbo)):
        assert np.array_equal(got.cpu().numpy().ravel(), want)
    assert nerr(t1.cpu().numpy().ravel(), t1o, K, x, a) < TOL_F32


@pytest.mark.parametrize("act", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("N,K,M,r", [
    (4200, 4160, 1100, 16),   # ragged M, N (256 x 128 tiles) and grad_x reduction (4200 rows)
    (4200, 4160, 1100, 0),    # no adapter
    (4096, 4096, 1024, 64),   # 256 x 256 tiles for grad_x, two LoRA steps
])
def test_bf16_mfma_path_parity(ctx, QD, N, K, M, r, act):
    """The large GEMMs on bf16 MFMA (weight as hi + lo bf16 parts; bf16
    activations exact, fp32 ones as hi + lo with three MFMAs per product;
    LoRA as three MFMAs): forward and grad_x against the oracle.  The bar is
    2e-4 for bf16 activations (tighter than their 5e-3) and fp32's 1e-4: the
    splits leave ~1e-5, while dropping any lo part would leave ~1e-3."""
    _say(f"bf16 MFMA path N={N} K={K} M={M} r={r} act={act}")
    rr = max(r, 1)
    d = _setup(QD, ctx, N, K, rr, M, SEED ^ (N + K + M + r), act)
    dev = torch.device("cuda:0")
    lora = QD.lora_struct(d["ta"], d["tb"], r, 16.0) if r else None
    y = torch.empty(M, N, device=dev)
    t1 = torch.empty(M, rr, device=dev) if r else None
    gx = torch.empty(M, K, device=dev)
    ga = torch.empty(rr, K, device=dev) if r else None
    gb = torch.empty(N, rr, device=dev) if r else None
    ctx.set_timing(True)
    ctx.timing_report(reset=True)
    QD.forward(d["W"], lora, d["tx"], M, y, t1=t1, ctx=ctx)
    QD.backward(d["W"], lora, d["tx"], d["tdy"], M, gx, ga, gb, t1=t1, ctx=ctx)
    torch.cuda.synchronize()
    rep = ctx.timing_report(reset=True)
    ctx.set_timing(False)
    assert "forward_gemm_bf16" in rep and "grad_x_gemm_bf16" in rep, rep
    wd = O.dequantize(O.quantize(d["w"]))
    rows = [0, 1, 255, 256, M // 2, M - 1]
    xs = d["x"].reshape(M, K)[rows].ravel()
    dys = d["dy"].reshape(M, N)[rows].ravel()
    a, b = (d["a"], d["b"]) if r else (None, None)
    yo = O.qlora_forward(wd, N, K, a, b, r, 16.0, xs, len(rows))
    gxo, _, _ = O.qlora_backward(wd, N, K, a, b, r, 16.0, xs, dys, len(rows))
    ey = nerr(y.cpu().numpy()[rows].ravel(), yo, K, xs, wd)
    egx = nerr(gx.cpu().numpy()[rows].ravel(), gxo, N, dys, wd)
    _say(dict(y=ey, gx=egx))
    bar = 2e-4 if act == torch.bfloat16 else TOL_F32
    assert ey < bar and egx < bar, (ey, egx)
