"""GPU parity of the block glue around the projections (qlora-model/src/
llama.rs): RMSNorm forward/backward, SwiGLU forward/backward and the softmax
cross-entropy, through the C ABI, against the oracle on seeded inputs.

Tolerance (fp32, different summation order and the GPU's expf / logf):
max |gpu - oracle| <= 1e-5 * max |oracle| per output tensor, 1e-5 relative
on the loss.  The cross-entropy takes 1e-4 against the oracle (the bound
for fp32 outputs): the oracle's sequential f32 sum over a 49152-long row is
itself 2.3e-5 off the float64 softmax (1.1e-5 on the loss at 128256), so the
GPU is also held to 1e-5 of the float64 softmax and 1e-6 of the float64
loss.  Every case also runs twice and must repeat bit
for bit.
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TOL = 1e-5
TOL_CE_ORACLE = 1e-4


def _say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def QD(ctx):
    from qlora_hip import device
    return device


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def _close(got, ref, what, tol=TOL):
    got = got.detach().cpu().numpy().ravel() if hasattr(got, "cpu") else np.ravel(got)
    ref = np.ravel(ref)
    assert got.shape == ref.shape, what
    scale = float(np.max(np.abs(ref))) if ref.size else 0.0
    err = float(np.max(np.abs(got.astype(np.float64) - ref))) if ref.size else 0.0
    assert err <= tol * scale, f"{what}: max err {err:.3e} vs scale {scale:.3e}"


def _loss64(logits, targets, seq, vocab):
    from scipy.special import logsumexp
    z = logits.astype(np.float64).reshape(seq, vocab)
    return float(np.mean(logsumexp(z, axis=1) - z[np.arange(seq), targets]))


def _check_loss(got, ref, logits, targets, seq, vocab):
    truth = _loss64(logits, targets, seq, vocab)
    assert abs(got - ref) <= TOL_CE_ORACLE * max(1.0, abs(ref)), (got, ref)
    assert abs(got - truth) <= 1e-6 * max(1.0, abs(truth)), (got, truth)


def _softmax_grad64(logits, targets, seq, vocab):
    from scipy.special import logsumexp
    z = logits.astype(np.float64).reshape(seq, vocab)
    p = np.exp(z - logsumexp(z, axis=1, keepdims=True))
    p[np.arange(seq), targets] -= 1.0
    return (p / seq).ravel()


def _misaligned(t):
    """A copy of t whose data pointer is 4 bytes past a 16-byte boundary."""
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    v = buf[1:].view(t.shape)
    v.copy_(t)
    assert v.data_ptr() % 16 != 0
    return v


RMS_SHAPES = [(2048, 576), (64, 4096), (3, 8192), (5, 13), (7, 1), (1, 260)]


@pytest.mark.parametrize("rows,h", RMS_SHAPES)
def test_rmsnorm_parity(QD, ctx, rows, h):
    _say(f"rmsnorm rows={rows} h={h}")
    g = O.Rng(100 + h)
    x = g.normal(rows * h)
    w = g.uniform(h, 0.5, 1.5)
    eps = 1e-5
    ref = O.rmsnorm(x, w, rows, h, eps)
    dx, dw = _dev(x).view(rows, h), _dev(w)
    y = QD.rmsnorm(dx, dw, eps, ctx=ctx)
    y2 = QD.rmsnorm(dx, dw, eps, ctx=ctx)
    torch.cuda.synchronize()
    _close(y, ref, "y")
    assert torch.equal(y, y2)
    # scalar path (misaligned rows) gives the same result within tolerance
    ym = QD.rmsnorm(_misaligned(dx), dw, eps, ctx=ctx)
    _close(ym, ref, "y misaligned")
    # in place, like rmsnorm_in_place
    xi = dx.clone()
    QD.rmsnorm(xi, dw, eps, out=xi, ctx=ctx)
    assert torch.equal(xi, y)


@pytest.mark.parametrize("rows,h", [(2048, 576), (33, 13), (4, 8192), (130, 4096)])
def test_rmsnorm_backward_parity(QD, ctx, rows, h):
    _say(f"rmsnorm_backward rows={rows} h={h}")
    g = O.Rng(200 + h)
    x = g.normal(rows * h)
    w = g.uniform(h, 0.5, 1.5)
    dy = g.normal(rows * h)
    eps = 1e-5
    rdx, rdw = O.rmsnorm_backward(x, w, dy, rows, h, eps)
    tx, tw, tdy = _dev(x).view(rows, h), _dev(w), _dev(dy).view(rows, h)
    dx, dw = QD.rmsnorm_backward(tx, tw, tdy, eps, ctx=ctx)
    dx2, dw2 = QD.rmsnorm_backward(tx, tw, tdy, eps, ctx=ctx)
    dx3, none = QD.rmsnorm_backward(tx, tw, tdy, eps, want_dw=False, ctx=ctx)
    torch.cuda.synchronize()
    assert none is None
    _close(dx, rdx, "dx")
    _close(dw, rdw, "dw")
    assert torch.equal(dx, dx2) and torch.equal(dw, dw2) and torch.equal(dx, dx3)


def test_rmsnorm_empty_and_host_slices(QD, ctx):
    L = ctx.lib
    h = 12
    w = O.Rng(3).uniform(h, 0.5, 1.5)
    # zero rows: dw is all zeros (llama.rs:609 starts from zeros)
    dw = torch.full((h,), 7.0, device="cuda:0")
    e = torch.empty(0, device="cuda:0")
    QD.check(L.qh_rmsnorm_backward_dev(ctx.h, C.c_void_p(e.data_ptr()), QD._p(_dev(w)),
                                       C.c_void_p(e.data_ptr()), 0, h, 1e-5,
                                       C.c_void_p(e.data_ptr()), QD._p(dw), None))
    torch.cuda.synchronize()
    assert torch.count_nonzero(dw).item() == 0
    # host-slice forms (blocking, staged through the context)
    rows = 9
    g = O.Rng(4)
    x, dy = g.normal(rows * h), g.normal(rows * h)
    y = np.empty(rows * h, np.float32)
    fp = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
    QD.check(L.qh_rmsnorm(ctx.h, fp(x), x.size, fp(w), h, 1e-6, fp(y)))
    _close(y, O.rmsnorm(x, w, rows, h, 1e-6), "host y")
    dx, dwh = np.empty_like(x), np.empty(h, np.float32)
    QD.check(L.qh_rmsnorm_backward(ctx.h, fp(x), x.size, fp(w), h, fp(dy), dy.size, 1e-6,
                                   fp(dx), fp(dwh)))
    rdx, rdw = O.rmsnorm_backward(x, w, dy, rows, h, 1e-6)
    _close(dx, rdx, "host dx")
    _close(dwh, rdw, "host dw")


@pytest.mark.parametrize("n", [2048 * 1536, 4097, 7, 1])
def test_swiglu_parity(QD, ctx, n):
    _say(f"swiglu n={n}")
    g = O.Rng(300 + n)
    gate, up, da = g.normal(n, 3.0), g.normal(n), g.normal(n)
    if n >= 4:
        gate[:4] = [0.0, 88.0, -88.0, -104.0]  # exp overflow / underflow edges
    ref = O.swiglu(gate, up)
    rdg, rdu = O.swiglu_backward(gate, up, da)
    tg, tu, ta = _dev(gate), _dev(up), _dev(da)
    act = QD.swiglu(tg, tu, ctx=ctx)
    act2 = QD.swiglu(tg, tu, ctx=ctx)
    dg, du = QD.swiglu_backward(tg, tu, ta, ctx=ctx)
    torch.cuda.synchronize()
    _close(act, ref, "act")
    assert torch.equal(act, act2)
    _close(dg, rdg, "d_gate")
    _close(du, rdu, "d_up")
    am = QD.swiglu(_misaligned(tg), _misaligned(tu), ctx=ctx)
    dgm, dum = QD.swiglu_backward(_misaligned(tg), _misaligned(tu), _misaligned(ta), ctx=ctx)
    _close(am, ref, "act misaligned")
    _close(dgm, rdg, "d_gate misaligned")
    _close(dum, rdu, "d_up misaligned")


def test_swiglu_host_slices_in_place(QD, ctx):
    L = ctx.lib
    n = 1001
    g = O.Rng(7)
    gate, up, da = g.normal(n), g.normal(n), g.normal(n)
    fp = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
    act = np.empty(n, np.float32)
    QD.check(L.qh_swiglu(ctx.h, fp(gate), n, fp(up), n, fp(act)))
    _close(act, O.swiglu(gate, up), "host act")
    dg, du = np.empty(n, np.float32), np.empty(n, np.float32)
    QD.check(L.qh_swiglu_backward(ctx.h, fp(gate), fp(up), fp(da), n, fp(dg), fp(du)))
    rdg, rdu = O.swiglu_backward(gate, up, da)
    _close(dg, rdg, "host dg")
    _close(du, rdu, "host du")
    # device form writing over its inputs
    tg, tu = _dev(gate), _dev(up)
    QD.check(L.qh_swiglu_backward_dev(ctx.h, QD._p(tg), QD._p(tu), QD._p(_dev(da)), n,
                                      QD._p(tg), QD._p(tu), None))
    torch.cuda.synchronize()
    _close(tg, rdg, "in-place dg")
    _close(tu, rdu, "in-place du")


# rows in registers (49152, 32000, ...), rows past the register cache read
# in a streaming pass (128256; 50001 on the scalar path)
CE_SHAPES = [(64, 49152), (16, 32000), (4, 128256), (3, 50001), (5, 1001), (3, 1), (1, 7),
             (300, 64)]


@pytest.mark.parametrize("seq,vocab", CE_SHAPES)
def test_softmax_ce_parity(QD, ctx, seq, vocab):
    _say(f"softmax_ce seq={seq} vocab={vocab}")
    g = O.Rng(400 + vocab)
    logits = g.normal(seq * vocab, 3.0)
    targets = np.array([(977 * t + 5) % vocab for t in range(seq)], np.uint32)
    targets[0] = vocab - 1
    rloss, rd = O.softmax_cross_entropy(logits, targets, seq, vocab)
    tl = _dev(logits).view(seq, vocab)
    tt = _dev(targets.view(np.int32))
    loss, d = QD.softmax_cross_entropy(tl, tt, ctx=ctx)
    loss2, d2 = QD.softmax_cross_entropy(tl, tt, ctx=ctx)
    torch.cuda.synchronize()
    _check_loss(loss.item(), rloss, logits, targets, seq, vocab)
    _close(d, rd, "dlogits", TOL_CE_ORACLE)
    _close(d, _softmax_grad64(logits, targets, seq, vocab), "dlogits vs float64")
    assert torch.equal(loss, loss2) and torch.equal(d, d2)
    # in place (dlogits over the logits)
    li = tl.clone()
    loss3, _ = QD.softmax_cross_entropy(li, tt, dlogits=li, ctx=ctx)
    torch.cuda.synchronize()
    assert torch.equal(li, d) and torch.equal(loss3, loss)


def test_softmax_ce_edges(QD, ctx):
    L = ctx.lib
    fp = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
    # large logits: the max subtraction keeps exp in range
    seq, vocab = 6, 4099
    g = O.Rng(9)
    logits = g.normal(seq * vocab, 40.0)
    targets = np.array([0, 1, 4098, 17, 2048, 3], np.uint32)
    rloss, rd = O.softmax_cross_entropy(logits, targets, seq, vocab)
    loss = np.zeros(1, np.float32)
    d = np.empty_like(logits)
    QD.check(L.qh_softmax_cross_entropy(ctx.h, fp(logits), logits.size, fp(targets), seq,
                                        vocab, fp(loss), fp(d)))
    _check_loss(float(loss[0]), rloss, logits, targets, seq, vocab)
    _close(d, rd, "host dlogits", TOL_CE_ORACLE)
    _close(d, _softmax_grad64(logits, targets, seq, vocab), "host dlogits vs float64")
    # seq == 0: loss 0 (llama.rs:493)
    e = torch.empty(0, device="cuda:0")
    tloss = torch.full((1,), 5.0, device="cuda:0")
    QD.check(L.qh_softmax_cross_entropy_dev(ctx.h, QD._p(e), QD._p(e), 0, 10, QD._p(tloss),
                                            QD._p(e), None))
    torch.cuda.synchronize()
    assert tloss.item() == 0.0
    # a target past the vocabulary on the device form: NaN loss, no one-hot
    # term, every other row unchanged
    tl = _dev(logits[: 2 * vocab]).view(2, vocab)
    tt = torch.tensor([vocab, 1], dtype=torch.int32, device="cuda:0")
    bl, bd = QD.softmax_cross_entropy(tl, tt, ctx=ctx)
    torch.cuda.synchronize()
    assert np.isnan(bl.item())
    row0 = bd[0].cpu().numpy()
    assert abs(float(row0.sum()) - 1.0 / 2) < 1e-5 and np.all(row0 >= 0)
    _, rd2 = O.softmax_cross_entropy(logits[: 2 * vocab], np.array([0, 1], np.uint32), 2, vocab)
    _close(bd[1], rd2[vocab:], "row with a valid target", TOL_CE_ORACLE)


def test_softmax_ce_masked_logits(QD, ctx):
    """-inf logits (a masked vocabulary), in the register part and in the
    streamed part of a long row: they get zero probability, like exp(-inf)
    in llama.rs:500."""
    seq, vocab = 3, 128256
    g = O.Rng(21)
    logits = g.normal(seq * vocab, 2.0).reshape(seq, vocab)
    logits[0, :60000] = -np.inf        # register part and beyond
    logits[1, 50000:] = -np.inf        # streamed part only
    logits[2, ::3] = -np.inf
    targets = np.array([70000, 7, 1], np.uint32)
    logits = logits.ravel()
    rloss, rd = O.softmax_cross_entropy(logits, targets, seq, vocab)
    loss, d = QD.softmax_cross_entropy(_dev(logits).view(seq, vocab),
                                       _dev(targets.view(np.int32)), ctx=ctx)
    torch.cuda.synchronize()
    _check_loss(loss.item(), rloss, logits, targets, seq, vocab)
    _close(d, rd, "masked dlogits", TOL_CE_ORACLE)
    assert torch.count_nonzero(d[0, :60000]).item() == 0
