"""Pins of the oracle's restatement of the glue around the projections in
qlora-model/src/llama.rs (RMSNorm, SwiGLU, softmax cross-entropy).

Each check is independent of the restated formula: the reference's own
known answer (llama.rs:846-853), float64 closed forms through numpy/scipy,
central finite differences of a float64 forward for every backward, and
invariants (shift invariance, rows of dlogits summing to zero).
"""
import numpy as np
import pytest
from scipy.special import expit, logsumexp

import oracle as O


def test_rmsnorm_known_answer():
    # llama.rs:846-853
    y = O.rmsnorm(np.array([1, 2, 3, 4], np.float32), np.ones(4, np.float32), 1, 4, 0.0)
    rms = np.float32(np.sqrt(np.float32(30.0) / 4))
    assert abs(y[0] - 1.0 / rms) < 1e-6
    assert abs(y[3] - 4.0 / rms) < 1e-6


def _rms64(x, w, rows, h, eps):
    x = x.astype(np.float64).reshape(rows, h)
    return (x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * w.astype(np.float64)).ravel()


@pytest.mark.parametrize("rows,h,eps", [(5, 576, 1e-5), (3, 7, 1e-6), (2, 1, 0.5)])
def test_rmsnorm_closed_form(rows, h, eps):
    g = O.Rng(11)
    x = g.normal(rows * h)
    w = g.uniform(h, 0.5, 1.5)
    y = O.rmsnorm(x, w, rows, h, eps)
    ref = _rms64(x, w, rows, h, eps)
    assert np.max(np.abs(y - ref)) <= 2e-6 * np.max(np.abs(ref))
    # scale invariance of the normalised part (eps = 0)
    y1 = O.rmsnorm(x, w, rows, h, 0.0)
    y2 = O.rmsnorm(x * np.float32(8.0), w, rows, h, 0.0)
    assert np.max(np.abs(y1 - y2)) <= 1e-6 * np.max(np.abs(y1))


def _fd(f, v, eps=1e-4):
    g = np.zeros_like(v)
    for i in range(v.size):
        p, m = v.copy(), v.copy()
        p[i] += eps
        m[i] -= eps
        g[i] = (f(p) - f(m)) / (2 * eps)
    return g


def test_rmsnorm_backward_finite_differences():
    rows, h, eps = 3, 9, 1e-3
    g = O.Rng(12)
    x = g.normal(rows * h)
    w = g.uniform(h, 0.5, 1.5)
    dy = g.normal(rows * h)
    dx, dw = O.rmsnorm_backward(x, w, dy, rows, h, eps)
    x64, w64, dy64 = x.astype(np.float64), w.astype(np.float64), dy.astype(np.float64)
    fdx = _fd(lambda v: float(np.dot(dy64, _rms64(v, w64, rows, h, eps))), x64)
    fdw = _fd(lambda v: float(np.dot(dy64, _rms64(x64, v, rows, h, eps))), w64)
    assert np.max(np.abs(dx - fdx)) < 1e-4 * max(1.0, np.max(np.abs(fdx)))
    assert np.max(np.abs(dw - fdw)) < 1e-4 * max(1.0, np.max(np.abs(fdw)))


def test_silu_closed_forms():
    xs = np.array([-30, -5.5, -1, -1e-3, 0, 1e-3, 0.5, 2, 7, 30], np.float32)
    for x in map(float, xs):
        ref = x * expit(x)
        assert abs(O.silu(x) - ref) <= 1e-6 * max(1.0, abs(ref))
        fd = ((x + 1e-4) * expit(x + 1e-4) - (x - 1e-4) * expit(x - 1e-4)) / 2e-4
        assert abs(O.silu_prime(x) - fd) < 1e-6
    assert O.silu(0.0) == 0.0 and O.silu_prime(0.0) == 0.5


def test_swiglu_and_backward():
    g = O.Rng(13)
    n = 41
    gate, up, da = g.normal(n, 3.0), g.normal(n), g.normal(n)
    act = O.swiglu(gate, up)
    g64, u64 = gate.astype(np.float64), up.astype(np.float64)
    ref = g64 * expit(g64) * u64
    assert np.max(np.abs(act - ref)) <= 2e-6 * np.max(np.abs(ref))
    dg, du = O.swiglu_backward(gate, up, da)
    d64 = da.astype(np.float64)
    fdg = _fd(lambda v: float(np.dot(d64, v * expit(v) * u64)), g64)
    fdu = _fd(lambda v: float(np.dot(d64, g64 * expit(g64) * v)), u64)
    assert np.max(np.abs(dg - fdg)) < 1e-4
    assert np.max(np.abs(du - fdu)) < 1e-4


def _ce64(logits, targets, seq, vocab):
    z = logits.astype(np.float64).reshape(seq, vocab)
    lse = logsumexp(z, axis=1)
    return float(np.mean(lse - z[np.arange(seq), targets]))


@pytest.mark.parametrize("seq,vocab", [(4, 10), (3, 1), (2, 4099)])
def test_softmax_ce_closed_form(seq, vocab):
    g = O.Rng(14)
    logits = g.normal(seq * vocab, 4.0)
    targets = np.array([(7 * t + 3) % vocab for t in range(seq)], np.uint32)
    loss, d = O.softmax_cross_entropy(logits, targets, seq, vocab)
    assert abs(loss - _ce64(logits, targets, seq, vocab)) <= 1e-5 * max(1.0, abs(loss))
    z = logits.astype(np.float64).reshape(seq, vocab)
    p = np.exp(z - logsumexp(z, axis=1, keepdims=True))
    p[np.arange(seq), targets] -= 1.0
    ref = (p / seq).ravel()
    # f32 sums over the vocabulary: relative error grows like n * 2^-24
    assert np.max(np.abs(d - ref)) <= 1e-5 * np.max(np.abs(ref))
    # rows of dlogits sum to zero; a shift of every logit changes nothing
    assert np.max(np.abs(d.reshape(seq, vocab).sum(axis=1))) < 1e-5
    loss2, d2 = O.softmax_cross_entropy(logits + np.float32(3.0), targets, seq, vocab)
    assert abs(loss2 - loss) < 1e-5 and np.max(np.abs(d2 - d)) < 1e-6


def test_softmax_ce_uniform_and_fd():
    loss, d = O.softmax_cross_entropy(np.zeros(2 * 16, np.float32),
                                      np.array([0, 15], np.uint32), 2, 16)
    assert abs(loss - np.log(16)) < 1e-6
    assert abs(d[0] - (1 / 16 - 1) / 2) < 1e-7 and abs(d[1] - 1 / 32) < 1e-7
    g = O.Rng(15)
    seq, vocab = 2, 6
    logits = g.normal(seq * vocab)
    tg = np.array([1, 5], np.uint32)
    _, d = O.softmax_cross_entropy(logits, tg, seq, vocab)
    fd = _fd(lambda v: _ce64(v, tg, seq, vocab), logits.astype(np.float64))
    assert np.max(np.abs(d - fd)) < 1e-6


def _tiny_block(seed, h=8, f=12, r=2, seq=3, adapters=(True, True, True)):
    g = O.Rng(seed)
    norm = g.uniform(h, 0.5, 1.5)

    def proj(out_dim, in_dim, ad):
        q = O.quantize(g.normal(out_dim * in_dim, 0.3))
        wd = O.dequantize(q)
        if not ad:
            return [wd, None, None, 0, 0.0]
        return [wd, g.uniform(r * in_dim, -0.5, 0.5), g.normal(out_dim * r, 0.5), r, 4.0]
    ps = [proj(f, h, adapters[0]), proj(f, h, adapters[1]), proj(h, f, adapters[2])]
    x = g.normal(seq * h)
    dy = g.normal(seq * h)
    return norm, ps, x, dy, seq, h, f


def test_mlp_block_backward_finite_differences():
    # the reference's own check of block_backward is a finite-difference
    # comparison of the adapter gradients (qlora-model/tests/backward.rs:168-195)
    norm, ps, x, dy, seq, h, f = _tiny_block(31)
    eps = 1e-5

    def loss(xv=None, which=None, k=None, val=None):
        pp = [list(p) for p in ps]
        if which is not None:
            arr = pp[which[0]][which[1]].copy()
            arr[k] = val
            pp[which[0]][which[1]] = arr
        out, _ = O.mlp_forward(norm, *pp, x if xv is None else xv, seq, h, f, eps)
        return float(np.dot(out.astype(np.float64), dy.astype(np.float64)))

    _, cache = O.mlp_forward(norm, *ps, x, seq, h, f, eps)
    dx, grads = O.mlp_backward(norm, *ps, cache, dy, seq, h, f, eps)
    d = 1e-2
    for k in range(0, seq * h, 5):
        xp, xm = x.copy(), x.copy()
        xp[k] += d
        xm[k] -= d
        fd = (loss(xp) - loss(xm)) / (2 * d)
        assert abs(dx[k] - fd) < 5e-3 * max(1.0, abs(fd)), (k, dx[k], fd)
    for pi in range(3):
        for slot in (1, 2):  # A, then B
            arr = ps[pi][slot]
            got = grads[pi][slot - 1]
            for k in range(0, arr.size, 7):
                fd = (loss(which=(pi, slot), k=k, val=arr[k] + d)
                      - loss(which=(pi, slot), k=k, val=arr[k] - d)) / (2 * d)
                assert abs(got[k] - fd) < 5e-3 * max(1.0, abs(fd)), (pi, slot, k, got[k], fd)


def test_mlp_block_without_adapters():
    norm, ps, x, dy, seq, h, f = _tiny_block(32, adapters=(False, True, False))
    out, cache = O.mlp_forward(norm, *ps, x, seq, h, f, 1e-5)
    dx, grads = O.mlp_backward(norm, *ps, cache, dy, seq, h, f, 1e-5)
    assert grads[0] is None and grads[2] is None and grads[1] is not None
    assert out.shape == x.shape and dx.shape == x.shape


def _tiny_attn(seed, h=8, kv=4, r=2, seq=3, adapters=(True, True, True, True)):
    g = O.Rng(seed)
    norm = g.uniform(h, 0.5, 1.5)

    def proj(out_dim, in_dim, ad):
        q = O.quantize(g.normal(out_dim * in_dim, 0.3))
        wd = O.dequantize(q)
        if not ad:
            return [wd, None, None, 0, 0.0]
        return [wd, g.uniform(r * in_dim, -0.5, 0.5), g.normal(out_dim * r, 0.5), r, 4.0]
    ps = [proj(h, h, adapters[0]), proj(kv, h, adapters[1]), proj(kv, h, adapters[2]),
          proj(h, h, adapters[3])]
    x = g.normal(seq * h)
    return norm, ps, x, seq, h, kv


def _fd_check(loss, x, got_dx, ps, grads, which_ps, d=1e-2, step_x=3, step_p=5):
    for k in range(0, x.size, step_x):
        xp, xm = x.copy(), x.copy()
        xp[k] += d
        xm[k] -= d
        fd = (loss(xp) - loss(xm)) / (2 * d)
        assert abs(got_dx[k] - fd) < 5e-3 * max(1.0, abs(fd)), (k, got_dx[k], fd)
    for gi, pi in enumerate(which_ps):
        for slot in (1, 2):  # A, then B
            arr = ps[pi][slot]
            got = grads[gi][slot - 1]
            for k in range(0, arr.size, step_p):
                fd = (loss(which=(pi, slot), k=k, val=arr[k] + d)
                      - loss(which=(pi, slot), k=k, val=arr[k] - d)) / (2 * d)
                assert abs(got[k] - fd) < 5e-3 * max(1.0, abs(fd)), (pi, slot, k, got[k], fd)


def _with(ps, which, k, val):
    pp = [list(p) for p in ps]
    if which is not None:
        arr = pp[which[0]][which[1]].copy()
        arr[k] = val
        pp[which[0]][which[1]] = arr
    return pp


def test_attn_qkv_backward_finite_differences():
    # L = <q, Gq> + <k, Gk> + <v, Gv> + <x, Gmid>: dL/dx is the block's dx_in
    # for upstream gradients dq = Gq, dk = Gk, dv = Gv and dx_mid = Gmid (the
    # residual's straight path), as block_backward composes them
    # (llama.rs:580-601; its own check: qlora-model/tests/backward.rs:168-195)
    norm, ps, x, seq, h, kv = _tiny_attn(41)
    eps = 1e-5
    g = O.Rng(42)
    gq, gk, gv, gmid = g.normal(seq * h), g.normal(seq * kv), g.normal(seq * kv), g.normal(seq * h)

    def loss(xv=None, which=None, k=None, val=None):
        pp = _with(ps, which, k, val)
        xv = x if xv is None else xv
        q, kk, v, _ = O.attn_qkv_forward(norm, pp[0], pp[1], pp[2], xv, seq, h, kv, eps)
        f64 = np.float64
        return float(np.dot(q.astype(f64), gq) + np.dot(kk.astype(f64), gk)
                     + np.dot(v.astype(f64), gv) + np.dot(xv.astype(f64), gmid))

    _, _, _, cache = O.attn_qkv_forward(norm, ps[0], ps[1], ps[2], x, seq, h, kv, eps)
    dx, grads = O.attn_qkv_backward(norm, ps[0], ps[1], ps[2], cache, gq, gk, gv, gmid,
                                    seq, h, kv, eps)
    _fd_check(loss, x, dx, ps, grads, (0, 1, 2))


def test_attn_o_backward_finite_differences():
    # L = <x + o(attn), G>: dL/dattn and o's adapter gradients (llama.rs:436-439, 577)
    norm, ps, x, seq, h, kv = _tiny_attn(43)
    g = O.Rng(44)
    attn, gout = g.normal(seq * h), g.normal(seq * h)

    def loss(av=None, which=None, k=None, val=None):
        pp = _with(ps, which, k, val)
        out = O.attn_o_forward(pp[3], attn if av is None else av, x, seq, h)
        return float(np.dot(out.astype(np.float64), gout))

    out = O.attn_o_forward(ps[3], attn, x, seq, h)
    # the straight path: x_out - x is exactly o(attn)
    np.testing.assert_array_equal(
        out, (x + O.qlora_forward(ps[3][0], h, h, ps[3][1], ps[3][2], ps[3][3], ps[3][4],
                                  attn, seq)).astype(np.float32))
    d_attn, go = O.attn_o_backward(ps[3], attn, gout, seq, h)
    _fd_check(loss, attn, d_attn, ps, [go], (3,))


def test_attn_half_without_adapters():
    norm, ps, x, seq, h, kv = _tiny_attn(45, adapters=(True, False, True, False))
    q, k, v, cache = O.attn_qkv_forward(norm, *ps[:3], x, seq, h, kv, 1e-5)
    assert q.shape == (seq * h,) and k.shape == (seq * kv,) and v.shape == (seq * kv,)
    dx, grads = O.attn_qkv_backward(norm, *ps[:3], cache, q, k, v, x, seq, h, kv, 1e-5)
    assert grads[1] is None and grads[0] is not None and grads[2] is not None
    d_attn, go = O.attn_o_backward(ps[3], q, x, seq, h)
    assert go is None and d_attn.shape == (seq * h,)
