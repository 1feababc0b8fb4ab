"""Shared helpers of the device-path GPU parity tests: seeded layer inputs in
HBM, one forward + backward through ``qh_qlora_forward_dev`` /
``qh_qlora_backward_dev``, and the oracle's answers for it.

Y and dX are compared on sampled rows (every row is an independent
reduction, so the oracle run on those rows alone gives exactly those rows);
T1, grad_A and grad_B are compared in full.  The oracle's GEMMs
(qlora-core/src/lora.rs:129-183 order) are the reference for all of them.
"""
import concurrent.futures as cf

import numpy as np
import torch

import oracle as O
from parity import bf16_round, nerr


def say(*a):
    print(*a, flush=True)


def setup_layer(QD, ctx, N, K, r, M, seed, act=torch.float32):
    """W = 0.02 N, A = U(+-1/sqrt(K)), B = 0.01 N, X = N, dY = N, in that
    order from the reference's generator; bf16 activations are the
    round-to-nearest-even of the same draws."""
    g = O.Rng(seed)
    w = g.normal(N * K, 0.02)
    a = g.uniform(r * K, -1 / np.sqrt(K), 1 / np.sqrt(K))
    b = g.normal(N * r, 0.01)
    x = g.normal(M * K)
    dy = g.normal(M * N)
    if act == torch.bfloat16:
        x, dy = bf16_round(x), bf16_round(dy)
    dev = torch.device("cuda:0")
    W = QD.DeviceWeight.quantize(torch.from_numpy(w).to(dev).view(N, K), ctx=ctx)
    t = lambda v: torch.from_numpy(v).to(dev)  # noqa: E731
    return dict(w=w, a=a, b=b, x=x, dy=dy, W=W, ta=t(a), tb=t(b),
                tx=t(x).to(act), tdy=t(dy).to(act))


def run_layer(QD, ctx, d, N, K, r, M, alpha, rows, wd=None):
    """Forward (with T1 kept) then backward on the device; returns the
    normalised error of y, T1, grad_x, grad_A and grad_B against the
    oracle.  ``d`` holds host copies ``w`` (or a dequantized ``wd``), ``a``,
    ``b``, ``x``, ``dy`` and their device tensors."""
    dev = torch.device("cuda:0")
    lora = QD.lora_struct(d["ta"], d["tb"], r, alpha)
    y = torch.empty(M, N, device=dev)
    t1 = torch.empty(M, r, device=dev)
    gx = torch.empty(M, K, device=dev)
    ga = torch.empty(r, K, device=dev)
    gb = torch.empty(N, r, device=dev)
    QD.forward(d["W"], lora, d["tx"], M, y, t1=t1, ctx=ctx)
    QD.backward(d["W"], lora, d["tx"], d["tdy"], M, gx, ga, gb, t1=t1, ctx=ctx)
    torch.cuda.synchronize()
    if wd is None:
        q = O.quantize(d["w"])
        # the device quantization is bit-exact with the oracle's
        assert np.array_equal(d["W"].codes.cpu().numpy(), q["codes"])
        assert np.array_equal(d["W"].scale_codes.cpu().numpy(), q["scale_codes"])
        wd = O.dequantize(q)
    x, dy = d["x"], d["dy"]
    xs, dys = x.reshape(M, K)[rows].ravel(), dy.reshape(M, N)[rows].ravel()
    s = np.float32(alpha / r)
    dys_full = (dy * s).astype(np.float32)

    # three independent chains of oracle calls (ctypes drops the GIL)
    def rows_fb():
        yo = O.qlora_forward(wd, N, K, d["a"], d["b"], r, alpha, xs, len(rows))
        gxo, _, _ = O.qlora_backward(wd, N, K, d["a"], d["b"], r, alpha, xs, dys, len(rows))
        return yo, gxo

    def t1_gb():
        t1o = O.matmul_trans_b(x, d["a"], M, K, r)
        return t1o, O.matmul_trans_a(dys_full, t1o, M, N, r)

    def ds_ga():
        ds = O.matmul(dys_full, d["b"], M, N, r)
        return ds, O.matmul_trans_a(ds, x, M, r, K)

    with cf.ThreadPoolExecutor(3) as ex:
        f1, f2, f3 = ex.submit(rows_fb), ex.submit(t1_gb), ex.submit(ds_ga)
        (yo, gxo), (t1o, gbo), (ds, gao) = f1.result(), f2.result(), f3.result()
    return dict(
        y=nerr(y.cpu().numpy()[rows].ravel(), yo, K, x, wd),
        t1=nerr(t1.cpu().numpy().ravel(), t1o, K, x, d["a"]),
        gx=nerr(gx.cpu().numpy()[rows].ravel(), gxo, N, dy, wd),
        ga=nerr(ga.cpu().numpy().ravel(), gao, M, ds, x),
        gb=nerr(gb.cpu().numpy().ravel(), gbo, M, dys_full, t1o))
