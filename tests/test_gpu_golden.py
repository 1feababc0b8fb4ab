"""The HIP library against the committed oracle vectors
(tests/golden/oracle_vectors.npz): quantize, dequantize and three 8-bit Adam
steps bit for bit; the layer's forward and backward and the block glue
within the fp32 bounds of the other parity tests."""
import os

import numpy as np
import pytest

from parity import TOL_F32, nerr

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                    "oracle_vectors.npz")


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


def test_library_matches_golden_vectors(ctx):
    import qlora_hip as QH
    g = np.load(GOLD)
    print("golden vectors", flush=True)
    for dq in (0, 1):
        q = QH.quantize(g["q_small_w"], 3, 67, 64, bool(dq), ctx=ctx)
        assert np.array_equal(q["codes"], g[f"q_small_dq{dq}_codes"])
        if dq:
            assert np.array_equal(q["scale_codes"], g["q_small_dq1_scale_codes"])
            assert np.array_equal(_bits(q["absmax"]), _bits(g["q_small_dq1_absmax"]))
        else:
            assert np.array_equal(_bits(q["scales"]), _bits(g["q_small_dq0_scales"]))
        assert np.array_equal(_bits(QH.dequantize(q, ctx=ctx)), _bits(g[f"q_small_dq{dq}_deq"]))
    q = QH.quantize(g["q_big_w"], 16, 1040, 64, True, ctx=ctx)
    assert np.array_equal(q["codes"], g["q_big_codes"])
    assert np.array_equal(q["scale_codes"], g["q_big_scale_codes"])
    assert np.array_equal(_bits(q["absmax"]), _bits(g["q_big_absmax"]))
    assert np.array_equal(_bits(QH.dequantize(q, ctx=ctx)), _bits(g["q_big_deq"]))

    N, K, r, B = 96, 128, 4, 5
    ql = QH.quantize(g["layer_w"], N, K, 64, True, ctx=ctx)
    wd = QH.dequantize(ql, ctx=ctx)
    y = QH.forward(ql, g["layer_a"], g["layer_b"], r, 8.0, g["layer_x"], B, ctx=ctx)
    assert nerr(y, g["layer_y"], K, g["layer_x"], wd) < TOL_F32
    gx, ga, gb = QH.backward(ql, g["layer_a"], g["layer_b"], r, 8.0, g["layer_x"],
                             g["layer_dy"], B, ctx=ctx)
    assert nerr(gx, g["layer_gx"], N, g["layer_dy"], wd) < TOL_F32
    assert np.max(np.abs(ga - g["layer_ga"])) < 1e-5 and np.max(np.abs(gb - g["layer_gb"])) < 1e-5

    opt = QH.Adam8bit(lr=1e-3, ctx=ctx)
    ps = [g["adam_p0"].copy(), g["adam_p1"].copy()]
    for i in range(3):
        opt.step(ps, [g[f"adam_g0_{i}"], g[f"adam_g1_{i}"]])
    assert np.array_equal(_bits(ps[0]), _bits(g["adam_p0_after"]))
    assert np.array_equal(_bits(ps[1]), _bits(g["adam_p1_after"]))

    import ctypes as C
    L = ctx.lib
    fp = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
    close = lambda a, b: np.max(np.abs(a - b)) <= 1e-5 * np.max(np.abs(b))  # noqa: E731
    x, w, dy = g["rms_x"], g["rms_w"], g["rms_dy"]
    y = np.empty_like(x)
    QH._lib.check(L.qh_rmsnorm(ctx.h, fp(x), x.size, fp(w), w.size, 1e-5, fp(y)))
    assert close(y, g["rms_y"])
    dx, dw = np.empty_like(x), np.empty_like(w)
    QH._lib.check(L.qh_rmsnorm_backward(ctx.h, fp(x), x.size, fp(w), w.size, fp(dy), dy.size,
                                        1e-5, fp(dx), fp(dw)))
    assert close(dx, g["rms_dx"]) and close(dw, g["rms_dw"])
    gate, up, da = g["swi_gate"], g["swi_up"], g["swi_da"]
    act = np.empty_like(gate)
    QH._lib.check(L.qh_swiglu(ctx.h, fp(gate), gate.size, fp(up), up.size, fp(act)))
    assert close(act, g["swi_act"])
    dg, du = np.empty_like(gate), np.empty_like(gate)
    QH._lib.check(L.qh_swiglu_backward(ctx.h, fp(gate), fp(up), fp(da), gate.size, fp(dg),
                                       fp(du)))
    assert close(dg, g["swi_dg"]) and close(du, g["swi_du"])
    lg, tg = g["ce_logits"], g["ce_targets"]
    loss, dl = np.zeros(1, np.float32), np.empty_like(lg)
    QH._lib.check(L.qh_softmax_cross_entropy(ctx.h, fp(lg), lg.size, fp(tg), 4, 50, fp(loss),
                                             fp(dl)))
    assert abs(loss[0] - g["ce_loss"][0]) <= 1e-5 * abs(g["ce_loss"][0]) and close(dl, g["ce_dlogits"])
