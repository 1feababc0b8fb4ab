"""Writes tests/golden/oracle_vectors.npz: small input/output vectors of the
CPU oracle (the restatement of qlora-core and of qlora-model's block glue),
from the reference's own test generator (xorshift64* + Box-Muller,
qlora-core/tests/quant.rs:6-24) with the reference's seed
0x1234_5678_9ABC_DEF0 (tests/quant.rs:40) xor a case index.

The reference itself (Rust) cannot run here; these vectors pin the oracle
against drift (tests/test_golden.py re-derives every one bit for bit) and
give the GPU library fixed cases to match (tests/test_gpu_golden.py).

Usage: python tests/golden/make_golden.py   (rewrites the .npz)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as O  # noqa: E402

SEED = 0x123456789ABCDEF0
OUT = os.path.join(HERE, "oracle_vectors.npz")


def build() -> dict:
    v = {}
    # quantize / dequantize: a ragged last block (3 x 67), fp32 and DQ stores,
    # and a 16 x 1040 tensor whose 260 blocks span 2 double-quant groups
    g = O.Rng(SEED ^ 1)
    w = g.normal(3 * 67, 0.02)
    w[64:128] = 0.0                    # an all-zero block (code 7, scale 0)
    w[128:131] = [0.5, -0.5, 0.5]      # equal magnitudes
    v["q_small_w"] = w
    for dq in (0, 1):
        q = O.quantize(w, 64, bool(dq))
        v[f"q_small_dq{dq}_codes"] = q["codes"]
        if dq:
            v["q_small_dq1_scale_codes"] = q["scale_codes"]
            v["q_small_dq1_absmax"] = q["absmax"]
        else:
            v["q_small_dq0_scales"] = q["scales"]
        v[f"q_small_dq{dq}_deq"] = O.dequantize(q)
    w2 = O.Rng(SEED ^ 2).normal(16 * 1040, 0.02)
    q2 = O.quantize(w2, 64, True)
    v["q_big_w"] = w2
    v["q_big_codes"], v["q_big_scale_codes"] = q2["codes"], q2["scale_codes"]
    v["q_big_absmax"], v["q_big_deq"] = q2["absmax"], O.dequantize(q2)
    # one QloraLinear: 96 x 128 (out x in), r = 4, alpha = 8, batch 5
    g = O.Rng(SEED ^ 3)
    N, K, r, B = 96, 128, 4, 5
    wl = g.normal(N * K, 0.02)
    a = g.uniform(r * K, -1 / np.sqrt(K), 1 / np.sqrt(K))
    b = g.normal(N * r, 0.01)
    x = g.normal(B * K)
    dy = g.normal(B * N)
    wd = O.dequantize(O.quantize(wl))
    v.update(layer_w=wl, layer_a=a, layer_b=b, layer_x=x, layer_dy=dy,
             layer_y=O.qlora_forward(wd, N, K, a, b, r, 8.0, x, B))
    gx, ga, gb = O.qlora_backward(wd, N, K, a, b, r, 8.0, x, dy, B)
    v.update(layer_gx=gx, layer_ga=ga, layer_gb=gb)
    # three 8-bit Adam steps over two tensors (one with a ragged 256-block)
    g = O.Rng(SEED ^ 4)
    p0, p1 = g.normal(600, 0.1), g.normal(256, 0.1)
    grads = [(g.normal(600, 0.01), g.normal(256, 0.01)) for _ in range(3)]
    v["adam_p0"], v["adam_p1"] = p0.copy(), p1.copy()
    for i, (g0, g1) in enumerate(grads):
        v[f"adam_g0_{i}"], v[f"adam_g1_{i}"] = g0, g1
    opt = O.Adam8bit(lr=1e-3)
    ps = [p0.copy(), p1.copy()]
    for g0, g1 in grads:
        opt.step(ps, [g0, g1])
    v["adam_p0_after"], v["adam_p1_after"] = ps[0], ps[1]
    # the block glue (qlora-model llama.rs)
    g = O.Rng(SEED ^ 5)
    rows, h = 3, 20
    xg, wg, dyg = g.normal(rows * h), g.uniform(h, 0.5, 1.5), g.normal(rows * h)
    v.update(rms_x=xg, rms_w=wg, rms_dy=dyg, rms_y=O.rmsnorm(xg, wg, rows, h, 1e-5))
    v["rms_dx"], v["rms_dw"] = O.rmsnorm_backward(xg, wg, dyg, rows, h, 1e-5)
    gate, up, da = g.normal(37, 3.0), g.normal(37), g.normal(37)
    v.update(swi_gate=gate, swi_up=up, swi_da=da, swi_act=O.swiglu(gate, up))
    v["swi_dg"], v["swi_du"] = O.swiglu_backward(gate, up, da)
    lg = g.normal(4 * 50, 4.0)
    tg = np.array([0, 49, 7, 23], np.uint32)
    loss, dl = O.softmax_cross_entropy(lg, tg, 4, 50)
    v.update(ce_logits=lg, ce_targets=tg, ce_loss=np.array([loss], np.float32), ce_dlogits=dl)
    return v


if __name__ == "__main__":
    np.savez(OUT, **build())
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")
