"""GPU parity of the device-resident attention projections
(qh_attn_qkv_forward_dev, qh_attn_o_forward_dev, qh_attn_o_backward_dev,
qh_attn_qkv_backward_dev): the half of block_forward / block_backward
around the attention (qlora-model/src/llama.rs:426-439, 577-601) with QLoRA
projections, against the oracle's composite of the same steps.  The
attention itself is the caller's; here its outputs and upstream gradients
are seeded random tensors.

Tolerance (fp32, GEMM and row sums in a different order): max |gpu -
oracle| <= 1e-4 * max |oracle| per output tensor.  Forwards are run twice and
must repeat bit for bit.
"""
import numpy as np
import pytest

import oracle as O

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(300)]

torch = pytest.importorskip("torch")

TOL = 1e-4


def _close(got, ref, what):
    got = got.detach().cpu().numpy().ravel()
    ref = np.ravel(ref)
    scale = float(np.max(np.abs(ref)))
    err = float(np.max(np.abs(got.astype(np.float64) - ref)))
    assert err <= TOL * scale, f"{what}: max err {err:.3e} vs scale {scale:.3e}"


# SmolLM-135M: hidden 576, 9 query heads and 3 kv heads of 64 (kv_dim 192)
@pytest.mark.parametrize("seq,adapters", [(2048, (True, True, True, True)),
                                          (4, (True, False, True, False)),
                                          (130, (False, True, True, False))])
def test_attn_projections_parity(ctx, seq, adapters):
    from qlora_hip import device as QD
    print(f"attn projections seq={seq} adapters={adapters}", flush=True)
    h, kv, r, alpha, eps = 576, 192, 8, 16.0, 1e-5
    dev = torch.device("cuda:0")
    g = O.Rng(0xA77E + seq)
    norm = g.uniform(h, 0.5, 1.5)
    ps, Ws, loras = [], [], []
    for out_dim, ad in zip((h, kv, kv, h), adapters):
        w = g.normal(out_dim * h, 0.02)
        W = QD.DeviceWeight.quantize(torch.from_numpy(w).to(dev).view(out_dim, h), ctx=ctx)
        wd = O.dequantize(O.quantize(w))
        if ad:
            a = g.uniform(r * h, -1 / np.sqrt(h), 1 / np.sqrt(h))
            b = g.normal(out_dim * r, 0.01)
            ps.append([wd, a, b, r, alpha])
            loras.append((torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev), r, alpha))
        else:
            ps.append([wd, None, None, 0, 0.0])
            loras.append(None)
        Ws.append(W)
    x = g.normal(seq * h)
    attn = g.normal(seq * h)      # the caller's attention output
    dx_mid = g.normal(seq * h)    # dL/d(x after the attention residual)
    dq, dk, dv = g.normal(seq * h), g.normal(seq * kv), g.normal(seq * kv)

    rq, rk, rv, cache = O.attn_qkv_forward(norm, *ps[:3], x, seq, h, kv, eps)
    r_out = O.attn_o_forward(ps[3], attn, x, seq, h)
    r_dattn, r_go = O.attn_o_backward(ps[3], attn, dx_mid, seq, h)
    r_dx, r_grads = O.attn_qkv_backward(norm, *ps[:3], cache, dq, dk, dv, dx_mid, seq, h, kv,
                                        eps)

    t = lambda a, n: torch.from_numpy(a).to(dev).view(seq, n)  # noqa: E731
    blk = QD.AttnProjections(torch.from_numpy(norm).to(dev), *Ws, loras=loras, eps=eps,
                             ctx=ctx)
    tx = t(x, h)
    c = blk.new_cache(seq)
    q1, k1, v1 = blk.qkv_forward(tx, c)
    q2, k2, v2 = blk.qkv_forward(tx, blk.new_cache(seq))
    torch.cuda.synchronize()
    assert torch.equal(tx, t(x, h)), "qkv_forward changed x"
    assert torch.equal(q1, q2) and torch.equal(k1, k2) and torch.equal(v1, v2)
    _close(q1, rq, "q")
    _close(k1, rk, "k")
    _close(v1, rv, "v")
    _close(c["xn"], cache["xn"], "xn")
    c["attn"].copy_(t(attn, h))
    x1 = blk.o_forward(tx.clone(), c)
    x2 = blk.o_forward(tx.clone(), c)
    torch.cuda.synchronize()
    assert torch.equal(x1, x2)
    _close(x1, r_out, "x_out")
    d_attn, go = blk.o_backward(c, t(dx_mid, h))
    dx, grads = blk.qkv_backward(c, t(dq, h), t(dk, kv), t(dv, kv), t(dx_mid, h))
    torch.cuda.synchronize()
    _close(d_attn, r_dattn, "d_attn")
    _close(dx, r_dx, "dx_in")
    for name, got, want in zip(("q", "k", "v", "o"), grads + [go], r_grads + [r_go]):
        assert (got is None) == (want is None), name
        if got is not None:
            _close(got[0], want[0], f"{name} grad_a")
            _close(got[1], want[1], f"{name} grad_b")


def test_attn_projections_reject_bad_shapes(ctx):
    import ctypes as C
    from qlora_hip import device as QD
    from qlora_hip._lib import QloraError, check
    dev = torch.device("cuda:0")
    h, kv = 64, 32
    mk = lambda n: QD.DeviceWeight.quantize(torch.randn(n, h, device=dev) * 0.02,  # noqa
                                            ctx=ctx)
    norm = torch.ones(h, device=dev)
    bad = QD.AttnProjections(norm, mk(h), mk(kv), mk(16), mk(h), ctx=ctx)
    with pytest.raises(QloraError, match="v weight is 16 x 64 but the block needs 32 x 64"):
        bad.qkv_forward(torch.zeros(2, h, device=dev), bad.new_cache(2))
    blk = QD.AttnProjections(norm, mk(h), mk(kv), mk(kv), mk(h), ctx=ctx)
    cs = blk._cs(blk.new_cache(2))
    dm, dkv = torch.zeros(2, h, device=dev), torch.zeros(2, kv, device=dev)
    with pytest.raises(QloraError, match="must not alias"):
        check(blk.ctx.lib.qh_attn_qkv_backward_dev(
            blk.ctx.h, C.byref(blk.s), C.byref(cs), dm.data_ptr(), dkv.data_ptr(),
            dkv.data_ptr(), dm.data_ptr(), 2, dm.data_ptr(), None, None, None))
