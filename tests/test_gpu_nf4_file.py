"""Packed NF4 files into HBM: a weight quantized on the GPU, written with
save_nf4 and loaded with qlora_hip.device.load_nf4 (pinned image, DMA into
HBM, no fp32 and no quantize on the way) holds the same bits, dequantizes to
the oracle's values and gives the same forward, bit for bit."""
import os
import tempfile

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.mark.parametrize("dq", [True, False])
def test_file_into_hbm(ctx, dq):
    import qlora_hip as QH
    from qlora_hip import device as QD
    print(f"nf4 file dq={dq}", flush=True)
    N, K, r = 4096, 4096, 16
    g = O.Rng(77)
    w = g.normal(N * K, 0.02)
    a = g.uniform(r * K, -1 / 64, 1 / 64)
    b = g.normal(N * r, 0.01)
    x = g.normal(3 * K)
    dev = torch.device("cuda:0")
    W = QD.DeviceWeight.quantize(torch.from_numpy(w).to(dev).view(N, K), double_quant=dq,
                                 ctx=ctx)
    host = dict(rows=N, cols=K, block_size=64, n=N * K, codes=W.codes.cpu().numpy())
    if dq:
        host.update(scale_codes=W.scale_codes.cpu().numpy(), absmax=W.absmax.cpu().numpy())
    else:
        host.update(scales=W.scales.cpu().numpy())
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "w.safetensors")
        QH.save_nf4(p, {"model.layers.0.mlp.up_proj": host})
        loaded = QD.load_nf4(p, ctx=ctx)
    L = loaded["model.layers.0.mlp.up_proj"]
    assert (L.rows, L.cols, L.block_size) == (N, K, 64)
    for part in ("codes", "scales", "scale_codes", "absmax"):
        t0, t1 = getattr(W, part), getattr(L, part)
        assert (t0 is None) == (t1 is None), part
        if t0 is not None:
            assert torch.equal(t0, t1), part
    ref = O.dequantize(O.quantize(w, 64, dq))
    got = L.dequantize(ctx=ctx).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    ta, tb = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    lora = QD.lora_struct(ta, tb, r, 32.0)
    tx = torch.from_numpy(x).to(dev).view(3, K)
    y0, y1 = torch.empty(3, N, device=dev), torch.empty(3, N, device=dev)
    QD.forward(W, lora, tx, 3, y0, ctx=ctx)
    QD.forward(L, lora, tx, 3, y1, ctx=ctx)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)
