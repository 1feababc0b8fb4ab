"""The C-ABI library loads without a GPU, exports every symbol that
include/qlora_hip.h declares, and rejects bad arguments exactly as the
reference does (messages and status kinds) before touching a device.
No compute runs here."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import qlora_hip
from qlora_hip import _lib
from qlora_hip._lib import AdamConfig, Lora, QWeight

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    src = open(os.path.join(ROOT, "include", "qlora_hip.h")).read()
    return sorted(set(re.findall(r"QH_API\s+[\w\s\*]+?\b(qh_\w+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    L = qlora_hip.load()
    names = declared_functions()
    assert len(names) >= 25
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(_lib.EXPORTED)
    assert L.qh_abi_version() == 1


def test_ctx_create_reports_no_device_without_gpu():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is visible")
    with pytest.raises(qlora_hip.NoDevice):
        qlora_hip.Context()


def test_layout_helpers():
    L = qlora_hip.load()
    assert L.qh_codes_len(2, 5) == 5 and L.qh_codes_len(1, 7) == 4
    assert L.qh_num_blocks(10, 10, 64) == 2
    assert L.qh_num_absmax(256, 256, 64) == 4
    # quant.rs:229-235 / tests/quant.rs:115-134: 1024 blocks
    q = QWeight(rows=256, cols=256, block_size=64, scale_kind=0)
    plain = L.qh_storage_bytes(C.byref(q))
    q.scale_kind = 1
    assert plain - L.qh_storage_bytes(C.byref(q)) == 4096 - 1040


def _err(L):
    return L.qh_last_error().decode()


def test_quantize_validation_messages():
    L = qlora_hip.load()
    w = np.ones(2, np.float32)
    p = w.ctypes.data_as(C.c_void_p)
    # quant.rs:72-79 then :114-119
    assert L.qh_quantize_nf4(None, p, 2, 1, 2, 0, 1, None, None, None, None) == 2
    assert _err(L) == "invalid config: block_size must be > 0"
    assert L.qh_quantize_nf4(None, p, 2, 1, 1, 64, 1, None, None, None, None) == 1
    assert _err(L) == "shape mismatch: weights.len() = 2 but rows*cols = 1"
    assert L.qh_quantize_nf4(None, p, 2, 1 << 40, 1 << 40, 64, 1, None, None,
                             None, None) == 2
    assert _err(L) == "invalid config: rows*cols overflow"


def test_matmul_validation_order():
    L = qlora_hip.load()
    a = np.ones(6, np.float32).ctypes.data_as(C.c_void_p)
    # kernels.rs:151-153: m == 0 returns an empty result before any check
    assert L.qh_matmul(None, a, 99, a, 99, 0, 3, 2, None) == 0
    assert L.qh_matmul(None, a, 6, a, 5, 2, 3, 2, None) == 1
    assert _err(L) == ("shape mismatch: gpu_matmul: a.len() = 6, b.len() = 5, "
                       "expected 2*3 and 3*2")
    assert L.qh_matmul_trans_b(None, a, 6, a, 5, 2, 3, 2, None) == 1
    assert _err(L) == ("shape mismatch: gpu_matmul_trans_b: a.len() = 6, "
                       "b.len() = 5, expected 2*3 and 2*3")
    # kernels.rs:231: trans_a checks k == 0 || n == 0 first
    assert L.qh_matmul_trans_a(None, a, 99, a, 99, 5, 0, 2, None) == 0
    assert L.qh_matmul_trans_a(None, a, 6, a, 5, 2, 3, 2, None) == 1
    assert _err(L) == ("shape mismatch: gpu_matmul_trans_a: a.len() = 6, "
                       "b.len() = 5, expected 2*3 and 2*2")


def test_layer_validation_messages():
    L = qlora_hip.load()
    codes = np.zeros(16, np.uint8)
    sc = np.ones(1, np.float32)
    w = QWeight(rows=4, cols=8, block_size=64, codes=codes.ctypes.data,
                scale_kind=0, scales=sc.ctypes.data)
    x = np.ones(16, np.float32)
    xp = x.ctypes.data_as(C.c_void_p)
    # lora.rs:36-52
    bad = Lora(a=x.ctypes.data, a_len=16, b=x.ctypes.data, b_len=8, r=0, alpha=1)
    assert L.qh_qlora_forward(None, C.byref(w), C.byref(bad), xp, 8, 1, None) == 2
    assert _err(L) == "invalid config: rank r must be > 0"
    bad.r = 2
    bad.a_len = 15
    assert L.qh_qlora_forward(None, C.byref(w), C.byref(bad), xp, 8, 1, None) == 1
    assert _err(L) == "shape mismatch: a.len() = 15 but r*in_dim = 16"
    bad.a_len, bad.b_len = 16, 7
    assert L.qh_qlora_forward(None, C.byref(w), C.byref(bad), xp, 8, 1, None) == 1
    assert _err(L) == "shape mismatch: b.len() = 7 but out_dim*r = 8"
    # qlora.rs:89-94 and :119-132
    assert L.qh_qlora_forward(None, C.byref(w), None, xp, 7, 1, None) == 1
    assert _err(L) == "shape mismatch: x.len() = 7 but batch*in_dim = 8"
    assert L.qh_qlora_backward(None, C.byref(w), None, xp, 8, xp, 3, 1, None, None,
                               None) == 1
    assert _err(L) == "shape mismatch: dy.len() = 3 but batch*out_dim = 4"
    w.block_size = 0
    assert L.qh_qlora_forward(None, C.byref(w), None, xp, 8, 1, None) == 2
    assert _err(L) == "invalid config: block_size must be > 0"
    # valid arguments without a context: a GPU error, never a CPU fallback
    w.block_size = 64
    assert L.qh_qlora_forward(None, C.byref(w), None, xp, 8, 1, None) == 3


def test_device_entry_points_reject_null_buffers():
    """The *_dev entry points refuse a NULL buffer that the call would read
    or write, before any launch (no device needed)."""
    L = qlora_hip.load()
    codes = np.zeros(16, np.uint8)
    sc = np.ones(1, np.float32)
    w = QWeight(rows=4, cols=8, block_size=64, codes=codes.ctypes.data,
                scale_kind=0, scales=sc.ctypes.data)
    buf = np.ones(64, np.float32)
    bp = C.c_void_p(buf.ctypes.data)
    lora = Lora(a=buf.ctypes.data, a_len=16, b=buf.ctypes.data, b_len=8, r=2, alpha=1)
    fwd, bwd = L.qh_qlora_forward_dev, L.qh_qlora_backward_dev
    assert fwd(None, C.byref(w), None, None, 0, 2, bp, None, None) == 1
    assert _err(L) == "shape mismatch: x is NULL but holds 16 elements"
    assert fwd(None, C.byref(w), None, bp, 0, 2, None, None, None) == 1
    assert _err(L) == "shape mismatch: y is NULL but holds 8 elements"
    # batch 0: nothing is read or written, so NULL buffers are fine
    assert fwd(None, C.byref(w), None, None, 0, 0, None, None, None) == 3
    # an adapter needs both gradient buffers
    assert bwd(None, C.byref(w), C.byref(lora), bp, bp, 0, 2, None, bp, None, bp,
               None) == 1
    assert _err(L) == "shape mismatch: grad_a is NULL but holds 16 elements"
    assert bwd(None, C.byref(w), C.byref(lora), bp, bp, 0, 2, None, bp, bp, None,
               None) == 1
    assert _err(L) == "shape mismatch: grad_b is NULL but holds 8 elements"
    assert bwd(None, C.byref(w), C.byref(lora), bp, bp, 0, 2, None, None, bp, bp,
               None) == 1
    assert _err(L) == "shape mismatch: grad_x is NULL but holds 16 elements"
    assert bwd(None, C.byref(w), None, bp, None, 0, 2, None, bp, None, None, None) == 1
    assert _err(L) == "shape mismatch: dy is NULL but holds 8 elements"
    # without an adapter the backward does not read x
    assert bwd(None, C.byref(w), None, None, bp, 0, 2, None, bp, None, None, None) == 3
    lora.a = 0
    assert fwd(None, C.byref(w), C.byref(lora), bp, 0, 2, bp, None, None) == 1
    assert _err(L) == "shape mismatch: the adapter's A or B is NULL"


def test_adam_config_validation():
    L = qlora_hip.load()
    cfg = AdamConfig()
    L.qh_adam_config_default(C.byref(cfg))
    # optim.rs:49-60
    assert (cfg.lr, cfg.block_size, cfg.max_resident_pages) == (
        pytest.approx(1e-3), 256, (1 << 64) - 1)
    assert cfg.beta1 == pytest.approx(0.9) and cfg.beta2 == pytest.approx(0.999)
    h = C.c_void_p()
    for field, val, msg in (
            ("lr", -0.1, "lr must be positive and finite"),
            ("lr", float("inf"), "lr must be positive and finite"),
            ("beta1", 1.0, "betas must be in (0, 1)"),
            ("beta2", -0.5, "betas must be in (0, 1)"),
            ("block_size", 0, "block_size and max_resident_pages must be > 0"),
            ("max_resident_pages", 0, "block_size and max_resident_pages must be > 0")):
        c2 = AdamConfig()
        L.qh_adam_config_default(C.byref(c2))
        setattr(c2, field, val)
        assert L.qh_adam8bit_create(None, C.byref(c2), C.byref(h)) == 2
        assert _err(L) == "invalid config: " + msg
    # beta = 0 is accepted by the reference (optim.rs:69: 0.0..1.0)
    c3 = AdamConfig()
    L.qh_adam_config_default(C.byref(c3))
    c3.beta1 = 0.0
    assert L.qh_adam8bit_create(None, C.byref(c3), C.byref(h)) == 3  # no ctx


def test_python_surface_validation():
    # qlora-python/src/lib.rs:144-174 messages, raised before any GPU work
    from qlora_hip.api import QuantizedWeight, _rebuild
    q = dict(rows=4, cols=8, block_size=64, n=32, codes=np.zeros(16, np.uint8),
             scales=np.ones(1, np.float32))
    wq = QuantizedWeight(q, False)
    with pytest.raises(ValueError, match="must be given together"):
        _rebuild(wq, [0.0] * 16, None, None)
    with pytest.raises(ValueError, match="multiple of in_dim"):
        _rebuild(wq, [0.0] * 15, [0.0] * 8, None)
    with pytest.raises(ValueError, match="out_dim \\* rank"):
        _rebuild(wq, [0.0] * 16, [0.0] * 7, None)
    a, b, r, alpha = _rebuild(wq, [0.0] * 16, [0.0] * 8, None)
    assert r == 2 and alpha == 2.0  # lora_alpha defaults to r (lib.rs:198)
    assert _rebuild(wq, None, None, None)[2] == 0
    q["codes"] = np.zeros(15, np.uint8)
    with pytest.raises(ValueError, match="codes length"):
        _rebuild(wq, None, None, None)


def test_block_glue_validation_messages():
    L = qlora_hip.load()
    x = np.ones(12, np.float32).ctypes.data_as(C.c_void_p)
    # h == 0 has no row (llama.rs:732 chunks of w.len() would panic)
    assert L.qh_rmsnorm(None, x, 12, x, 0, 1e-5, x) == 1
    assert _err(L) == "shape mismatch: hidden size (w.len()) is 0"
    assert L.qh_rmsnorm(None, x, 12, x, 5, 1e-5, x) == 1
    assert _err(L) == "shape mismatch: x.len() = 12 is not a multiple of the hidden size 5"
    assert L.qh_rmsnorm_backward(None, x, 12, x, 4, x, 8, 1e-5, x, None) == 1
    assert _err(L) == "shape mismatch: dy.len() = 8 but x.len() = 12"
    assert L.qh_rmsnorm_dev(None, x, x, 3, 0, 1e-5, x, None) == 1
    assert L.qh_rmsnorm_backward_dev(None, x, x, x, 3, 4, 1e-5, x, x, None) == 2
    assert _err(L) == "invalid config: dx may alias dy only when dw is not requested"
    assert L.qh_swiglu(None, x, 12, x, 11, x) == 1
    assert _err(L) == "shape mismatch: gate.len() = 12 but up.len() = 11"
    # llama.rs:507 indexes row[targets[t]]: a target >= vocab is rejected
    t = np.array([0, 3], np.uint32)
    tp = t.ctypes.data_as(C.c_void_p)
    assert L.qh_softmax_cross_entropy(None, x, 6, tp, 2, 3, None, x) == 1
    assert _err(L) == "shape mismatch: target 3 at position 1 is out of range for vocab 3"
    assert L.qh_softmax_cross_entropy(None, x, 5, tp, 2, 3, None, x) == 1
    assert _err(L) == "shape mismatch: logits.len() = 5 but seq*vocab = 6"
    assert L.qh_softmax_cross_entropy_dev(None, x, tp, 2, 0, None, x, None) == 1
    assert _err(L) == "shape mismatch: vocab is 0"
    # valid arguments reach the context check
    assert L.qh_swiglu_backward(None, x, x, x, 4, x, x) == 3
    assert _err(L) == "gpu error: context is NULL"


def test_weight_upload_validation():
    L = qlora_hip.load()
    q = QWeight()
    q.rows, q.cols, q.block_size, q.scale_kind = 2, 64, 64, 0
    h = C.c_void_p(123)
    assert L.qh_weight_upload(None, C.byref(q), None) == 1
    q.block_size = 0
    assert L.qh_weight_upload(None, C.byref(q), C.byref(h)) == 2
    assert h.value is None
    q.block_size = 64
    assert L.qh_weight_upload(None, C.byref(q), C.byref(h)) == 1  # NULL parts
    w = np.zeros(128, np.float32)
    q.codes = w.ctypes.data
    q.scales = w.ctypes.data
    assert L.qh_weight_upload(None, C.byref(q), C.byref(h)) == 3
    assert L.qh_last_error().decode() == "gpu error: context is NULL"
    L.qh_dweight_destroy(None)


def test_noalloc_backward_checks_before_any_launch():
    """The allocation-free backward validates like qh_qlora_backward_dev and
    refuses a call whose scratch exceeds its fixed region, with no device."""
    L = qlora_hip.load()
    codes = np.zeros(64 * 64 // 2, np.uint8)
    sc = np.ones(64, np.float32)
    w = QWeight(rows=64, cols=64, block_size=64, codes=codes.ctypes.data,
                scale_kind=0, scales=sc.ctypes.data)
    buf = np.ones(64 * 64, np.float32)
    bp = C.c_void_p(buf.ctypes.data)
    lora = Lora(a=buf.ctypes.data, a_len=64 * 64, b=buf.ctypes.data, b_len=64 * 64, r=64,
                alpha=1)
    f = L.qh_qlora_backward_dev_noalloc
    assert f(None, C.byref(w), C.byref(lora), bp, bp, 0, 8, None, bp, None, bp, None) == 1
    assert _err(L) == "shape mismatch: grad_a is NULL but holds 4096 elements"
    # 300000 tokens at r = 64: T1 and Ds (2 x 76.8 MB) plus the split
    # reduction partials of grad_A and grad_B on the dense bf16 kernel
    # (2 x 16 splits x 64 x 64 floats)
    assert f(None, C.byref(w), C.byref(lora), bp, bp, 0, 300000, None, bp, bp, bp,
             None) == 2
    assert _err(L) == ("invalid config: the call needs 154124288 bytes of scratch but the "
                       f"allocation-free backward has {_lib.QH_NOALLOC_SCRATCH_BYTES}")
    # within the region: reaches the context check (a GPU error without one)
    assert f(None, C.byref(w), C.byref(lora), bp, bp, 0, 8, None, bp, bp, bp, None) == 3
