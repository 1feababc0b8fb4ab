"""Host-side mirror of the reference's Python module ``qlora_wgpu``
(qlora-python/src/lib.rs:24-310) over the C ABI, plus numpy-level helpers.

Names, signatures, defaults and error behaviour follow the reference:
invalid arguments raise ``ValueError`` carrying the ``QloraError`` text.
Unlike the reference, there is no CPU path: every call runs the gfx950
kernels (``use_gpu`` is accepted for signature compatibility only).
"""
from __future__ import annotations

import ctypes as C
from typing import Optional, Sequence

import numpy as np

from . import _lib
from ._lib import (AdamConfig, AdamStats, Lora, QWeight, QH_SCALES_DQ_INT8,
                   QH_SCALES_F32, check, default_context)

DOUBLE_QUANT_BLOCK = 256


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32).ravel())


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _ctx(ctx):
    return (ctx or default_context())


# ---- quantized weights ------------------------------------------------------
def quantize(w, rows: int, cols: int, block_size: int = 64,
             double_quant: bool = True, ctx=None) -> dict:
    """GPU ``QuantizedTensor::quantize`` (quant.rs:104-154).  Returns
    ``dict(rows, cols, block_size, n, codes, scales | scale_codes + absmax)``
    with numpy arrays in the reference's storage layout."""
    c = _ctx(ctx)
    w = _f32(w)
    L = c.lib
    n = rows * cols
    nb = -(-n // block_size) if block_size else 0
    codes = np.zeros((n + 1) // 2, np.uint8)
    out = dict(rows=rows, cols=cols, block_size=block_size, n=n, codes=codes)
    if double_quant:
        sc = np.zeros(nb, np.uint8)
        am = np.zeros(-(-nb // DOUBLE_QUANT_BLOCK), np.float32)
        check(L.qh_quantize_nf4(c.h, _ptr(w), w.size, rows, cols, block_size, 1,
                                _ptr(codes), None, _ptr(sc), _ptr(am)))
        out.update(scale_codes=sc, absmax=am)
    else:
        sf = np.zeros(nb, np.float32)
        check(L.qh_quantize_nf4(c.h, _ptr(w), w.size, rows, cols, block_size, 0,
                                _ptr(codes), _ptr(sf), None, None))
        out.update(scales=sf)
    return out


def qweight_struct(q: dict) -> QWeight:
    """``qh_qweight`` over the host arrays of ``q`` (kept alive by ``q``)."""
    s = QWeight()
    s.rows, s.cols, s.block_size = q["rows"], q["cols"], q["block_size"]
    s.codes = _ptr(q["codes"])
    if "scales" in q:
        s.scale_kind = QH_SCALES_F32
        s.scales = _ptr(q["scales"])
    else:
        s.scale_kind = QH_SCALES_DQ_INT8
        s.scale_codes = _ptr(q["scale_codes"])
        s.absmax = _ptr(q["absmax"])
    return s


def block_scales(q: dict, ctx=None) -> np.ndarray:
    """``QuantizedTensor::block_scales`` (quant.rs:212-221) on the GPU."""
    c = _ctx(ctx)
    nb = -(-q["n"] // q["block_size"])
    out = np.zeros(nb, np.float32)
    s = qweight_struct(q)
    check(c.lib.qh_block_scales(c.h, C.byref(s), _ptr(out)))
    return out


def dequantize(q: dict, ctx=None) -> np.ndarray:
    """``gpu_dequantize`` (qlora-wgpu/src/kernels.rs:44-103)."""
    c = _ctx(ctx)
    out = np.zeros(q["n"], np.float32)
    s = qweight_struct(q)
    check(c.lib.qh_dequantize(c.h, C.byref(s), _ptr(out)))
    return out


def storage_bytes(q: dict) -> int:
    s = qweight_struct(q)
    return int(_lib.load().qh_storage_bytes(C.byref(s)))


# ---- GEMMs ------------------------------------------------------------------
def _mm(fn: str, a, b, m, k, n, out_len, ctx=None):
    c = _ctx(ctx)
    a, b = _f32(a), _f32(b)
    out = np.zeros(out_len, np.float32)
    check(getattr(c.lib, fn)(c.h, _ptr(a), a.size, _ptr(b), b.size, m, k, n,
                             _ptr(out)))
    return out


def matmul(a, b, m, k, n, ctx=None):
    """``gpu_matmul`` (kernels.rs:140-176): C(m,n) = A(m,k) B(k,n)."""
    return _mm("qh_matmul", a, b, m, k, n, m * n if m and n else 0, ctx)


def matmul_trans_a(a, b, m, k, n, ctx=None):
    """``gpu_matmul_trans_a`` (kernels.rs:220-257): C(k,n) = A(m,k)^T B(m,n)."""
    return _mm("qh_matmul_trans_a", a, b, m, k, n, k * n if k and n else 0, ctx)


def matmul_trans_b(a, b, m, k, n, ctx=None):
    """``gpu_matmul_trans_b`` (kernels.rs:180-216): C(m,n) = A(m,k) B(n,k)^T."""
    return _mm("qh_matmul_trans_b", a, b, m, k, n, m * n if m and n else 0, ctx)


# ---- the layer ---------------------------------------------------------------
def _lora_struct(a, b, r, alpha):
    if a is None:
        return None, None
    s = Lora()
    s.a, s.a_len = _ptr(a), a.size
    s.b, s.b_len = _ptr(b), b.size
    s.r, s.alpha = r, alpha
    return s, C.byref(s)


def forward(q: dict, a, b, r: int, alpha: float, x, batch: int, ctx=None):
    """``gpu_qlora_forward`` (kernels.rs:262-296).  ``a``/``b`` None = no
    adapter."""
    c = _ctx(ctx)
    x = _f32(x)
    a = None if a is None else _f32(a)
    b = None if b is None else _f32(b)
    y = np.zeros(batch * q["rows"], np.float32)
    s = qweight_struct(q)
    ls, lp = _lora_struct(a, b, r, alpha)
    check(c.lib.qh_qlora_forward(c.h, C.byref(s), lp, _ptr(x), x.size, batch,
                                 _ptr(y)))
    return y


def backward(q: dict, a, b, r: int, alpha: float, x, dy, batch: int, ctx=None):
    """``gpu_qlora_backward`` (kernels.rs:301-353).  Returns
    ``(grad_x, grad_a, grad_b)``; grads are None without an adapter."""
    c = _ctx(ctx)
    x, dy = _f32(x), _f32(dy)
    a = None if a is None else _f32(a)
    b = None if b is None else _f32(b)
    gx = np.zeros(batch * q["cols"], np.float32)
    ga = gb = None
    if a is not None:
        ga = np.zeros(r * q["cols"], np.float32)
        gb = np.zeros(q["rows"] * r, np.float32)
    s = qweight_struct(q)
    ls, lp = _lora_struct(a, b, r, alpha)
    check(c.lib.qh_qlora_backward(c.h, C.byref(s), lp, _ptr(x), x.size, _ptr(dy),
                                  dy.size, batch, _ptr(gx), _ptr(ga), _ptr(gb)))
    return gx, ga, gb


class Adam8bit:
    """``Adam8bit`` (qlora-core/src/optim.rs:147-249) with its state in HBM.
    ``step`` updates float32 numpy arrays in place and returns AdamStats."""

    def __init__(self, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8,
                 block_size=256, max_resident_pages=None, ctx=None):
        self.ctx = _ctx(ctx)
        cfg = AdamConfig()
        cfg.lr, cfg.beta1, cfg.beta2, cfg.eps = lr, beta1, beta2, eps
        cfg.block_size = block_size
        cfg.max_resident_pages = ((1 << 64) - 1 if max_resident_pages is None
                                  else max_resident_pages)
        self.block_size = block_size
        h = C.c_void_p()
        check(self.ctx.lib.qh_adam8bit_create(self.ctx.h, C.byref(cfg), C.byref(h)))
        self.h = h

    def __del__(self):
        if getattr(self, "h", None):
            try:
                self.ctx.lib.qh_adam8bit_destroy(self.h)
            except Exception:
                pass
            self.h = None

    def step(self, params: Sequence[np.ndarray], grads: Sequence) -> AdamStats:
        if len(params) != len(grads):
            raise _lib.QloraError(_lib.QH_ERR_SHAPE_MISMATCH,
                                  f"shape mismatch: params.len() = {len(params)} "
                                  f"but grads.len() = {len(grads)}")
        cnt = len(params)
        gs = [_f32(g) for g in grads]
        for p in params:
            if p.dtype != np.float32 or not p.flags.c_contiguous:
                raise TypeError("params must be contiguous float32 arrays")
        pp = (C.c_void_p * max(cnt, 1))(*[p.ctypes.data for p in params])
        gp = (C.c_void_p * max(cnt, 1))(*[g.ctypes.data for g in gs])
        pl = (C.c_size_t * max(cnt, 1))(*[p.size for p in params])
        gl = (C.c_size_t * max(cnt, 1))(*[g.size for g in gs])
        st = AdamStats()
        check(self.ctx.lib.qh_adam8bit_step(self.h, pp, pl, gp, gl, cnt,
                                            C.byref(st)))
        return st

    def state_bytes(self) -> int:
        return int(self.ctx.lib.qh_adam8bit_state_bytes(self.h))

    def state(self, idx: int, numel: int) -> dict:
        nb = -(-numel // self.block_size)
        mc, vc = np.zeros(numel, np.uint8), np.zeros(numel, np.uint8)
        ms, vs = np.zeros(nb, np.float32), np.zeros(nb, np.float32)
        step = C.c_uint64(0)
        check(self.ctx.lib.qh_adam8bit_get_state(self.h, idx, _ptr(mc), _ptr(ms),
                                                 _ptr(vc), _ptr(vs),
                                                 C.byref(step)))
        return dict(m_codes=mc, m_scales=ms, v_codes=vc, v_scales=vs,
                    step=step.value)


# =============================================================================
# ``qlora_wgpu`` surface (qlora-python/src/lib.rs)
# =============================================================================
class QuantizedWeight:
    """lib.rs:24-78.  Keeps the double-quantized store (codes, i8 scale codes,
    absmax) so the GPU reads the compact form; ``scales`` is the decoded fp32
    view the reference exposes."""

    def __init__(self, q: dict, double_quant: bool):
        self._q = q
        self.rows, self.cols = q["rows"], q["cols"]
        self.block_size = q["block_size"]
        self.double_quant = double_quant
        self._scales = None

    @property
    def scales(self):
        if self._scales is None:
            if "scales" in self._q:
                self._scales = self._q["scales"].tolist()
            else:
                self._scales = block_scales(self._q).tolist()
        return self._scales

    @property
    def codes_list(self):
        return self._q["codes"].tolist()

    def codes_bytes(self) -> bytes:
        return self._q["codes"].tobytes()

    def dequantize(self):
        return dequantize(self._q).tolist()

    def __repr__(self):
        return (f"QuantizedWeight(rows={self.rows}, cols={self.cols}, "
                f"block_size={self.block_size}, double_quant={self.double_quant})")


def quantize_nf4(weights, rows: int, cols: int, block_size: int = 64,
                 double_quant: bool = True) -> QuantizedWeight:
    """lib.rs:80-103."""
    q = quantize(weights, rows, cols, block_size, double_quant)
    return QuantizedWeight(q, double_quant)


def _rebuild(weight: QuantizedWeight, lora_a, lora_b, lora_alpha):
    """lib.rs:136-204 (shared validation of forward/backward)."""
    in_dim, out_dim = weight.cols, weight.rows
    if lora_a is None and lora_b is None:
        r = 0
    elif lora_a is not None and lora_b is not None:
        a, b = _f32(lora_a), _f32(lora_b)
        if a.size % max(in_dim, 1) != 0:
            raise ValueError("lora_a length must be a multiple of in_dim")
        r = a.size // max(in_dim, 1)
        if b.size != out_dim * r:
            raise ValueError("lora_b length must equal out_dim * rank")
    else:
        raise ValueError("lora_a and lora_b must be given together")
    if weight._q["codes"].size != (out_dim * in_dim + 1) // 2:
        raise ValueError("QuantizedWeight codes length does not match rows*cols")
    if r == 0:
        return None, None, 0, 0.0
    alpha = float(r) if lora_alpha is None else float(lora_alpha)
    return a, b, r, alpha


def qlora_linear_forward(x, batch: int, weight: QuantizedWeight, lora_a=None,
                         lora_b=None, lora_alpha=None, use_gpu: bool = False):
    """lib.rs:105-133."""
    a, b, r, alpha = _rebuild(weight, lora_a, lora_b, lora_alpha)
    return forward(weight._q, a, b, r, alpha, x, batch).tolist()


class BackwardOut:
    """lib.rs:238-247."""

    def __init__(self, grad_a, grad_b, grad_x):
        self.grad_a, self.grad_b, self.grad_x = grad_a, grad_b, grad_x


def qlora_linear_backward(x, dy, batch: int, weight: QuantizedWeight, lora_a=None,
                          lora_b=None, lora_alpha=None, use_gpu: bool = False):
    """lib.rs:206-236."""
    a, b, r, alpha = _rebuild(weight, lora_a, lora_b, lora_alpha)
    gx, ga, gb = backward(weight._q, a, b, r, alpha, x, dy, batch)
    return BackwardOut(None if ga is None else ga.tolist(),
                       None if gb is None else gb.tolist(), gx.tolist())


class PagedAdam:
    """lib.rs:249-298."""

    def __init__(self, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, block_size=256,
                 max_resident_pages=None):
        self.opt = Adam8bit(lr, beta1, beta2, eps, block_size, max_resident_pages)

    def step(self, params, grads):
        owned = [_f32(p).copy() for p in params]
        self.opt.step(owned, grads)
        return [p.tolist() for p in owned]

    def state_bytes(self) -> int:
        return self.opt.state_bytes()


# ---- packed NF4 files (safetensors; no fp32 round trip, no re-quantize) ----
def _qdict(w) -> dict:
    return w._q if isinstance(w, QuantizedWeight) else w


def nf4_file_bytes(weights) -> bytes:
    """A safetensors image of ``{name: QuantizedWeight or quantize() dict}``
    holding the packed parts (codes, int8 scale codes + absmax, or fp32
    scales) and each weight's rows, cols and block size."""
    L = _lib.load()
    names = list(weights)
    qs = [_qdict(weights[n]) for n in names]
    arr = (QWeight * max(1, len(qs)))()
    for i, q in enumerate(qs):
        arr[i] = qweight_struct(q)
    cn = (C.c_char_p * max(1, len(names)))(*[n.encode() for n in names])
    size = C.c_size_t()
    check(L.qh_nf4_file_size(arr, cn, len(names), C.byref(size)))
    buf = np.empty(size.value, np.uint8)
    check(L.qh_nf4_file_write(arr, cn, len(names), _ptr(buf), size.value))
    return buf.tobytes()


def save_nf4(path: str, weights) -> int:
    """Write ``nf4_file_bytes(weights)`` to ``path``; returns its size."""
    data = nf4_file_bytes(weights)
    with open(path, "wb") as f:
        f.write(data)
    return len(data)


def nf4_file_views(buf: np.ndarray):
    """[(name, qh_qweight view into buf)] of a file image held in ``buf``
    (a uint8 array the caller keeps alive)."""
    L = _lib.load()
    cnt = C.c_size_t()
    check(L.qh_nf4_file_count(_ptr(buf), buf.size, C.byref(cnt)))
    out = []
    for i in range(cnt.value):
        name = C.create_string_buffer(4096)
        v = QWeight()
        check(L.qh_nf4_file_entry(_ptr(buf), buf.size, i, name, 4096, C.byref(v)))
        out.append((name.value.decode(), v))
    return out


def _copy_part(addr: int, count: int, dtype) -> np.ndarray:
    nbytes = count * np.dtype(dtype).itemsize
    raw = (C.c_uint8 * nbytes).from_address(addr) if nbytes else b""
    return np.frombuffer(bytes(raw), dtype=dtype).copy()


def load_nf4(src) -> dict:
    """``{name: quantize()-style dict}`` from a path or a bytes image; the
    parts are copied out of the file bit for bit."""
    if isinstance(src, (bytes, bytearray)):
        buf = np.frombuffer(bytes(src), np.uint8).copy()
    else:
        buf = np.fromfile(src, dtype=np.uint8)
    out = {}
    for name, v in nf4_file_views(buf):
        n = v.rows * v.cols
        nb = -(-n // v.block_size)
        q = dict(rows=v.rows, cols=v.cols, block_size=v.block_size, n=n,
                 codes=_copy_part(v.codes, (n + 1) // 2, np.uint8))
        if v.scale_kind == QH_SCALES_DQ_INT8:
            q["scale_codes"] = _copy_part(v.scale_codes, nb, np.uint8)
            q["absmax"] = _copy_part(v.absmax, -(-nb // 256), np.float32)
        else:
            q["scales"] = _copy_part(v.scales, nb, np.float32)
        out[name] = q
    return out
