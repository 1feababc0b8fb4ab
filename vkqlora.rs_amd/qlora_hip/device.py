"""Device-resident use of the C ABI from PyTorch (torch is only the HBM
allocator and stream provider here; all compute is the library's kernels).

``DeviceWeight`` keeps a packed NF4 weight in HBM (codes, i8 scale codes,
fp32 absmax); ``forward`` / ``backward`` call the ``*_dev`` entry points on
torch's current stream without synchronising.

Import torch before the library is first loaded: torch's wheel bundles its
own ``libamdhip64.so.7`` (same soname as the one the library links), the
first one loaded serves the process, and torch finds no GPU on the other.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional

import torch

from ._lib import (AttnBlock, AttnCache, Lora, MlpBlock, MlpCache, QWeight, QH_BF16, QH_F32, QH_SCALES_DQ_INT8,
                   QH_SCALES_F32, check, default_context)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _p(t: Optional[torch.Tensor]):
    return None if t is None else C.c_void_p(t.data_ptr())


class DeviceWeight:
    """A rows x cols NF4 weight resident in HBM."""

    def __init__(self, rows, cols, block_size, codes, scales=None,
                 scale_codes=None, absmax=None):
        self.rows, self.cols, self.block_size = rows, cols, block_size
        self.codes, self.scales = codes, scales
        self.scale_codes, self.absmax = scale_codes, absmax

    @property
    def n(self) -> int:
        return self.rows * self.cols

    @property
    def nbytes(self) -> int:
        """Packed bytes (quant.rs:229-235 storage_bytes)."""
        t = self.codes.numel()
        if self.scales is not None:
            return t + 4 * self.scales.numel()
        return t + self.scale_codes.numel() + 4 * self.absmax.numel()

    @classmethod
    def quantize(cls, w: torch.Tensor, block_size: int = 64,
                 double_quant: bool = True, ctx=None) -> "DeviceWeight":
        """GPU quantize_nf4 of a (rows, cols) float32 CUDA tensor."""
        ctx = ctx or default_context()
        rows, cols = w.shape
        w = w.contiguous()
        n = rows * cols
        nb = -(-n // block_size)
        dev = w.device
        codes = torch.empty((n + 1) // 2, dtype=torch.uint8, device=dev)
        if double_quant:
            sc = torch.empty(nb, dtype=torch.uint8, device=dev)
            am = torch.empty(-(-nb // 256), dtype=torch.float32, device=dev)
            check(ctx.lib.qh_quantize_nf4_dev(ctx.h, _p(w), rows, cols, block_size, 1,
                                              _p(codes), None, _p(sc), _p(am),
                                              C.c_void_p(_stream())))
            return cls(rows, cols, block_size, codes, scale_codes=sc, absmax=am)
        sf = torch.empty(nb, dtype=torch.float32, device=dev)
        check(ctx.lib.qh_quantize_nf4_dev(ctx.h, _p(w), rows, cols, block_size, 0,
                                          _p(codes), _p(sf), None, None,
                                          C.c_void_p(_stream())))
        return cls(rows, cols, block_size, codes, scales=sf)

    @classmethod
    def from_host_view(cls, v: QWeight, device, ctx=None) -> "DeviceWeight":
        """Copy a host ``qh_qweight`` (e.g. a view into a file image) into
        HBM with ``qh_weight_upload_dev`` on the current stream."""
        ctx = ctx or default_context()
        n = v.rows * v.cols
        nb = -(-n // v.block_size)
        codes = torch.empty((n + 1) // 2, dtype=torch.uint8, device=device)
        if v.scale_kind == QH_SCALES_DQ_INT8:
            sc = torch.empty(nb, dtype=torch.uint8, device=device)
            am = torch.empty(-(-nb // 256), dtype=torch.float32, device=device)
            check(ctx.lib.qh_weight_upload_dev(ctx.h, C.byref(v), _p(codes), None, _p(sc),
                                               _p(am), C.c_void_p(_stream())))
            return cls(v.rows, v.cols, v.block_size, codes, scale_codes=sc, absmax=am)
        sf = torch.empty(nb, dtype=torch.float32, device=device)
        check(ctx.lib.qh_weight_upload_dev(ctx.h, C.byref(v), _p(codes), _p(sf), None, None,
                                           C.c_void_p(_stream())))
        return cls(v.rows, v.cols, v.block_size, codes, scales=sf)

    def clone(self) -> "DeviceWeight":
        c = lambda t: None if t is None else t.clone()  # noqa: E731
        return DeviceWeight(self.rows, self.cols, self.block_size, c(self.codes),
                            c(self.scales), c(self.scale_codes), c(self.absmax))

    def struct(self) -> QWeight:
        s = QWeight()
        s.rows, s.cols, s.block_size = self.rows, self.cols, self.block_size
        s.codes = self.codes.data_ptr()
        if self.scales is not None:
            s.scale_kind = QH_SCALES_F32
            s.scales = self.scales.data_ptr()
        else:
            s.scale_kind = QH_SCALES_DQ_INT8
            s.scale_codes = self.scale_codes.data_ptr()
            s.absmax = self.absmax.data_ptr()
        return s

    def dequantize(self, ctx=None) -> torch.Tensor:
        ctx = ctx or default_context()
        out = torch.empty(self.n, dtype=torch.float32, device=self.codes.device)
        s = self.struct()
        check(ctx.lib.qh_dequantize_dev(ctx.h, C.byref(s), _p(out),
                                        C.c_void_p(_stream())))
        return out


def lora_struct(a: Optional[torch.Tensor], b: Optional[torch.Tensor], r: int,
                alpha: float):
    if a is None:
        return None
    s = Lora()
    s.a, s.a_len = a.data_ptr(), a.numel()
    s.b, s.b_len = b.data_ptr(), b.numel()
    s.r, s.alpha = r, alpha
    s._refs = (a, b)  # the struct holds raw pointers: keep the tensors alive
    return s


def _dt(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return QH_F32
    if t.dtype == torch.bfloat16:
        return QH_BF16
    raise TypeError(f"activations must be float32 or bfloat16, got {t.dtype}")


def forward(w: DeviceWeight, lora, x: torch.Tensor, batch: int, y: torch.Tensor,
            t1: Optional[torch.Tensor] = None, ctx=None, qw=None) -> None:
    """Y = X.dequant(W)^T + (alpha/r) (X.A^T).B^T on the current stream.
    ``lora`` is a ``Lora`` struct (or None); ``t1`` receives X.A^T."""
    ctx = ctx or default_context()
    s = qw if qw is not None else w.struct()
    check(ctx.lib.qh_qlora_forward_dev(
        ctx.h, C.byref(s), None if lora is None else C.byref(lora), _p(x), _dt(x),
        batch, _p(y), _p(t1), C.c_void_p(_stream())))


def forward_group(layers, batch: int, ctx=None) -> None:
    """The forward of several independent layers on the current stream
    (qh_qlora_forward_group_dev): ``layers`` holds (weight, lora, x, y, t1)
    per layer, weight a DeviceWeight or a QWeight view, lora a ``Lora``
    struct or None, t1 a tensor or None.  Each layer's outputs are those of
    ``forward`` bit for bit; at batch 1, consecutive layers served by the
    one-launch decode kernel run in pairs, one launch per pair."""
    ctx = ctx or default_context()
    n = len(layers)
    if n == 0:
        return
    dts = {_dt(L[2]) for L in layers}
    if len(dts) != 1:
        raise TypeError("all layers' x must share a dtype")
    ws = (QWeight * n)(*[L[0] if isinstance(L[0], QWeight) else L[0].struct() for L in layers])
    loras = (C.POINTER(Lora) * n)(*[C.pointer(L[1]) if L[1] is not None else C.POINTER(Lora)()
                                    for L in layers])
    xs = (C.c_void_p * n)(*[L[2].data_ptr() for L in layers])
    ys = (C.c_void_p * n)(*[L[3].data_ptr() for L in layers])
    t1s = (C.c_void_p * n)(*[L[4].data_ptr() if L[4] is not None else None for L in layers])
    check(ctx.lib.qh_qlora_forward_group_dev(ctx.h, n, ws, loras, xs, dts.pop(), batch, ys,
                                             t1s, C.c_void_p(_stream())))


def backward(w: DeviceWeight, lora, x: torch.Tensor, dy: torch.Tensor, batch: int,
             gx: torch.Tensor, ga: Optional[torch.Tensor] = None,
             gb: Optional[torch.Tensor] = None, t1: Optional[torch.Tensor] = None,
             ctx=None, qw=None) -> None:
    ctx = ctx or default_context()
    if x.dtype != dy.dtype:
        raise TypeError("x and dy must share a dtype")
    if lora is not None and (ga is None or gb is None):
        raise ValueError("grad_a and grad_b buffers are required with an adapter")
    s = qw if qw is not None else w.struct()
    check(ctx.lib.qh_qlora_backward_dev(
        ctx.h, C.byref(s), None if lora is None else C.byref(lora), _p(x), _p(dy),
        _dt(x), batch, _p(t1), _p(gx), _p(ga), _p(gb), C.c_void_p(_stream())))


def _layer_arrays(layers):
    n = len(layers)
    ws = (QWeight * n)(*[w if isinstance(w, QWeight) else w.struct() for w, _ in layers])
    loras = (C.POINTER(Lora) * n)(*[C.pointer(l) if l is not None else C.POINTER(Lora)()
                                    for _, l in layers])
    return n, ws, loras


def _ptrs(ts):
    return (C.c_void_p * len(ts))(*[t.data_ptr() if t is not None else None for t in ts])


def forward_shared(layers, x: torch.Tensor, batch: int, ys, t1s=None, ctx=None) -> None:
    """The forward of layers that read the same activations x
    (qh_qlora_forward_shared_dev): ``layers`` holds (weight, lora) per
    layer (weight a DeviceWeight or QWeight view, lora a ``Lora`` or None);
    ``ys[i]`` / ``t1s[i]`` receive layer i's Y and T1."""
    ctx = ctx or default_context()
    n, ws, loras = _layer_arrays(layers)
    if n == 0:
        return
    t1p = _ptrs(t1s if t1s is not None else [None] * n)
    check(ctx.lib.qh_qlora_forward_shared_dev(ctx.h, n, ws, loras, _p(x), _dt(x), batch,
                                              _ptrs(ys), t1p, C.c_void_p(_stream())))


def backward_shared(layers, x: torch.Tensor, dys, batch: int, gx: torch.Tensor,
                    gas=None, gbs=None, t1s=None, ctx=None) -> None:
    """The backward of layers that read the same activations x
    (qh_qlora_backward_shared_dev): gx receives the sum of the layers' input
    gradients, gas[i] / gbs[i] layer i's grad_A / grad_B (None without an
    adapter), t1s[i] the forward's T1 (or None)."""
    ctx = ctx or default_context()
    n, ws, loras = _layer_arrays(layers)
    if n == 0:
        return
    if any(d.dtype != x.dtype for d in dys):
        raise TypeError("x and every dy must share a dtype")
    none = [None] * n
    check(ctx.lib.qh_qlora_backward_shared_dev(
        ctx.h, n, ws, loras, _p(x), _ptrs(dys), _dt(x), batch,
        _ptrs(t1s if t1s is not None else none), _p(gx),
        _ptrs(gas if gas is not None else none), _ptrs(gbs if gbs is not None else none),
        C.c_void_p(_stream())))


# ---- the glue of a decoder block (qlora-model/src/llama.rs) ------------------
def _f32c(t: torch.Tensor, what: str) -> torch.Tensor:
    if t.dtype != torch.float32 or not t.is_contiguous():
        raise TypeError(f"{what} must be a contiguous float32 tensor")
    return t


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float,
            out: Optional[torch.Tensor] = None, ctx=None) -> torch.Tensor:
    """rmsnorm_in_place (llama.rs:730-739) over the last dimension of x;
    ``out`` may be ``x`` itself."""
    ctx = ctx or default_context()
    _f32c(x, "x"), _f32c(w, "w")
    h = w.numel()
    out = torch.empty_like(x) if out is None else _f32c(out, "out")
    check(ctx.lib.qh_rmsnorm_dev(ctx.h, _p(x), _p(w), x.numel() // max(h, 1), h, eps,
                                 _p(out), C.c_void_p(_stream())))
    return out


def rmsnorm_backward(x: torch.Tensor, w: torch.Tensor, dy: torch.Tensor, eps: float,
                     want_dw: bool = True, ctx=None):
    """rmsnorm_backward (llama.rs:605-628) -> (dx, dw or None)."""
    ctx = ctx or default_context()
    for t, n in ((x, "x"), (w, "w"), (dy, "dy")):
        _f32c(t, n)
    h = w.numel()
    dx = torch.empty_like(x)
    dw = torch.empty(h, dtype=torch.float32, device=x.device) if want_dw else None
    check(ctx.lib.qh_rmsnorm_backward_dev(ctx.h, _p(x), _p(w), _p(dy), x.numel() // max(h, 1),
                                          h, eps, _p(dx), _p(dw), C.c_void_p(_stream())))
    return dx, dw


def swiglu(gate: torch.Tensor, up: torch.Tensor, out: Optional[torch.Tensor] = None,
           ctx=None) -> torch.Tensor:
    """act = silu(gate) * up (llama.rs:452-456)."""
    ctx = ctx or default_context()
    _f32c(gate, "gate"), _f32c(up, "up")
    if gate.numel() != up.numel():
        raise ValueError("gate and up differ in size")
    out = torch.empty_like(gate) if out is None else _f32c(out, "out")
    check(ctx.lib.qh_swiglu_dev(ctx.h, _p(gate), _p(up), gate.numel(), _p(out),
                                C.c_void_p(_stream())))
    return out


def swiglu_backward(gate: torch.Tensor, up: torch.Tensor, d_act: torch.Tensor, ctx=None):
    """(d_gate, d_up) of act = silu(gate) * up (llama.rs:559-562)."""
    ctx = ctx or default_context()
    for t, n in ((gate, "gate"), (up, "up"), (d_act, "d_act")):
        _f32c(t, n)
    dg, du = torch.empty_like(gate), torch.empty_like(up)
    check(ctx.lib.qh_swiglu_backward_dev(ctx.h, _p(gate), _p(up), _p(d_act), gate.numel(),
                                         _p(dg), _p(du), C.c_void_p(_stream())))
    return dg, du


def softmax_cross_entropy(logits: torch.Tensor, targets: torch.Tensor,
                          dlogits: Optional[torch.Tensor] = None, ctx=None):
    """softmax_cross_entropy (llama.rs:487-514) of (seq, vocab) logits and
    int32 targets -> (loss tensor of one float, dlogits).  ``dlogits`` may be
    ``logits`` itself."""
    ctx = ctx or default_context()
    _f32c(logits, "logits")
    if targets.dtype != torch.int32 or not targets.is_contiguous():
        raise TypeError("targets must be a contiguous int32 tensor")
    seq, vocab = logits.shape
    d = torch.empty_like(logits) if dlogits is None else _f32c(dlogits, "dlogits")
    loss = torch.empty(1, dtype=torch.float32, device=logits.device)
    check(ctx.lib.qh_softmax_cross_entropy_dev(ctx.h, _p(logits), _p(targets), seq, vocab,
                                               _p(loss), _p(d), C.c_void_p(_stream())))
    return loss, d


# ---- packed NF4 files straight into HBM ---------------------------------------
def read_file_pinned(path: str) -> torch.Tensor:
    """The file's bytes in pinned host memory (so uploads are DMA)."""
    import os
    n = os.path.getsize(path)
    buf = torch.empty(n, dtype=torch.uint8, pin_memory=True)
    with open(path, "rb") as f:
        f.readinto(buf.numpy())
    return buf


def load_nf4(src, device="cuda:0", ctx=None) -> dict:
    """``{name: DeviceWeight}`` from a packed NF4 file (path, or a host uint8
    tensor / array holding its image): each weight's parts are copied from the
    image into HBM as they are stored, with no fp32 and no quantize on the
    way.  The copies are enqueued on the current stream; the call waits for
    them before the image can go away."""
    from .api import nf4_file_views
    buf = read_file_pinned(src) if isinstance(src, str) else src
    arr = buf.numpy() if isinstance(buf, torch.Tensor) else buf
    out = {name: DeviceWeight.from_host_view(v, device, ctx=ctx)
           for name, v in nf4_file_views(arr)}
    torch.cuda.current_stream().synchronize()
    return out


# ---- a decoder block's MLP on device (qh_mlp_forward_dev / _backward_dev) ----
class MLPBlock:
    """The MLP half of a decoder block (llama.rs:449-463, 554-574): RMSNorm,
    gate / up / down QLoRA projections, SwiGLU and the residual add, with
    every activation in HBM.  ``loras`` holds (a, b, r, alpha) per
    projection (gate, up, down) or None."""

    def __init__(self, norm_w: torch.Tensor, gate: DeviceWeight, up: DeviceWeight,
                 down: DeviceWeight, loras=(None, None, None), eps: float = 1e-5, ctx=None):
        self.ctx = ctx or default_context()
        self.norm_w, self.w = _f32c(norm_w, "norm_w"), (gate, up, down)
        self.loras = [None if l is None else lora_struct(*l) for l in loras]
        self.ranks = [0 if l is None else l[2] for l in loras]
        self.hidden, self.inter = down.rows, gate.rows
        b = MlpBlock()
        b.hidden, b.inter, b.eps = self.hidden, self.inter, eps
        b.norm_w = norm_w.data_ptr()
        b.gate, b.up, b.down = gate.struct(), up.struct(), down.struct()
        b.gate_lora, b.up_lora, b.down_lora = [
            C.pointer(l) if l is not None else C.POINTER(Lora)() for l in self.loras]
        self.s = b

    def new_cache(self, seq: int, device="cuda:0") -> dict:
        e = lambda n: torch.empty(seq, n, device=device)  # noqa: E731
        c = dict(x_mid=e(self.hidden), xn=e(self.hidden), gate=e(self.inter),
                 up=e(self.inter), act=e(self.inter))
        for name, r in zip(("t1_gate", "t1_up", "t1_down"), self.ranks):
            c[name] = e(r) if r else None
        return c

    @staticmethod
    def _cs(c: dict) -> MlpCache:
        s = MlpCache()
        for k in ("x_mid", "xn", "gate", "up", "act", "t1_gate", "t1_up", "t1_down"):
            setattr(s, k, None if c[k] is None else c[k].data_ptr())
        return s

    def forward(self, x: torch.Tensor, cache: dict) -> torch.Tensor:
        """x (seq, hidden) is updated in place: x + mlp(rmsnorm(x))."""
        _f32c(x, "x")
        cs = self._cs(cache)
        check(self.ctx.lib.qh_mlp_forward_dev(self.ctx.h, C.byref(self.s), _p(x), x.shape[0],
                                              C.byref(cs), C.c_void_p(_stream())))
        return x

    def backward(self, cache: dict, dx_out: torch.Tensor):
        """-> (dx_in, [(grad_a, grad_b) or None for gate, up, down]); the
        cache's gate and up buffers are consumed."""
        _f32c(dx_out, "dx_out")
        seq = dx_out.shape[0]
        dx_in = torch.empty_like(dx_out)
        grads, ga, gb = [], (C.c_void_p * 3)(), (C.c_void_p * 3)()
        for i, (l, w) in enumerate(zip(self.loras, self.w)):
            if l is None:
                grads.append(None)
                continue
            a = torch.empty(l.r * w.cols, device=dx_out.device)
            b = torch.empty(w.rows * l.r, device=dx_out.device)
            ga[i], gb[i] = a.data_ptr(), b.data_ptr()
            grads.append((a, b))
        cs = self._cs(cache)
        check(self.ctx.lib.qh_mlp_backward_dev(self.ctx.h, C.byref(self.s), C.byref(cs),
                                               _p(dx_out), seq, _p(dx_in), ga, gb,
                                               C.c_void_p(_stream())))
        return dx_in, grads


class AttnProjections:
    """The projections around a decoder block's attention (llama.rs:426-439,
    577-601): RMSNorm and the q / k / v QLoRA projections before it, the o
    projection and the residual add after it, and their backward, with every
    activation in HBM.  The attention itself is the caller's.  ``loras``
    holds (a, b, r, alpha) per projection (q, k, v, o) or None."""

    def __init__(self, norm_w: torch.Tensor, q: DeviceWeight, k: DeviceWeight,
                 v: DeviceWeight, o: DeviceWeight, loras=(None, None, None, None),
                 eps: float = 1e-5, ctx=None):
        self.ctx = ctx or default_context()
        self.norm_w, self.w = _f32c(norm_w, "norm_w"), (q, k, v, o)
        self.loras = [None if l is None else lora_struct(*l) for l in loras]
        self.ranks = [0 if l is None else l[2] for l in loras]
        self.hidden, self.kv_dim = q.rows, k.rows
        b = AttnBlock()
        b.hidden, b.kv_dim, b.eps = self.hidden, self.kv_dim, eps
        b.norm_w = norm_w.data_ptr()
        b.q, b.k, b.v, b.o = q.struct(), k.struct(), v.struct(), o.struct()
        b.q_lora, b.k_lora, b.v_lora, b.o_lora = [
            C.pointer(l) if l is not None else C.POINTER(Lora)() for l in self.loras]
        self.s = b

    def new_cache(self, seq: int, device="cuda:0") -> dict:
        e = lambda n: torch.empty(seq, n, device=device)  # noqa: E731
        c = dict(x_in=e(self.hidden), xn=e(self.hidden), attn=e(self.hidden))
        for name, r in zip(("t1_q", "t1_k", "t1_v", "t1_o"), self.ranks):
            c[name] = e(r) if r else None
        return c

    @staticmethod
    def _cs(c: dict) -> AttnCache:
        s = AttnCache()
        for k in ("x_in", "xn", "attn", "t1_q", "t1_k", "t1_v", "t1_o"):
            setattr(s, k, None if c[k] is None else c[k].data_ptr())
        return s

    def _grads(self, idx, dev):
        grads, ga, gb = [], (C.c_void_p * len(idx))(), (C.c_void_p * len(idx))()
        for j, i in enumerate(idx):
            l, w = self.loras[i], self.w[i]
            if l is None:
                grads.append(None)
                continue
            a = torch.empty(l.r * w.cols, device=dev)
            b = torch.empty(w.rows * l.r, device=dev)
            ga[j], gb[j] = a.data_ptr(), b.data_ptr()
            grads.append((a, b))
        return grads, ga, gb

    def qkv_forward(self, x: torch.Tensor, cache: dict):
        """-> (q, k, v) of rmsnorm(x); x is unchanged."""
        _f32c(x, "x")
        seq = x.shape[0]
        q = torch.empty(seq, self.hidden, device=x.device)
        k = torch.empty(seq, self.kv_dim, device=x.device)
        v = torch.empty(seq, self.kv_dim, device=x.device)
        cs = self._cs(cache)
        check(self.ctx.lib.qh_attn_qkv_forward_dev(self.ctx.h, C.byref(self.s), _p(x), seq,
                                                   C.byref(cs), _p(q), _p(k), _p(v),
                                                   C.c_void_p(_stream())))
        return q, k, v

    def o_forward(self, x: torch.Tensor, cache: dict) -> torch.Tensor:
        """x (seq, hidden) is updated in place: x + o(cache["attn"])."""
        _f32c(x, "x")
        cs = self._cs(cache)
        check(self.ctx.lib.qh_attn_o_forward_dev(self.ctx.h, C.byref(self.s), _p(x),
                                                 x.shape[0], C.byref(cs),
                                                 C.c_void_p(_stream())))
        return x

    def o_backward(self, cache: dict, dx_mid: torch.Tensor):
        """-> (d_attn, (grad_a, grad_b) of o or None)."""
        _f32c(dx_mid, "dx_mid")
        seq = dx_mid.shape[0]
        d_attn = torch.empty(seq, self.hidden, device=dx_mid.device)
        grads, ga, gb = self._grads((3,), dx_mid.device)
        cs = self._cs(cache)
        check(self.ctx.lib.qh_attn_o_backward_dev(self.ctx.h, C.byref(self.s), C.byref(cs),
                                                  _p(dx_mid), seq, _p(d_attn), ga[0], gb[0],
                                                  C.c_void_p(_stream())))
        return d_attn, grads[0]

    def qkv_backward(self, cache: dict, dq: torch.Tensor, dk: torch.Tensor,
                     dv: torch.Tensor, dx_mid: torch.Tensor):
        """-> (dx_in, [(grad_a, grad_b) or None for q, k, v])."""
        for t, n in ((dq, "dq"), (dk, "dk"), (dv, "dv"), (dx_mid, "dx_mid")):
            _f32c(t, n)
        seq = dx_mid.shape[0]
        dx_in = torch.empty_like(dx_mid)
        grads, ga, gb = self._grads((0, 1, 2), dx_mid.device)
        cs = self._cs(cache)
        check(self.ctx.lib.qh_attn_qkv_backward_dev(self.ctx.h, C.byref(self.s), C.byref(cs),
                                                    _p(dq), _p(dk), _p(dv), _p(dx_mid), seq,
                                                    _p(dx_in), ga, gb, C.c_void_p(_stream())))
        return dx_in, grads
