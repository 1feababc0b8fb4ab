"""ctypes view of the CPU oracle (``liboracle.so``, built from qlora_oracle.c).

TEST INFRASTRUCTURE ONLY: the checker for the HIP library.  Only tests/,
``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg import this
module; the product path (``vkqlora.rs_amd``) never does.

Each wrapper restates one function of stuarch/VkQLoRA.rs ``qlora-core``;
the C source cites the reference file:line it follows.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# QH_ORACLE_LIB names another build of the same source (the sanitizer build
# under tests/sanitize); by default the Makefile's liboracle.so.
_LIB_PATH = os.environ.get("QH_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")
_lib = None

NF4_ZERO_CODE = 7
DOUBLE_QUANT_BLOCK = 256

_f32p = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)


def build() -> None:
    """Compile the oracle with its Makefile (always re-run by callers)."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        L.or_rng_next_f64.restype = C.c_double
        L.or_rng_next_f64.argtypes = [C.POINTER(C.c_uint64)]
        L.or_rng_next_normal.restype = C.c_float
        L.or_nearest_nf4_code.restype = C.c_uint8
        L.or_nearest_nf4_code.argtypes = [C.c_float, C.c_float]
        L.or_quantize.restype = C.c_int
        L.or_quantize.argtypes = [_f32p, C.c_size_t, C.c_size_t, C.c_int, _u8p,
                                  _f32p, _u8p, _f32p]
        L.or_block_scales_dq.argtypes = [_u8p, _f32p, C.c_size_t, _f32p]
        L.or_dequantize.argtypes = [_u8p, _f32p, C.c_size_t, C.c_size_t, _f32p]
        for fn in ("or_matmul", "or_matmul_trans_a", "or_matmul_trans_b"):
            getattr(L, fn).argtypes = [_f32p, _f32p, C.c_size_t, C.c_size_t,
                                       C.c_size_t, _f32p]
        L.or_qlora_forward.argtypes = [_f32p, C.c_size_t, C.c_size_t, _f32p, _f32p,
                                       C.c_size_t, C.c_float, _f32p, C.c_size_t,
                                       _f32p]
        L.or_qlora_backward.argtypes = [_f32p, C.c_size_t, C.c_size_t, _f32p,
                                        _f32p, C.c_size_t, C.c_float, _f32p,
                                        _f32p, C.c_size_t, _f32p, _f32p, _f32p]
        L.or_fill_normal.argtypes = [C.POINTER(C.c_uint64), _f32p, C.c_size_t,
                                     C.c_float]
        L.or_fill_uniform.argtypes = [C.POINTER(C.c_uint64), _f32p, C.c_size_t,
                                      C.c_float, C.c_float]
        L.or_adam_create.restype = C.c_void_p
        L.or_adam_create.argtypes = [C.c_float, C.c_float, C.c_float, C.c_float,
                                     C.c_size_t, C.c_size_t]
        L.or_adam_destroy.argtypes = [C.c_void_p]
        L.or_adam_step.restype = C.c_size_t
        L.or_adam_step.argtypes = [C.c_void_p, C.POINTER(_f32p),
                                   C.POINTER(_f32p), C.POINTER(C.c_size_t),
                                   C.c_size_t]
        L.or_adam_state_bytes.restype = C.c_size_t
        L.or_adam_state_bytes.argtypes = [C.c_void_p]
        L.or_quantize_block_i8.restype = C.c_float
        L.or_quantize_block_i8.argtypes = [_f32p, C.c_size_t, _u8p]
        L.or_dequant_block_i8.argtypes = [_u8p, C.c_float, C.c_size_t, _f32p]
        L.or_adam_get_state.restype = C.c_int
        L.or_adam_get_state.argtypes = [C.c_void_p, C.c_size_t, _u8p, _f32p, _u8p,
                                        _f32p, C.POINTER(C.c_uint64)]
        L.or_rmsnorm.argtypes = [_f32p, _f32p, C.c_size_t, C.c_size_t, C.c_float,
                                 _f32p]
        L.or_rmsnorm_backward.argtypes = [_f32p, _f32p, _f32p, C.c_size_t,
                                          C.c_size_t, C.c_float, _f32p, _f32p]
        L.or_silu.restype = C.c_float
        L.or_silu.argtypes = [C.c_float]
        L.or_silu_prime.restype = C.c_float
        L.or_silu_prime.argtypes = [C.c_float]
        L.or_swiglu.argtypes = [_f32p, _f32p, C.c_size_t, _f32p]
        L.or_swiglu_backward.argtypes = [_f32p, _f32p, _f32p, C.c_size_t, _f32p,
                                         _f32p]
        L.or_softmax_cross_entropy.restype = C.c_float
        L.or_softmax_cross_entropy.argtypes = [_f32p, C.POINTER(C.c_uint32),
                                               C.c_size_t, C.c_size_t, _f32p]
        _lib = L
    return _lib


def _fp(a):
    return a.ctypes.data_as(_f32p)


def _bp(a):
    return a.ctypes.data_as(_u8p)


def nf4_levels() -> np.ndarray:
    arr = (C.c_float * 16).in_dll(lib(), "OR_NF4_LEVELS")
    return np.array(arr[:], dtype=np.float32)


# ---- generator (qlora-core/tests/quant.rs:6-24) ---------------------------
class Rng:
    """xorshift64* + Box-Muller, as in the reference's tests."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(seed & 0xFFFFFFFFFFFFFFFF)

    def normal(self, n: int, scale: float = 1.0) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        lib().or_fill_normal(C.byref(self.state), _fp(out), n, scale)
        return out

    def uniform(self, n: int, lo: float, hi: float) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        lib().or_fill_uniform(C.byref(self.state), _fp(out), n, lo, hi)
        return out

    def next_f64(self) -> float:
        return float(lib().or_rng_next_f64(C.byref(self.state)))


# ---- quant.rs -------------------------------------------------------------
def nearest_nf4_code(w: float, absmax: float) -> int:
    return int(lib().or_nearest_nf4_code(w, absmax))


def quantize(w: np.ndarray, block_size: int = 64, double_quant: bool = True):
    """Returns dict(codes, scales | scale_codes+absmax) (quant.rs:104-154)."""
    w = np.ascontiguousarray(w, dtype=np.float32).ravel()
    n = w.size
    if block_size == 0:
        raise ValueError("invalid config: block_size must be > 0")
    nb = -(-n // block_size)
    codes = np.zeros((n + 1) // 2, dtype=np.uint8)
    out = {"codes": codes, "n": n, "block_size": block_size}
    if double_quant:
        sc = np.zeros(nb, dtype=np.uint8)
        am = np.zeros(-(-nb // DOUBLE_QUANT_BLOCK), dtype=np.float32)
        rc = lib().or_quantize(_fp(w), n, block_size, 1, _bp(codes), None,
                               _bp(sc), _fp(am))
        out.update(scale_codes=sc, absmax=am)
    else:
        sf = np.zeros(nb, dtype=np.float32)
        rc = lib().or_quantize(_fp(w), n, block_size, 0, _bp(codes), _fp(sf),
                               None, None)
        out.update(scales=sf)
    if rc != 0:
        raise ValueError("invalid config: block_size must be > 0")
    return out


def block_scales(q) -> np.ndarray:
    """quant.rs:212-221."""
    if "scales" in q:
        return q["scales"].copy()
    nb = q["scale_codes"].size
    out = np.empty(nb, dtype=np.float32)
    lib().or_block_scales_dq(_bp(q["scale_codes"]), _fp(q["absmax"]), nb,
                             _fp(out))
    return out


def dequantize(q) -> np.ndarray:
    """quant.rs:157-167."""
    sc = block_scales(q)
    out = np.empty(q["n"], dtype=np.float32)
    lib().or_dequantize(_bp(q["codes"]), _fp(sc), q["n"], q["block_size"],
                        _fp(out))
    return out


def storage_bytes(q) -> int:
    """quant.rs:229-235."""
    if "scales" in q:
        return q["codes"].size + 4 * q["scales"].size
    return q["codes"].size + q["scale_codes"].size + 4 * q["absmax"].size


# ---- lora.rs --------------------------------------------------------------
def _mm(fn, a, b, m, k, n, out_len):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    c = np.empty(out_len, dtype=np.float32)
    getattr(lib(), fn)(_fp(a), _fp(b), m, k, n, _fp(c))
    return c


def matmul(a, b, m, k, n):
    return _mm("or_matmul", a, b, m, k, n, m * n)


def matmul_trans_a(a, b, m, k, n):
    return _mm("or_matmul_trans_a", a, b, m, k, n, k * n)


def matmul_trans_b(a, b, m, k, n):
    return _mm("or_matmul_trans_b", a, b, m, k, n, m * n)


# ---- qlora.rs -------------------------------------------------------------
def qlora_forward(w_deq, out_dim, in_dim, a, b, r, alpha, x, batch):
    w_deq = np.ascontiguousarray(w_deq, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(batch * out_dim, dtype=np.float32)
    if a is None:
        lib().or_qlora_forward(_fp(w_deq), out_dim, in_dim, None, None, 0, 0.0,
                               _fp(x), batch, _fp(y))
    else:
        a = np.ascontiguousarray(a, dtype=np.float32)
        b = np.ascontiguousarray(b, dtype=np.float32)
        lib().or_qlora_forward(_fp(w_deq), out_dim, in_dim, _fp(a), _fp(b), r,
                               alpha, _fp(x), batch, _fp(y))
    return y


def qlora_backward(w_deq, out_dim, in_dim, a, b, r, alpha, x, dy, batch):
    w_deq = np.ascontiguousarray(w_deq, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    dy = np.ascontiguousarray(dy, dtype=np.float32)
    gx = np.empty(batch * in_dim, dtype=np.float32)
    if a is None:
        lib().or_qlora_backward(_fp(w_deq), out_dim, in_dim, None, None, 0, 0.0,
                                _fp(x), _fp(dy), batch, _fp(gx), None, None)
        return gx, None, None
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    ga = np.empty(r * in_dim, dtype=np.float32)
    gb = np.empty(out_dim * r, dtype=np.float32)
    lib().or_qlora_backward(_fp(w_deq), out_dim, in_dim, _fp(a), _fp(b), r,
                            alpha, _fp(x), _fp(dy), batch, _fp(gx), _fp(ga),
                            _fp(gb))
    return gx, ga, gb


# ---- optim.rs -------------------------------------------------------------
class Adam8bit:
    """optim.rs:147-249 (paged 8-bit Adam, `v` in the sqrt domain)."""

    def __init__(self, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8,
                 block_size=256, max_resident_pages=None):
        mrp = (1 << 64) - 1 if max_resident_pages is None else max_resident_pages
        self.block_size = block_size
        self._h = lib().or_adam_create(lr, beta1, beta2, eps, block_size, mrp)
        if not self._h:
            raise ValueError("invalid config")

    def __del__(self):
        if getattr(self, "_h", None):
            lib().or_adam_destroy(self._h)
            self._h = None

    def step(self, params, grads):
        """Updates the float32 arrays in ``params`` in place; returns
        pages_streamed."""
        if len(params) != len(grads):
            raise ValueError("shape mismatch")
        for p, g in zip(params, grads):
            if p.size != g.size:
                raise ValueError("shape mismatch")
            assert p.dtype == np.float32 and p.flags.c_contiguous
        cnt = len(params)
        pp = (_f32p * cnt)(*[_fp(p) for p in params])
        gs = [np.ascontiguousarray(g, dtype=np.float32) for g in grads]
        gp = (_f32p * cnt)(*[_fp(g) for g in gs])
        lens = (C.c_size_t * cnt)(*[p.size for p in params])
        return int(lib().or_adam_step(self._h, pp, gp, lens, cnt))

    def state_bytes(self) -> int:
        return int(lib().or_adam_state_bytes(self._h))

    def state(self, idx: int, numel: int):
        nb = -(-numel // self.block_size)
        mc = np.zeros(numel, np.uint8)
        vc = np.zeros(numel, np.uint8)
        ms = np.zeros(nb, np.float32)
        vs = np.zeros(nb, np.float32)
        step = C.c_uint64(0)
        rc = lib().or_adam_get_state(self._h, idx, _bp(mc), _fp(ms), _bp(vc),
                                     _fp(vs), C.byref(step))
        if rc != 0:
            raise IndexError(idx)
        return dict(m_codes=mc, m_scales=ms, v_codes=vc, v_scales=vs,
                    step=step.value)


def quantize_block_i8(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    codes = np.zeros(x.size, np.uint8)
    am = lib().or_quantize_block_i8(_fp(x), x.size, _bp(codes))
    return codes, float(am)


def dequant_block_i8(codes, absmax):
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    out = np.empty(codes.size, np.float32)
    lib().or_dequant_block_i8(_bp(codes), absmax, codes.size, _fp(out))
    return out


# ---- qlora-model/src/llama.rs: the glue around the projections -------------
def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def rmsnorm(x, w, rows, h, eps):
    """llama.rs:730-739"""
    x, w = _f32(x), _f32(w)
    y = np.empty(rows * h, np.float32)
    lib().or_rmsnorm(_fp(x), _fp(w), rows, h, eps, _fp(y))
    return y


def rmsnorm_backward(x, w, dy, rows, h, eps):
    """llama.rs:605-628 -> (dx, dw)"""
    x, w, dy = _f32(x), _f32(w), _f32(dy)
    dx = np.empty(rows * h, np.float32)
    dw = np.empty(h, np.float32)
    lib().or_rmsnorm_backward(_fp(x), _fp(w), _fp(dy), rows, h, eps, _fp(dx), _fp(dw))
    return dx, dw


def silu(x: float) -> float:
    return float(lib().or_silu(x))


def silu_prime(x: float) -> float:
    return float(lib().or_silu_prime(x))


def swiglu(gate, up):
    """llama.rs:452-456"""
    gate, up = _f32(gate), _f32(up)
    act = np.empty(gate.size, np.float32)
    lib().or_swiglu(_fp(gate), _fp(up), gate.size, _fp(act))
    return act


def swiglu_backward(gate, up, d_act):
    """llama.rs:559-562 -> (d_gate, d_up)"""
    gate, up, d_act = _f32(gate), _f32(up), _f32(d_act)
    dg = np.empty(gate.size, np.float32)
    du = np.empty(gate.size, np.float32)
    lib().or_swiglu_backward(_fp(gate), _fp(up), _fp(d_act), gate.size, _fp(dg), _fp(du))
    return dg, du


def softmax_cross_entropy(logits, targets, seq, vocab):
    """llama.rs:487-514 -> (loss, dlogits)"""
    logits = _f32(logits)
    targets = np.ascontiguousarray(targets, dtype=np.uint32)
    assert targets.size == seq and logits.size == seq * vocab
    assert seq == 0 or int(targets.max()) < vocab
    d = np.empty(seq * vocab, np.float32)
    loss = lib().or_softmax_cross_entropy(
        _fp(logits), targets.ctypes.data_as(C.POINTER(C.c_uint32)), seq, vocab, _fp(d))
    return float(loss), d


def mlp_forward(norm_w, gate, up, down, x, seq, hidden, inter, eps):
    """The MLP half of block_forward (llama.rs:449-463) with QLoRA
    projections (llama.rs:106-114).  ``gate``/``up``/``down`` are
    (w_deq, a, b, r, alpha) with a = b = None for no adapter.  Returns
    (x_out, cache)."""
    x = _f32(x)
    xn = rmsnorm(x, norm_w, seq, hidden, eps)

    def proj(p, inp, out_dim, in_dim):
        wd, a, b, r, alpha = p
        return qlora_forward(wd, out_dim, in_dim, a, b, r, alpha, inp, seq)
    g = proj(gate, xn, inter, hidden)
    u = proj(up, xn, inter, hidden)
    act = swiglu(g, u)
    dn = proj(down, act, hidden, inter)
    x_out = (x + dn).astype(np.float32)   # x_i += d (llama.rs:458-460)
    return x_out, dict(x_mid=x, xn=xn, gate=g, up=u, act=act)


def mlp_backward(norm_w, gate, up, down, cache, dx_out, seq, hidden, inter, eps):
    """The MLP branch of block_backward (llama.rs:554-574) -> (dx_in,
    [(grad_a, grad_b) or None for gate, up, down])."""
    def proj_bwd(p, inp, dy, out_dim, in_dim):
        wd, a, b, r, alpha = p
        gx, ga, gb = qlora_backward(wd, out_dim, in_dim, a, b, r, alpha, inp, dy, seq)
        return gx, (None if a is None else (ga, gb))
    dx_out = _f32(dx_out)
    d_act, gd = proj_bwd(down, cache["act"], dx_out, hidden, inter)
    dg, du = swiglu_backward(cache["gate"], cache["up"], d_act)
    dxn_g, gg = proj_bwd(gate, cache["xn"], dg, inter, hidden)
    dxn_u, gu = proj_bwd(up, cache["xn"], du, inter, hidden)
    dxn = (dxn_g + dxn_u).astype(np.float32)
    dx_norm, _ = rmsnorm_backward(cache["x_mid"], norm_w, dxn, seq, hidden, eps)
    return (dx_norm + dx_out).astype(np.float32), [gg, gu, gd]


def _proj(p, inp, out_dim, in_dim, seq):
    wd, a, b, r, alpha = p
    return qlora_forward(wd, out_dim, in_dim, a, b, r, alpha, inp, seq)


def _proj_bwd(p, inp, dy, out_dim, in_dim, seq):
    wd, a, b, r, alpha = p
    gx, ga, gb = qlora_backward(wd, out_dim, in_dim, a, b, r, alpha, inp, dy, seq)
    return gx, (None if a is None else (ga, gb))


def attn_qkv_forward(norm_w, q, k, v, x, seq, hidden, kv_dim, eps):
    """The projections before the attention in block_forward
    (llama.rs:426-434): xn = rmsnorm(x), then q (hidden outputs), k and v
    (kv_dim outputs) of xn.  Projections as in mlp_forward.  Returns
    (q_out, k_out, v_out, cache)."""
    x = _f32(x)
    xn = rmsnorm(x, norm_w, seq, hidden, eps)
    return (_proj(q, xn, hidden, hidden, seq), _proj(k, xn, kv_dim, hidden, seq),
            _proj(v, xn, kv_dim, hidden, seq), dict(x_in=x, xn=xn))


def attn_o_forward(o, attn, x, seq, hidden):
    """llama.rs:436-439: x + o(attn)."""
    return (_f32(x) + _proj(o, _f32(attn), hidden, hidden, seq)).astype(np.float32)


def attn_o_backward(o, attn, dx_mid, seq, hidden):
    """llama.rs:577: (d_attn, (grad_a, grad_b) or None) of the o projection."""
    return _proj_bwd(o, _f32(attn), _f32(dx_mid), hidden, hidden, seq)


def attn_qkv_backward(norm_w, q, k, v, cache, dq, dk, dv, dx_mid, seq, hidden, kv_dim, eps):
    """llama.rs:580-601: the q, k, v backward, dxn = (dxn_q + dxn_k) + dxn_v,
    the norm's dx and the residual: returns (dx_mid + dx_norm,
    [grads of q, k, v])."""
    dxn_q, gq = _proj_bwd(q, cache["xn"], _f32(dq), hidden, hidden, seq)
    dxn_k, gk = _proj_bwd(k, cache["xn"], _f32(dk), kv_dim, hidden, seq)
    dxn_v, gv = _proj_bwd(v, cache["xn"], _f32(dv), kv_dim, hidden, seq)
    dxn = ((dxn_q + dxn_k).astype(np.float32) + dxn_v).astype(np.float32)
    dx_norm, _ = rmsnorm_backward(cache["x_in"], norm_w, dxn, seq, hidden, eps)
    return (_f32(dx_mid) + dx_norm).astype(np.float32), [gq, gk, gv]
