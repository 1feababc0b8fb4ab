"""Pins the CPU oracle (oracle/qlora_oracle.c) before it is trusted.

Each check is independent of the oracle's own code: the reference's known
answers and invariants (qlora-core tests), closed forms, exact-arithmetic
(f64 / integer) recomputation, or brute force on tiny inputs.
"""
import math

import numpy as np
import pytest

import oracle as O
from parity import SEED

# quant.rs:27-44 as f32 bit patterns (every f64 literal is exact in f32).
NF4_BITS = [0xbf800000, 0xbf3239b1, 0xbf066b30, 0xbeca32a0, 0xbe91a24d,
            0xbe3d353f, 0xbdba7871, 0x00000000, 0x3da2faff, 0x3e24cae3,
            0x3e7c04dd, 0x3ead033a, 0x3ee1a4b8, 0x3f1007ab, 0x3f3913b3,
            0x3f800000]
NF4_F64 = [-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
           -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
           0.07958029955625534, 0.16093020141124725, 0.24611230194568634,
           0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
           0.7229568362236023, 1.0]


def test_codebook_bits_sorted_and_exact():
    L = O.nf4_levels()
    assert list(L.view(np.uint32)) == NF4_BITS
    # quant.rs:305-313
    assert np.all(np.diff(L) > 0) and L[0] == -1.0 and L[15] == 1.0
    assert L[O.NF4_ZERO_CODE] == 0.0
    # every f64 literal equals its f32 rounding
    assert [float(v) for v in L] == NF4_F64


# ---- generator (qlora-core/tests/quant.rs:8-24) -----------------------------
def test_xorshift_closed_form():
    # recompute xorshift64* with Python integers
    s = SEED
    want = []
    for _ in range(5):
        s ^= s >> 12
        s ^= (s << 25) & 0xFFFFFFFFFFFFFFFF
        s ^= s >> 27
        want.append(((s * 0x2545F4914F6CDD1D) & 0xFFFFFFFFFFFFFFFF) >> 11)
    r = O.Rng(SEED)
    got = [r.next_f64() for _ in range(5)]
    assert got == [w / float((1 << 53) - 1) for w in want]


def test_normal_generator_moments():
    x = O.Rng(SEED).normal(200000)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01


# ---- nearest code (quant.rs:263-278) ------------------------------------------
def _scan_f64(t):
    """First index of the minimum distance, computed exactly in f64 on the
    f32 values (the f32 distance rounding can only merge distances that are
    within an ulp; those cases are checked separately below)."""
    d = [abs(l - t) for l in NF4_F64]
    return d.index(min(d))


def test_nearest_code_matches_exact_scan_random():
    rng = np.random.default_rng(1)
    ts = rng.uniform(-1, 1, 20000).astype(np.float32)
    for t in ts:
        assert O.nearest_nf4_code(float(t), 1.0) == _scan_f64(float(t))


def test_nearest_code_levels_and_midpoints():
    L = O.nf4_levels()
    for j in range(16):
        assert O.nearest_nf4_code(float(L[j]), 1.0) == j
    for j in range(15):
        # f32 values straddling the exact midpoint
        mid = np.float32((NF4_F64[j] + NF4_F64[j + 1]) / 2)
        for t in (np.nextafter(mid, np.float32(-2)), mid,
                  np.nextafter(mid, np.float32(2))):
            lo = np.float32(abs(np.float32(L[j]) - t))
            hi = np.float32(abs(np.float32(L[j + 1]) - t))
            want = j + 1 if hi < lo else j  # strict '<' keeps the first
            assert O.nearest_nf4_code(float(t), 1.0) == want


def test_nearest_code_specials():
    assert O.nearest_nf4_code(0.3, 0.0) == 7          # zero block
    assert O.nearest_nf4_code(-0.0, 1.0) == 7
    assert O.nearest_nf4_code(float("nan"), 1.0) == 0  # no '<' ever true
    assert O.nearest_nf4_code(float("inf"), float("inf")) == 0
    assert O.nearest_nf4_code(1.0, float("inf")) == 7


# ---- quantize / dequantize (qlora-core/tests/quant.rs) ----------------------
def test_roundtrip_normal_weights_bound_and_mse():
    # tests/quant.rs:37-68
    rows, cols = 64, 128
    w = O.Rng(SEED).normal(rows * cols)
    for dq in (False, True):
        q = O.quantize(w, 64, dq)
        back = O.dequantize(q)
        sc = O.block_scales(q)
        bound = 0.16 * np.repeat(sc, 64)[: w.size] + 1e-6
        assert np.all(np.abs(back - w) <= bound)
        assert np.mean((back.astype(np.float64) - w) ** 2) < 0.01


def test_roundtrip_uniform_bound():
    # tests/quant.rs:70-87
    r = O.Rng(0xDEAD_BEEF_CAFE_1234)
    w = np.array([np.float32(r.next_f64()) * np.float32(2.0) - np.float32(1.0)
                  for _ in range(16 * 64)], np.float32)
    q = O.quantize(w, 64, False)
    assert np.max(np.abs(O.dequantize(q) - w)) <= 0.15


def test_packed_layout_known_answer():
    # tests/quant.rs:89-98: 0.0..0.9, absmax 0.9, 5 bytes, 1 block
    w = np.array([i / 10 for i in range(10)], np.float32)
    q = O.quantize(w, 64, True)
    assert q["codes"].size == 5 and O.block_scales(q).size == 1
    assert abs(O.block_scales(q)[0] - 0.9) < 1e-6
    # codes by hand (exact f64 scan of t = w/0.9), low nibble first
    am = np.float32(0.9)
    codes = [_scan_f64(float(np.float32(v) / am)) for v in w]
    want = [codes[2 * i] | (codes[2 * i + 1] << 4) for i in range(5)]
    assert list(q["codes"]) == want
    # scale code: 0.9 is the only (hence max) block scale -> 127
    assert list(q["scale_codes"]) == [127] and q["absmax"][0] == am


def test_partial_last_block():
    # tests/quant.rs:100-113
    w = np.array([(i - 50) / 50 for i in range(100)], np.float32)
    q = O.quantize(w, 64, True)
    assert q["scale_codes"].size == 2 and O.dequantize(q).size == 100
    sc = O.block_scales(q)
    # block 0 absmax = 1.0 (i=0), block 1 absmax = 49/50
    assert q["absmax"][0] == 1.0
    assert list(q["scale_codes"]) == [127, int(math.floor(0.98 * 127 + 0.5))]
    assert sc[0] == np.float32(np.float32(127) / np.float32(127) * np.float32(1.0))


def test_odd_length_high_nibble_is_zero():
    w = np.linspace(-1, 1, 7).astype(np.float32)
    q = O.quantize(w, 64, False)
    assert q["codes"].size == 4 and (q["codes"][3] >> 4) == 0


def test_double_quant_storage_bytes():
    # tests/quant.rs:115-134: 1024 blocks -> 4096 vs 1024 + 4*4 bytes
    w = np.array([((i % 251) - 125) / 125 for i in range(65536)], np.float32)
    plain, dq = O.quantize(w, 64, False), O.quantize(w, 64, True)
    assert O.storage_bytes(plain) - O.storage_bytes(dq) == 4096 - 1040


def test_from_raw_parts_roundtrip_and_decoded_scales():
    # tests/quant.rs:136-154: fp32 store of the decoded scales dequantizes
    # identically to the double-quantized store.
    w = np.array([((i * 7) % 31) / 31 - 0.5 for i in range(512)], np.float32)
    q = O.quantize(w, 64, True)
    raw = dict(codes=q["codes"], n=q["n"], block_size=64, scales=O.block_scales(q))
    assert np.array_equal(O.dequantize(raw), O.dequantize(q))


def test_dequantize_matches_vectorised_closed_form():
    w = O.Rng(3).normal(4096 + 37, 0.02)
    for bs, dq in ((64, True), (64, False), (32, True), (100, False), (5, True)):
        q = O.quantize(w, bs, dq)
        nib = np.empty(w.size, np.int64)
        nib[0::2] = q["codes"][: (w.size + 1) // 2] & 15
        nib[1::2] = q["codes"][: w.size // 2] >> 4
        if dq:
            c = q["scale_codes"].view(np.int8).astype(np.float32)
            sc = (c / np.float32(127)) * np.repeat(q["absmax"], 256)[: c.size]
            sc = sc.astype(np.float32)
        else:
            sc = q["scales"]
        want = O.nf4_levels()[nib] * np.repeat(sc, bs)[: w.size]
        assert np.array_equal(O.dequantize(q).view(np.uint32),
                              want.astype(np.float32).view(np.uint32))


def test_scales_are_block_absmax_and_dq_codes_round_half_away():
    w = O.Rng(5).normal(64 * 600, 0.02)
    q = O.quantize(w, 64, False)
    assert np.array_equal(q["scales"], np.abs(w).reshape(-1, 64).max(1))
    qd = O.quantize(w, 64, True)
    s = q["scales"]
    for sb in range(qd["absmax"].size):
        chunk = s[sb * 256:(sb + 1) * 256]
        am = chunk.max()
        assert qd["absmax"][sb] == am
        t = (chunk / am).astype(np.float32) * np.float32(127)
        want = (np.sign(t) * np.floor(np.abs(t) + 0.5)).clip(-127, 127)
        assert np.array_equal(qd["scale_codes"][sb * 256:(sb + 1) * 256]
                              .view(np.int8), want.astype(np.int8))


def test_zero_block_decodes_to_exact_zero():
    # quant.rs:315-320
    q = O.quantize(np.zeros(64, np.float32), 64, True)
    assert np.all(q["codes"] == 0x77)
    assert np.array_equal(O.dequantize(q), np.zeros(64, np.float32))


def test_quantize_rejects_zero_block_size():
    with pytest.raises(ValueError):
        O.quantize(np.ones(1, np.float32), 0, False)


# ---- GEMMs (lora.rs:129-215) ---------------------------------------------------
def test_matmul_known_answer_and_transposes():
    assert list(O.matmul([1, 2, 3, 4], [5, 6, 7, 8], 2, 2, 2)) == [19, 22, 43, 50]
    a = np.array([1, 2, 3, 4, 5, 6], np.float32)
    b = np.array([1, -1, 0.5, 2, 0, 1.5], np.float32)
    assert np.array_equal(O.matmul_trans_a(a, b, 3, 2, 2),
                          O.matmul([1, 3, 5, 2, 4, 6], b, 2, 3, 2))
    b2 = np.array([1, 0, -1, 0.5, 2, 1.5], np.float32)
    assert np.array_equal(O.matmul_trans_b(a, b2, 2, 3, 2),
                          O.matmul(a, [1, 0.5, 0, 2, -1, 1.5], 2, 3, 2))


@pytest.mark.parametrize("m,k,n", [(18, 20, 33), (3, 1, 5), (7, 64, 9)])
def test_matmuls_match_f64(m, k, n):
    rng = np.random.default_rng(m * 100 + n)
    a = rng.standard_normal(m * k).astype(np.float32)
    b = rng.standard_normal(k * n).astype(np.float32)
    A, B = a.reshape(m, k).astype(np.float64), b.reshape(k, n).astype(np.float64)
    tol = 1e-5 * math.sqrt(k)
    assert np.allclose(O.matmul(a, b, m, k, n), (A @ B).ravel(), atol=tol)
    bt = rng.standard_normal(n * k).astype(np.float32)
    assert np.allclose(O.matmul_trans_b(a, bt, m, k, n),
                       (A @ bt.reshape(n, k).T.astype(np.float64)).ravel(), atol=tol)
    bm = rng.standard_normal(m * n).astype(np.float32)
    assert np.allclose(O.matmul_trans_a(a, bm, m, k, n),
                       (A.T @ bm.reshape(m, n).astype(np.float64)).ravel(),
                       atol=1e-5 * math.sqrt(m))


def test_matmul_trans_b_is_sequential_f32_sum():
    # ascending-p f32 accumulation without FMA: the sum 1 + 2^-24 + 2^-24
    # stays 1 in f32 (each add rounds), while an f64 or fused sum does not.
    a = np.array([1.0, 1.0, 1.0], np.float32)
    b = np.array([1.0, 2.0 ** -24, 2.0 ** -24], np.float32)
    assert O.matmul_trans_b(a, b, 1, 3, 1)[0] == np.float32(1.0)


# ---- layer (qlora-core/tests/qlora.rs) ---------------------------------------
def _layer(out_dim, in_dim, wfn):
    w = np.array([wfn(i) for i in range(out_dim * in_dim)], np.float32)
    return O.dequantize(O.quantize(w, 64, True)), w


def test_forward_matches_unfused_reference():
    # tests/qlora.rs:13-68 (scale 4, max_err < 0.2 against the fp32 W)
    out_dim, in_dim, r = 4, 8, 2
    wd, w = _layer(out_dim, in_dim, lambda i: ((i * 37) % 17) / 8 - 1)
    a = np.array([((i * 13) % 7) / 7 - 0.5 for i in range(r * in_dim)], np.float32)
    b = np.array([((i * 29) % 5) / 5 - 0.5 for i in range(out_dim * r)], np.float32)
    x = np.full(2 * in_dim, 0.5, np.float32)
    y = O.qlora_forward(wd, out_dim, in_dim, a, b, r, 8.0, x, 2)
    X, W = x.reshape(2, in_dim).astype(np.float64), w.reshape(out_dim, in_dim)
    A, B = a.reshape(r, in_dim), b.reshape(out_dim, r)
    want = X @ W.T + 4.0 * (X @ A.T) @ B.T
    assert np.max(np.abs(y - want.ravel())) < 0.2
    # and exactly consistent with the dequantized weight in f64
    want_q = X @ wd.reshape(out_dim, in_dim).T.astype(np.float64) + 4.0 * (X @ A.T) @ B.T
    assert np.max(np.abs(y - want_q.ravel())) < 1e-5


def test_forward_without_adapter():
    # tests/qlora.rs:70-86
    out_dim, in_dim = 8, 32
    wd, w = _layer(out_dim, in_dim, lambda i: ((i * 11) % 13) / 13 - 0.5)
    y = O.qlora_forward(wd, out_dim, in_dim, None, None, 0, 0.0,
                        np.ones(in_dim, np.float32), 1)
    exact = w.reshape(out_dim, in_dim).sum(1)
    assert np.max(np.abs(y - exact)) < 0.3


def test_backward_finite_differences():
    # tests/qlora.rs:88-148: L = sum(Y), eps 1e-3, tolerance 2e-2
    out_dim, in_dim, r, batch = 3, 4, 2, 2
    wd, _ = _layer(out_dim, in_dim, lambda i: ((i * 37) % 11) / 11 - 0.5)
    a = np.array([((i * 13) % 7) / 7 - 0.5 for i in range(r * in_dim)], np.float32)
    b = np.array([((i * 29) % 5) / 5 - 0.5 for i in range(out_dim * r)], np.float32)
    x = np.array([0.5, -0.25, 0.75, 1.0, 0.0, 0.25, -0.5, 1.5], np.float32)
    dy = np.ones(batch * out_dim, np.float32)
    gx, ga, gb = O.qlora_backward(wd, out_dim, in_dim, a, b, r, 8.0, x, dy, batch)

    def loss(x_, a_, b_):
        return float(np.sum(O.qlora_forward(wd, out_dim, in_dim, a_, b_, r, 8.0,
                                            x_, batch), dtype=np.float32))

    for buf, g in ((0, gx), (1, ga), (2, gb)):
        for i in range(g.size):
            bufs = [x.copy(), a.copy(), b.copy()]
            bufs[buf][i] += np.float32(1e-3)
            hi = loss(*bufs)
            bufs[buf][i] -= np.float32(2e-3)
            lo = loss(*bufs)
            assert abs(g[i] - (hi - lo) / 2e-3) < 2e-2


def test_backward_without_adapter_is_column_sums():
    # tests/qlora.rs:150-170
    out_dim, in_dim = 4, 8
    wd, _ = _layer(out_dim, in_dim, lambda i: ((i * 11) % 13) / 13 - 0.5)
    gx, ga, gb = O.qlora_backward(wd, out_dim, in_dim, None, None, 0, 0.0,
                                  np.full(in_dim, 0.5, np.float32),
                                  np.ones(out_dim, np.float32), 1)
    assert ga is None and gb is None
    assert np.max(np.abs(gx - wd.reshape(out_dim, in_dim).sum(0))) < 1e-6


def test_backward_matches_f64_on_random_layer():
    out_dim, in_dim, r, batch = 24, 40, 5, 7
    g = O.Rng(9)
    w = g.normal(out_dim * in_dim, 0.02)
    wd = O.dequantize(O.quantize(w, 64, True))
    a, b = g.normal(r * in_dim, 0.1), g.normal(out_dim * r, 0.1)
    x, dy = g.normal(batch * in_dim), g.normal(batch * out_dim)
    alpha = 3.0  # s = 0.6: not a power of two
    gx, ga, gb = O.qlora_backward(wd, out_dim, in_dim, a, b, r, alpha, x, dy, batch)
    W = wd.reshape(out_dim, in_dim).astype(np.float64)
    A, B = a.reshape(r, in_dim).astype(np.float64), b.reshape(out_dim, r).astype(np.float64)
    X, DY = x.reshape(batch, in_dim).astype(np.float64), dy.reshape(batch, out_dim)
    s = alpha / r
    ds = s * DY @ B
    assert np.allclose(gx, (DY @ W + ds @ A).ravel(), atol=1e-5)
    assert np.allclose(ga, (ds.T @ X).ravel(), atol=1e-5)
    assert np.allclose(gb, (s * DY.T @ (X @ A.T)).ravel(), atol=1e-5)


# ---- Adam (qlora-core/tests/optim.rs, optim.rs:251-272) -----------------------
def test_adam_tracks_f64_reference():
    # tests/optim.rs:27-60
    n = 64
    g = np.array([((i * 13) % 17) / 17 - 0.5 for i in range(n)], np.float32)
    p = np.ones(n, np.float32)
    opt = O.Adam8bit(lr=0.01, block_size=32)
    pr, m, v = np.ones(n), np.zeros(n), np.zeros(n)
    gr = g.astype(np.float64)
    for t in range(1, 6):
        opt.step([p], [g])
        m = 0.9 * m + 0.1 * gr
        v = 0.999 * v + 0.001 * gr * gr
        pr -= 0.01 * (m / (1 - 0.9 ** t)) / (np.sqrt(v / (1 - 0.999 ** t)) + 1e-8)
        assert np.max(np.abs(p - pr)) < 5e-3


def test_adam_paging_is_bitwise_invariant():
    # tests/optim.rs:62-87
    g = np.array([((i * 7) % 43) / 43 - 0.5 for i in range(256)], np.float32)
    pa = [np.full(256, 0.5, np.float32), np.full(256, -1.0, np.float32)]
    pb = [p.copy() for p in pa]
    oa = O.Adam8bit(lr=0.01, block_size=16, max_resident_pages=1)
    ob = O.Adam8bit(lr=0.01, block_size=16)
    for _ in range(3):
        assert oa.step(pa, [g, g]) == ob.step(pb, [g, g]) == 32
        assert all(np.array_equal(x, y) for x, y in zip(pa, pb))


def test_adam_converges_on_quadratic():
    # tests/optim.rs:89-105
    p = np.full(32, 2.0, np.float32)
    opt = O.Adam8bit(lr=0.05, block_size=32)
    for _ in range(300):
        opt.step([p], [2.0 * p])
    assert np.max(np.abs(p)) < 0.05


def test_adam_state_bytes_exact():
    # tests/optim.rs:107-131
    opt = O.Adam8bit()
    p = np.full(1024, 0.1, np.float32)
    opt.step([p], [np.full(1024, 0.01, np.float32)])
    assert opt.state_bytes() == 2048 + 2 * 4 * 4
    with pytest.raises(ValueError):
        O.Adam8bit(lr=-0.1)
    with pytest.raises(ValueError):
        O.Adam8bit(block_size=0)


def test_int8_block_roundtrip():
    # optim.rs:255-271
    x = np.array([((i * 7) % 101) / 101 - 0.5 for i in range(300)], np.float32)
    codes, scale = O.quantize_block_i8(x)
    assert abs(scale - 0.5) < 1e-6
    back = O.dequant_block_i8(codes, scale)
    assert np.all(np.abs(x - back) <= 0.5 / 127 * scale + 1e-7)
    zc, zs = O.quantize_block_i8(np.zeros(8, np.float32))
    assert zs == 0.0 and np.all(zc == 0)


def test_adam_first_step_closed_form():
    # step 1 from zero state: m = 0.1 g, var = 0.001 g^2, so
    # p1 = p0 - lr * (m/0.1) / (sqrt(var/0.001) + eps) = p0 - lr*g/(|g|+eps)
    g = np.array([0.5, -0.25, 2.0, -4.0], np.float32)
    p = np.zeros(4, np.float32)
    O.Adam8bit(lr=0.01, block_size=4).step([p], [g])
    assert np.allclose(p, -0.01 * np.sign(g), rtol=1e-6)
