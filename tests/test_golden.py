"""The committed oracle vectors (tests/golden/oracle_vectors.npz, written by
tests/golden/make_golden.py) against the oracle as built now, bit for bit,
plus the known answers the vectors must show (reference file:line)."""
import os
import sys

import numpy as np

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)


def _load():
    return np.load(os.path.join(GOLDEN, "oracle_vectors.npz"))  # allow_pickle=False


def test_oracle_reproduces_committed_vectors():
    import make_golden
    fresh = make_golden.build()
    gold = _load()
    assert sorted(fresh) == sorted(gold.files)
    for k in gold.files:
        a, b = np.asarray(fresh[k]), gold[k]
        assert a.dtype == b.dtype and a.shape == b.shape, k
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), k


def test_vectors_known_answers():
    g = _load()
    codes = g["q_small_dq1_codes"]
    lo, hi = codes & 15, codes >> 4
    nib = np.empty(2 * codes.size, np.uint8)
    nib[0::2], nib[1::2] = lo, hi
    # quant.rs:315-320: an all-zero block quantizes to code 7 and scale 0
    assert np.all(nib[64:128] == O.NF4_ZERO_CODE)
    assert g["q_small_dq0_scales"][1] == 0.0
    assert np.all(g["q_small_dq0_deq"][64:128] == 0.0)
    # block 2 holds +-0.5 over a 0.02-scale rest: absmax 0.5, codes 15 / 0
    assert g["q_small_dq0_scales"][2] == np.float32(0.5)
    assert list(nib[128:131]) == [15, 0, 15]
    # 201 elements: 101 code bytes, the odd last nibble left 0 (quant.rs:129-135)
    assert codes.size == 101 and (codes[-1] >> 4) == 0
    # 260 blocks -> two fp32 absmax values (quant.rs:283-299)
    assert g["q_big_absmax"].size == 2 and g["q_big_scale_codes"].size == 260
    # cross-entropy rows of dlogits sum to zero (llama.rs:507-511)
    assert np.max(np.abs(g["ce_dlogits"].reshape(4, 50).sum(axis=1))) < 1e-6
