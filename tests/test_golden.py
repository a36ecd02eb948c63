"""The oracle against the committed golden fixtures of tests/golden/ (written by tests/golden/make_golden.py): every
GGML type x MID/OUT pair of the dequantisation (typical, zero, subnormal and largest float16 scales), the plain and
ConvRot row quantisers, and the int8 linear's accumulators and epilogue -- bit for bit."""
import os

import numpy as np
import pytest

from oracle import lib, np_oracle

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
PER_BLOCK = {2: 32, 3: 32, 6: 32, 7: 32, 8: 32, 10: 256, 11: 256, 12: 256, 13: 256, 14: 256}


def _load(name):
    with np.load(os.path.join(G, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == np.float32:
        return bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))
    return np.array_equal(a, b)


@pytest.mark.parametrize("qtype", sorted(PER_BLOCK))
def test_dequant_fixtures(qtype):
    d = _load("dequant.npz")
    raw = d[f"raw_{qtype}"]
    n = raw.size // {2: 18, 3: 20, 6: 22, 7: 24, 8: 34, 10: 84, 11: 110, 12: 144, 13: 176, 14: 210}[qtype] \
        * PER_BLOCK[qtype]
    for m in range(3):
        for o in range(3):
            assert _same(lib.dequant(raw, qtype, m, o, n), d[f"out_{qtype}_{m}_{o}"]), (qtype, m, o)


def test_quant_rows_fixtures():
    q = _load("quant_rows.npz")
    for mode in (0, 1):
        xq, xs = lib.quant_rows(q["x"], mode)
        assert np.array_equal(xq, q[f"q_{mode}"]) and _same(xs, q[f"s_{mode}"]), mode
    assert q["s_0"][1] == np.float32(1e-30) and not q["q_0"][1].any()     # the zero row: the scale floor


def test_linear_i8_fixtures():
    z = _load("linear_i8.npz")
    y, acc = lib.linear_i8(z["xq"], z["wq"], z["xs"], z["ws"], out_dt=lib.BF16, want_acc=True)
    assert np.array_equal(acc, z["acc"]) and np.array_equal(y, z["y"])
    # the accumulators are the exact integer products
    assert np.array_equal(z["acc"], z["xq"].astype(np.int64) @ z["wq"].astype(np.int64).T)


def test_convrot_stage_order_fixture():
    # rows on which the order of a radix-4 stage's sums decides int8 values: the C oracle and the numpy
    # restatement in the reference's left-to-right order both give the fixture, and each other order misses it
    z = _load("convrot_order.npz")
    xq, xs = lib.quant_rows(z["x"], 1)
    assert np.array_equal(xq, z["q"]) and _same(xs, z["s"])
    nq, ns = np_oracle.quant_rows_convrot(z["x"], "ltr")
    assert np.array_equal(nq, z["q"]) and _same(ns, z["s"])
    for order in ("pair", "rtl"):
        oq, _ = np_oracle.quant_rows_convrot(z["x"], order)
        assert (oq != z["q"]).any(axis=1).all(), order


def test_numpy_convrot_restatement_equals_the_c_oracle():
    q = _load("quant_rows.npz")
    nq, ns = np_oracle.quant_rows_convrot(q["x"])
    assert np.array_equal(nq, q["q_1"]) and _same(ns, q["s_1"])
