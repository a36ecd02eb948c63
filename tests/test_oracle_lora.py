"""The oracle's LoRA add (wfo_dequant_add: the reference's _deq_add, enhancers/gguf_dequant.py:99-133, as
_add_loras launches it, :387-409) pinned without the reference.

* A zero difference (or a zero scale) leaves exactly the dequantisation, for every format (identity; up to the
  sign of zero: IEEE gives -0 + 0 = +0, and the reference's add does the same).
* The fused first LoRA equals the dequantisation followed by the add onto it (composition).
* The add itself against an independent restatement: numpy float32 products and sums, numpy's own float16
  conversion and torch's bfloat16 conversion (not the oracle's C textbook / bit-rule code).
* Known answers where the inner rounding decides the result: a planted mistake that drops R_OUT(diff * sa) (or
  fuses the product into the sum) gives the neighbouring value and fails them."""
import numpy as np
import pytest
import torch

from conftest import sub

from oracle import lib

encode = sub("gguf_encode")

F16, BF16, F32 = 0, 1, 2
ALL_TYPES = [2, 3, 6, 7, 8, 10, 11, 12, 13, 14]


def _f32(bits, D):
    if D == F32:
        return np.asarray(bits, dtype=np.float32)
    if D == BF16:
        return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def _round_bits(x, D):
    """float32 -> dtype D bits, round to nearest even, by numpy (f16) and torch (bf16)."""
    x = np.asarray(x, dtype=np.float32)
    if D == F32:
        return x.copy()
    if D == F16:
        return x.astype(np.float16).view(np.uint16)
    return torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _same_up_to_zero_sign(a, b, D):
    fa, fb = _f32(a, D), _f32(b, D)
    bits_eq = np.asarray(a).view(np.uint8).reshape(fa.size, -1) == np.asarray(b).view(np.uint8).reshape(fb.size, -1)
    return bool((bits_eq.all(axis=1) | ((fa == 0) & (fb == 0))).all())


@pytest.mark.parametrize("qtype", ALL_TYPES)
def test_zero_difference_leaves_the_dequantisation(qtype):
    nblk = 37 if encode.PER_BLOCK[qtype] == 256 else 301
    raw = encode.random_blocks(qtype, nblk, seed=70 + qtype, family="finite")
    n = nblk * encode.PER_BLOCK[qtype]
    rng = np.random.default_rng(qtype)
    for mid, out in [(F16, BF16), (BF16, F16), (F32, F32), (F16, F16)]:
        ref = lib.dequant(raw, qtype, mid, out, n)
        got = lib.dequant_add(raw, qtype, mid, out, np.zeros(n, np.float32), 0.8)
        assert _same_up_to_zero_sign(got, ref, out)
        assert not np.signbit(_f32(got, out)[_f32(got, out) == 0]).any()      # -0 + 0 = +0
        diff = rng.standard_normal(n).astype(np.float32)
        assert _same_up_to_zero_sign(lib.dequant_add(raw, qtype, mid, out, diff, 0.0), ref, out)


@pytest.mark.parametrize("qtype", [3, 8, 11, 12, 14])
def test_first_lora_is_dequantisation_then_add(qtype):
    nblk = 19 if encode.PER_BLOCK[qtype] == 256 else 157
    raw = encode.random_blocks(qtype, nblk, seed=90 + qtype, family="normal")
    n = nblk * encode.PER_BLOCK[qtype]
    diff = (np.random.default_rng(5).standard_normal(n) * 0.01).astype(np.float32)
    for mid, out in [(F16, BF16), (F32, F16), (BF16, F32)]:
        fused = lib.dequant_add(raw, qtype, mid, out, diff, 0.61)
        base = lib.dequant(raw, qtype, mid, out, n)
        assert np.array_equal(fused, lib.dequant_add(None, 0, 0, out, diff, 0.61, base=base))


@pytest.mark.parametrize("out", [F16, BF16, F32])
def test_add_against_numpy_and_torch_rounding(out):
    rng = np.random.default_rng(11 + out)
    n = 20000
    w = _round_bits(rng.standard_normal(n).astype(np.float32) * 0.05, out)
    diff = (rng.standard_normal(n) * np.exp2(rng.integers(-12, 4, n))).astype(np.float32)
    sa = np.float32(0.3125 * 0.77)
    got = lib.dequant_add(None, 0, 0, out, diff, float(sa), base=w)
    p = diff * sa                                                # float32 product
    rp = _f32(_round_bits(p, out), out)
    expect = _round_bits(_f32(w, out) + rp, out)                  # float32 sum, then the rounding
    assert np.array_equal(np.asarray(got).view(np.uint8), np.asarray(expect).view(np.uint8))


def test_inner_rounding_decides_ties():
    # bf16: w = 1.0; diff * sa just above 2^-8 (half the spacing at 1.0). R(diff * sa) = 2^-8, so the sum is the
    # tie 1 + 2^-8, which goes to the even 1.0; without the inner rounding it would round up to 1 + 2^-7.
    p = np.float32(np.exp2(-8) * (1 + np.exp2(-12)))
    got = lib.dequant_add(None, 0, 0, BF16, np.array([p], np.float32), 1.0, base=np.array([0x3F80], np.uint16))
    assert got[0] == 0x3F80
    # float16: the same at the float16 spacing of 1.0 (2^-10)
    p = np.float32(np.exp2(-11) * (1 + np.exp2(-12)))
    got = lib.dequant_add(None, 0, 0, F16, np.array([p], np.float32), 1.0, base=np.array([0x3C00], np.uint16))
    assert got[0] == 0x3C00
    # and above the tie both ways agree: 1 + 3 * 2^-9 rounds to 1 + 2^-7 in bf16
    p = np.float32(3 * np.exp2(-9))
    got = lib.dequant_add(None, 0, 0, BF16, np.array([p], np.float32), 1.0, base=np.array([0x3F80], np.uint16))
    assert got[0] == 0x3F81


def test_product_is_rounded_in_float32_before_the_cast():
    # diff * sa = (1 + 2^-23) * (1 + 2^-23) = 1 + 2^-22 + 2^-46: float32 keeps 1 + 2^-22; f32 output shows it
    d = np.float32(1 + np.exp2(-23))
    got = lib.dequant_add(None, 0, 0, F32, np.array([d], np.float32), float(d), base=np.array([0.0], np.float32))
    assert got[0] == np.float32(1 + np.exp2(-22))
