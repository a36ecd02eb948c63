"""Pins the oracle's int8 path (enhancers/fused_kernels.py:137-174 and enhancers/fused_int8.py:191-206 of the
reference) against what the mathematics fixes:

* the ConvRot rotation equals x @ (H4 (x) H4 (x) H4 (x) H4) / 16 with the reference's H4 (checked through q * scale
  within the quantisation error: a sign, index or stage-stride slip moves values by whole multiples of |x|);
* the rotation is its own inverse (H4 is symmetric with H4 @ H4 = 4 I);
* hand-computed rows: ties to even in rint, a zero row (scale 1e-30), the amax clamp at bf16's largest value;
* the int32 accumulator against an exact float64 matmul, and the epilogue against torch's own float32 ops and
  bfloat16 rounding (an independent implementation of the same order of operations).
"""
import numpy as np
import pytest
import torch

from oracle import lib

H4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64)


def _bf16_bits(x):
    return torch.from_numpy(np.asarray(x, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).numpy() \
        .view(np.uint16)


def _bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def _rotation():
    h = H4
    for _ in range(3):
        h = np.kron(h, H4)
    return h / 16.0


def test_convrot_matches_kronecker_hadamard():
    rng = np.random.default_rng(1)
    x = _bits_to_f32(_bf16_bits(rng.standard_normal((8, 512))))
    q, s = lib.quant_rows(_bf16_bits(x), 1)
    T = _rotation()
    y = np.concatenate([x[:, g * 256:(g + 1) * 256].astype(np.float64) @ T for g in range(2)], axis=1)
    approx = q.astype(np.float64) * s[:, None].astype(np.float64)
    # q = rint(bf16(bf16(y) / bf16(s))): error <= s / 2 + relative bf16 roundings (3 x 2^-8 of |y|)
    bound = s[:, None] * 0.5 + np.abs(y) * 3 * 2.0 ** -8 + s[:, None] * 2.0 ** -7 * 128
    assert np.all(np.abs(approx - y) <= bound)
    assert np.allclose(np.abs(y).max(axis=1) / 127, s, rtol=1e-6)


def test_rotation_is_an_involution():
    T = _rotation()
    assert np.allclose(T @ T, np.eye(256))
    assert np.allclose(T, T.T)


def test_plain_mode_is_per_token_absmax():
    rng = np.random.default_rng(2)
    x = _bits_to_f32(_bf16_bits(rng.standard_normal((16, 640)) * 3))
    q, s = lib.quant_rows(_bf16_bits(x), 0)
    amax = np.abs(x).max(axis=1)
    assert np.array_equal(s, (amax / np.float32(127)).astype(np.float32))
    approx = q.astype(np.float64) * s[:, None]
    assert np.all(np.abs(approx - x) <= s[:, None] * (0.5 + 128 * 2.0 ** -7) + np.abs(x) * 2.0 ** -7)
    assert q.max() == 127 or q.min() == -127


def test_kat_ties_zero_row_and_clamp():
    # row 0: amax 127 -> scale 1 exactly; values k + 0.5 tie to even
    row0 = np.zeros(256, dtype=np.float32)
    row0[:6] = [127, 2.5, 3.5, -2.5, -3.5, 0.5]
    # row 1: all zeros -> scale 1e-30, q 0
    row1 = np.zeros(256, dtype=np.float32)
    # row 2: bf16's largest finite value -> amax clamped at 3.38953139e38
    row2 = np.zeros(256, dtype=np.float32)
    row2[0] = 3.3895313892515355e38
    row2[1] = -1.0e38
    q, s = lib.quant_rows(_bf16_bits(np.stack([row0, row1, row2])), 0)
    assert s[0] == 1.0 and list(q[0, :6]) == [127, 2, 4, -2, -4, 0]
    assert s[1] == np.float32(1e-30) and not q[1].any()
    scale = torch.tensor(3.38953139e38, dtype=torch.float32) / 127
    assert s[2] == scale.item()
    sb = scale.to(torch.bfloat16).float()                   # rounds up: the top value lands on 126.5 -> 126
    xb = torch.tensor([3.3895313892515355e38, -1.0e38]).to(torch.bfloat16).float()
    expect = torch.round((xb / sb).to(torch.bfloat16).float()).clamp(-128, 127)   # torch.round: ties to even
    assert list(q[2, :2]) == [int(v) for v in expect] == [126, -37]


def test_linear_accumulator_and_epilogue():
    rng = np.random.default_rng(3)
    M, N, K = 24, 40, 512
    xq = rng.integers(-128, 128, size=(M, K), dtype=np.int64).astype(np.int8)
    wq = rng.integers(-128, 128, size=(N, K), dtype=np.int64).astype(np.int8)
    xs = (rng.random(M) * 0.1 + 1e-3).astype(np.float32)
    ws = (rng.random(N) * 0.01 + 1e-4).astype(np.float32)
    out, acc = lib.linear_i8(xq, wq, xs, ws, out_dt=lib.BF16, want_acc=True)
    ref_acc = xq.astype(np.float64) @ wq.astype(np.float64).T
    assert np.array_equal(acc.astype(np.float64), ref_acc)
    t = (torch.from_numpy(ref_acc).float() * torch.from_numpy(xs)[:, None]) * torch.from_numpy(ws)[None, :]
    assert np.array_equal(out, t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
    # float16 output and a bias (added in float32 before the single rounding)
    bias = rng.standard_normal(N).astype(np.float16)
    out16 = lib.linear_i8(xq, wq, xs, ws, out_dt=lib.F16, bias=bias.view(np.uint16))
    t16 = t + torch.from_numpy(bias.astype(np.float32))[None, :]
    assert np.array_equal(out16, t16.to(torch.float16).view(torch.int16).numpy().view(np.uint16))


def test_residual_epilogue():
    rng = np.random.default_rng(4)
    M, N, K, rows = 64, 96, 256, 4
    xq = rng.integers(-128, 128, size=(M, K)).astype(np.int8)
    wq = rng.integers(-128, 128, size=(N, K)).astype(np.int8)
    xs = np.full(M, 0.01, np.float32)
    ws = np.full(N, 0.02, np.float32)
    gate = _bf16_bits(rng.standard_normal((M // rows, N)))
    resid = _bf16_bits(rng.standard_normal((M, N)))
    got = lib.linear_i8_residual(xq, wq, xs, ws, gate, resid, rows)
    acc = torch.from_numpy(xq.astype(np.float64) @ wq.astype(np.float64).T).float()
    t = (acc * torch.from_numpy(xs)[:, None]) * torch.from_numpy(ws)[None, :]
    g = torch.from_numpy(_bits_to_f32(gate)).repeat_interleave(rows, 0)
    # the plain linear's bf16 output, then the gated residual in float32 (gate * out exact) rounded once to bf16
    tb = t.to(torch.bfloat16).float()
    ref = (torch.from_numpy(_bits_to_f32(resid)) + g * tb).to(torch.bfloat16)
    assert np.array_equal(got, ref.view(torch.int16).numpy().view(np.uint16))
    # ... which is torch's own addcmul on the bf16 tensors, as the unfused block computes it
    r16 = torch.from_numpy(_bits_to_f32(resid)).to(torch.bfloat16)
    add = torch.addcmul(r16, g.to(torch.bfloat16), t.to(torch.bfloat16))
    assert np.array_equal(got, add.view(torch.int16).numpy().view(np.uint16))
    # and not the unrounded product: dropping the bf16 rounding of the linear's value changes some results
    loose = (torch.from_numpy(_bits_to_f32(resid)) + g * t).to(torch.bfloat16)
    assert not np.array_equal(got, loose.view(torch.int16).numpy().view(np.uint16))


def test_rejects_bad_convrot_width():
    with pytest.raises(ValueError):
        lib.quant_rows(np.zeros((2, 300), dtype=np.uint16), 1)
