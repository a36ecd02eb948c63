"""The oracle's quantiser operations (wfo_quant_rows_pre / wfo_ln_stats: the reference's _quant_row with PRE 1..3,
enhancers/fused_kernels.py:84-174) pinned without the reference.

* LayerNorm statistics: a numpy restatement in the reference's own tensor form (128 threads as a vector, the
  shuffle-down merges as slices of a [4, 32] array; fma through 64-bit-mantissa long doubles) agrees bit for bit
  with the C loops; constant rows give the exact mean and zero variance; the statistics sit within float32
  rounding of the float64 mean / variance.
* MOD and GELU: the fused result equals torch's own bf16 operations (x * (1 + scale) + shift; torch's GELU through
  the table torch builds) followed by the already pinned ConvRot quantiser.
* LNMOD: the same with the normalisation (x - mean) * rstd computed in numpy float32, and within one bf16 step of
  torch's layer_norm."""
import numpy as np
import pytest
import torch

from oracle import lib

LD = np.longdouble


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _fma(a, b, c):
    return (np.asarray(a, LD) * np.asarray(b, LD) + np.asarray(c, LD)).astype(np.float32)


def _combine(m, s, c, mo, so, co):
    delta = (m - mo).astype(np.float32)
    count = (co + c).astype(np.float32)
    coef = (np.float32(1) / count).astype(np.float32)
    na, nb = (co * coef).astype(np.float32), (c * coef).astype(np.float32)
    mean = _fma(na, mo, (nb * m).astype(np.float32))
    sig = _fma(((delta * delta).astype(np.float32) * co).astype(np.float32), nb, (so + s).astype(np.float32))
    return mean, sig, count


def ln_stats_np(row_bits):
    x = (row_bits.astype(np.uint32) << 16).view(np.float32)
    K = x.size
    t = np.arange(128)
    mean = np.zeros(128, np.float32)
    sig = np.zeros(128, np.float32)
    cnt = np.zeros(128, np.float32)
    for j in range(K // 512):
        for ii in range(4):
            v = x[(t + j * 128) * 4 + ii]
            delta = (v - mean).astype(np.float32)
            cnt = (cnt + np.float32(1)).astype(np.float32)
            mean = _fma(delta, (np.float32(1) / cnt).astype(np.float32), mean)
            sig = _fma(delta, (v - mean).astype(np.float32), sig)
    m, s, c = mean.reshape(4, 32), sig.reshape(4, 32), cnt.reshape(4, 32)
    for N in (32, 16, 8, 4, 2):
        h = N // 2
        m2, s2, c2 = _combine(m[:, :h], s[:, :h], c[:, :h], m[:, h:N], s[:, h:N], c[:, h:N])
        m, s, c = m2, s2, c2
    m, s, c = m.reshape(4), s.reshape(4), c.reshape(4)
    m, s, c = _combine(m[:2], s[:2], c[:2], m[2:], s[2:], c[2:])
    m, s, c = _combine(m[:1], s[:1], c[:1], m[1:], s[1:], c[1:])
    return m[0], np.float32(s[0] / np.float32(K))


@pytest.mark.parametrize("K", [512, 1024, 2048, 5120])
def test_ln_stats_matches_tensor_form_restatement(K):
    g = torch.Generator().manual_seed(K)
    for scale, shift in ((1.0, 0.0), (30.0, 5.0), (1e-3, -2.0)):
        x = (torch.randn((3, K), generator=g) * scale + shift).to(torch.bfloat16)
        for r in _bits(x):
            mu, var = lib.ln_stats(r)
            mu2, var2 = ln_stats_np(r)
            assert np.float32(mu).view(np.uint32) == np.float32(mu2).view(np.uint32)
            assert np.float32(var).view(np.uint32) == np.float32(var2).view(np.uint32)
            xf = (r.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
            assert abs(mu - xf.mean()) <= 1e-5 * (abs(xf).mean() + 1e-30)
            assert abs(var - xf.var()) <= 1e-4 * xf.var() + 1e-30


def test_ln_stats_constant_rows():
    for bits in (0x3FC0, 0xC2F7, 0x0000):
        mu, var = lib.ln_stats(np.full(1024, bits, np.uint16))
        assert mu == np.float32((np.uint32(bits) << 16).view(np.float32)) and var == 0.0


def _rand(g, shape, scale=1.0):
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("K,groups,rows", [(1024, 2, 3), (5120, 1, 4), (2048, 4, 1)])
def test_mod_is_torch_modulate_then_quantiser(K, groups, rows):
    g = torch.Generator().manual_seed(K + rows)
    x = _rand(g, (groups * rows, K))
    scale, shift = _rand(g, (groups, K), 0.3), _rand(g, (groups, K), 0.5)
    s1 = (1 + scale)
    xq, xs = lib.quant_rows_pre(_bits(x), 2, _bits(s1), _bits(shift), rows)
    y = (x.view(groups, rows, K) * s1[:, None, :] + shift[:, None, :]).reshape(-1, K)   # torch bf16 ops
    rq, rs = lib.quant_rows(_bits(y), 1)
    assert np.array_equal(xq, rq) and np.array_equal(xs.view(np.uint32), rs.view(np.uint32))


def test_gelu_is_table_lookup_of_torch_gelu():
    table = torch.nn.functional.gelu(torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16))
    g = torch.Generator().manual_seed(3)
    x = _rand(g, (5, 2048), 3.0)
    xq, xs = lib.quant_rows_pre(_bits(x), 1, _bits(table))
    rq, rs = lib.quant_rows(_bits(torch.nn.functional.gelu(x)), 1)
    assert np.array_equal(xq, rq) and np.array_equal(xs.view(np.uint32), rs.view(np.uint32))


@pytest.mark.parametrize("K", [1024, 5120])
def test_lnmod_is_normalise_modulate_then_quantiser(K):
    g = torch.Generator().manual_seed(K)
    groups, rows, eps = 2, 3, 1e-6
    x = _rand(g, (groups * rows, K), 2.0)
    scale, shift = _rand(g, (groups, K), 0.3), _rand(g, (groups, K), 0.5)
    s1 = 1 + scale
    xq, xs = lib.quant_rows_pre(_bits(x), 3, _bits(s1), _bits(shift), rows, eps)
    xb = _bits(x)
    normed = []
    for r in range(groups * rows):
        mu, var = lib.ln_stats(xb[r])
        rstd = np.float32(1.0 / np.sqrt(np.float64(np.float32(var + np.float32(eps)))))
        xf = (xb[r].astype(np.uint32) << 16).view(np.float32)
        normed.append(torch.from_numpy(((xf - mu).astype(np.float32) * rstd).astype(np.float32)))
    normed = torch.stack(normed).to(torch.bfloat16)
    ref_ln = torch.nn.functional.layer_norm(x.float(), (K,), eps=eps).to(torch.bfloat16)
    assert ((normed.float() - ref_ln.float()).abs() <= ref_ln.float().abs() * 2 ** -7 + 1e-6).all()
    y = (normed.view(groups, rows, K) * s1[:, None, :] + shift[:, None, :]).reshape(-1, K)
    rq, rs = lib.quant_rows(_bits(y), 1)
    assert np.array_equal(xq, rq) and np.array_equal(xs.view(np.uint32), rs.view(np.uint32))
