"""GPU check of wf_linear_gguf (fused K-quant dequant + bf16 MFMA GEMM) through the C ABI.

Reference: a float64 GEMM of the same bf16 activations with the oracle's bit-exact dequantised bf16 weight (the
reference path: dequantize, then F.linear in bf16). The tolerance is the north-star bound, max relative error
<= 1e-2 (max |y - ref| / max |ref|); each element is also held to |y - ref| <= 2^-8 |ref| + 1e-3 max |ref|, which
only a correct weight meets (float32 accumulation order and the final bf16 rounding stay well inside it)."""
import numpy as np
import pytest
import torch

from conftest import sub

from oracle import lib

encode = sub("gguf_encode")

pytestmark = pytest.mark.gpu
TS = {12: 144, 13: 176, 14: 210}


def fused(native, x, raw_dev, qtype, N, bias=None, mid=0):
    M, K = x.shape
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    rc = native.lib().wf_linear_gguf(x.data_ptr(), M, K, raw_dev.data_ptr(), raw_dev.numel(), qtype, N,
                                     bias.data_ptr() if bias is not None else None, y.data_ptr(), mid,
                                     native.stream_of(x.device))
    assert rc == 0, native.last_error()
    torch.cuda.synchronize()
    return y


def weight_bf16(raw, qtype, mid, N, K):
    bits = lib.dequant(raw, qtype, mid, lib.BF16, N * K)
    return torch.from_numpy((bits.astype(np.uint32) << 16).view(np.float32).reshape(N, K))


def check(y, x, w, rows=None, bias=None):
    xs = x.float().cpu() if rows is None else x.float().cpu()[rows]
    ref = xs.double() @ w.double().T
    if bias is not None:
        ref = ref + bias.float().cpu().double()[None, :]
    got = (y.cpu() if rows is None else y.cpu()[rows]).double()
    scale = ref.abs().max().item()
    err = (got - ref).abs()
    assert err.max().item() / scale <= 1e-2
    assert bool((err <= ref.abs() * 2.0 ** -8 + 1e-3 * scale).all()), float((err - ref.abs() * 2.0 ** -8).max())


@pytest.mark.parametrize("qtype", [12, 13, 14])
@pytest.mark.parametrize("mid", [0, 2])
@pytest.mark.parametrize("M,N,K", [(77, 300, 512), (256, 256, 256), (512, 768, 5120)])
def test_fused_against_dequant_then_gemm(native, qtype, mid, M, N, K):
    raw = encode.random_blocks(qtype, N * K // 256, seed=qtype + M, family="normal")
    g = torch.Generator().manual_seed(M + N)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    y = fused(native, x.cuda(), torch.from_numpy(raw).cuda(), qtype, N, mid=mid)
    check(y, x, weight_bf16(raw, qtype, mid, N, K))


def test_fused_bias_and_encoded_weights(native):
    M, N, K = 300, 520, 1024
    w = encode.weights((N, K), seed=1234)
    raw = encode.encode(w, 13)
    g = torch.Generator().manual_seed(1)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    y = fused(native, x.cuda(), torch.from_numpy(raw).cuda(), 13, N, bias=bias.cuda())
    check(y, x, weight_bf16(raw, 13, 0, N, K), bias=bias)


@pytest.mark.parametrize("qtype", [12, 13, 14])
@pytest.mark.parametrize("M,N,K,with_bias", [(4096, 4500, 256, False), (4000, 4480, 512, True)])
def test_wide_tiles_whole_output(native, qtype, M, N, K, with_bias):
    # outputs of more than one round of 256 x 256 tiles but one round of 256 x 320 tiles take the 320-row weight
    # tiles (two dequantisation tasks for the first two waves); N = 4500 leaves a partial last tile and an odd row
    # length (element stores), N = 4480 whole 16-byte runs; every output element is checked
    raw = encode.random_blocks(qtype, N * K // 256, seed=qtype + N, family="normal")
    g = torch.Generator().manual_seed(M + K)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    bias = torch.randn(N, generator=g).to(torch.bfloat16) if with_bias else None
    y = fused(native, x.cuda(), torch.from_numpy(raw).cuda(), qtype, N,
              bias=bias.cuda() if with_bias else None)
    check(y, x, weight_bf16(raw, qtype, 0, N, K), bias=bias)


@pytest.mark.parametrize("qtype", [13, 14])
@pytest.mark.parametrize("N,K", [(5120, 5120), (13824, 5120), (5120, 13824)])
def test_wan_block_shapes_sampled_rows(native, qtype, N, K):
    M = 4096
    raw = encode.encode(encode.weights((N, K), seed=1234 + N + K), qtype)
    g = torch.Generator().manual_seed(99)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    y = fused(native, x.cuda(), torch.from_numpy(raw).cuda(), qtype, N)
    rows = torch.tensor([0, 1, 31, 32, 255, 256, 1000, 2047, 2048, 4095])
    check(y, x, weight_bf16(raw, qtype, 0, N, K), rows=rows)


@pytest.mark.parametrize("qtype", [12, 13, 14])
@pytest.mark.parametrize("mid", [0, 2])
@pytest.mark.parametrize("M,N,K,with_bias", [(1, 300, 256, True), (5, 5120, 5120, False), (16, 61, 512, True),
                                             (17, 1000, 1024, False), (33, 300, 2048, True), (64, 5120, 512, False),
                                             (48, 777, 1280, True), (65, 256, 768, False)])
def test_few_rows_whole_output(native, qtype, mid, M, N, K, with_bias):
    # up to 64 activation rows take the few-rows kernel (16 weight rows per workgroup, K split over its 8 waves,
    # 1 to 4 row tiles of 16; K = 256 and 512 leave waves with no super-block); 65 rows the tiled kernel: ragged M
    # and N, every output element checked
    raw = encode.random_blocks(qtype, N * K // 256, seed=qtype * 7 + M, family="normal")
    g = torch.Generator().manual_seed(M * 31 + N)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    bias = torch.randn(N, generator=g).to(torch.bfloat16) if with_bias else None
    y = fused(native, x.cuda(), torch.from_numpy(raw).cuda(), qtype, N, bias=bias.cuda() if with_bias else None,
              mid=mid)
    check(y, x, weight_bf16(raw, qtype, mid, N, K), bias=bias)


def test_rejects_what_it_does_not_handle(native):
    lib_ = native.lib()
    assert lib_.wf_linear_gguf(None, 4, 300, None, 0, 12, 4, None, None, 0, None) == native.EUNSUPPORTED   # K
    assert lib_.wf_linear_gguf(None, 4, 256, None, 144 * 4, 8, 4, None, None, 0, None) == native.EUNSUPPORTED
    assert lib_.wf_linear_gguf(None, 4, 256, None, 144 * 3, 12, 4, None, None, 0, None) == native.EUNSUPPORTED
