"""GPU parity of wf_dequant (the gfx950 kernels) against the oracle, bit for bit (NaN payloads excepted).

Covers every format x every MID / OUT pair on random blocks (three scale families, block counts that leave ragged
tails), Q8_0 on every finite float16 scale x every quant, the drop-in Python entry points on the GPU, and one
full-size 14B-DiT FFN weight (13824 x 5120, Q4_K, MID float16 -> bfloat16) compared value by value."""
import numpy as np
import pytest
import torch

from conftest import sub
from oracle import lib, np_oracle

encode = sub("gguf_encode")

pytestmark = pytest.mark.gpu

F16, BF16, F32 = 0, 1, 2
TD = {F16: torch.float16, BF16: torch.bfloat16, F32: torch.float32}
ALL_TYPES = [2, 3, 6, 7, 8, 10, 11, 12, 13, 14]
PAIRS = [(m, o) for m in range(3) for o in range(3)]


def _bits(t, D):
    t = t.cpu()
    if D == F32:
        return t.numpy().astype(np.float32)
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _same(a, b, D):
    fa, fb = np_oracle.bits_to_f32(a, D), np_oracle.bits_to_f32(b, D)
    eq = np.asarray(a).view(np.uint8).reshape(fa.size, -1) == np.asarray(b).view(np.uint8).reshape(fb.size, -1)
    ok = eq.all(axis=1) | (np.isnan(fa) & np.isnan(fb))
    return bool(ok.all()), np.nonzero(~ok)[0][:8]


def gpu_dequant(native, raw_dev, qtype, mid, out, n):
    res = torch.empty(n, dtype=TD[out], device=raw_dev.device)
    rc = native.lib().wf_dequant(raw_dev.data_ptr(), raw_dev.numel(), qtype, mid, out, res.data_ptr(), n,
                                 native.stream_of(raw_dev.device))
    assert rc == 0, native.last_error()
    torch.cuda.synchronize()
    return res


@pytest.mark.parametrize("qtype", ALL_TYPES)
@pytest.mark.parametrize("family", ["normal", "finite", "edge"])
def test_random_blocks_all_dtypes(native, qtype, family):
    nblk = 4093 if encode.PER_BLOCK[qtype] == 256 else 16381    # not a multiple of any launch tile
    raw = encode.random_blocks(qtype, nblk, seed=1000 + qtype, family=family)
    n = nblk * encode.PER_BLOCK[qtype]
    raw_dev = torch.from_numpy(raw).cuda()
    for mid, out in PAIRS:
        got = _bits(gpu_dequant(native, raw_dev, qtype, mid, out, n), out)
        ref = lib.dequant(raw, qtype, mid, out, n)
        ok, where = _same(got, ref, out)
        assert ok, (qtype, family, mid, out, where)


def test_q8_0_every_scale_and_quant(native):
    d = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    d = d[(d & 0x7C00) != 0x7C00]
    q = np.arange(256, dtype=np.int32).astype(np.int8).view(np.uint8).reshape(8, 32)
    blocks = np.empty((d.size, 8, 34), dtype=np.uint8)
    blocks[:, :, 0:2] = d.view(np.uint8).reshape(-1, 1, 2)
    blocks[:, :, 2:] = q[None]
    raw = blocks.ravel()
    n = d.size * 256
    raw_dev = torch.from_numpy(raw).cuda()
    for mid, out in PAIRS:
        got = _bits(gpu_dequant(native, raw_dev, 8, mid, out, n), out)
        ok, where = _same(got, lib.dequant(raw, 8, mid, out, n), out)
        assert ok, (mid, out, where)


def test_full_size_ffn_weight_q4_k(native):
    w = encode.weights((13824, 5120), seed=1234)
    raw = encode.encode_q4_k(w)
    del w
    raw_dev = torch.from_numpy(raw).cuda()
    got = _bits(gpu_dequant(native, raw_dev, 12, F16, BF16, 13824 * 5120), BF16)
    ref = lib.dequant(raw, 12, F16, BF16, 13824 * 5120)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("qtype", [2, 3, 6, 7, 10, 11, 13, 14])
def test_large_weight_every_format(native, qtype):
    """One 3072 x 5120 weight per format (encoded from N(0, 0.02) weights; Q2_K / Q3_K as random blocks): several
    thousand workgroups of the tiled kernels, MID float16 -> bfloat16, value by value."""
    shape = (3072, 5120)
    if qtype in encode.ENCODERS:
        raw = encode.encode(encode.weights(shape, seed=77), qtype)
    else:
        raw = encode.random_blocks(qtype, shape[0] * shape[1] // 256, seed=77)
    got = _bits(gpu_dequant(native, torch.from_numpy(raw).cuda(), qtype, F16, BF16, shape[0] * shape[1]), BF16)
    assert np.array_equal(got, lib.dequant(raw, qtype, F16, BF16, shape[0] * shape[1]))


def test_dequantize_entry_point(native):
    gd = sub("enhancers.gguf_dequant")
    raw = encode.random_blocks(12, 64, seed=3)
    dev = torch.from_numpy(raw).cuda()
    out = gd.dequantize(dev, 12, (64, 256), None, torch.bfloat16)     # MID defaults to float16
    torch.cuda.synchronize()
    assert out.shape == (64, 256) and out.dtype == torch.bfloat16
    assert np.array_equal(_bits(out, BF16).ravel(), lib.dequant(raw, 12, F16, BF16, 64 * 256))
    out = gd.dequantize(dev, 12, (64, 256), torch.float32, None)       # OUT defaults to MID
    assert out.dtype == torch.float32
    assert np.array_equal(_bits(out, F32).ravel(), lib.dequant(raw, 12, F32, F32, 64 * 256))
    # not this path's case -> None (the host application's code runs)
    assert gd.dequantize(dev.cpu(), 12, (64, 256), None, torch.bfloat16) is None          # CPU data
    assert gd.dequantize(dev, 12, (64, 255), None, torch.bfloat16) is None                 # size mismatch
    assert gd.dequantize(dev, 99, (64, 256), None, torch.bfloat16) is None                 # unknown type
    assert gd.dequantize(dev, 12, (64, 256), torch.int8, torch.bfloat16) is None           # dtype
    big = torch.from_numpy(np.concatenate([np.zeros(8, np.uint8), raw])).cuda()
    assert gd.dequantize(big[8:], 12, (64, 256), None, torch.bfloat16) is None             # not 16-byte aligned
    legacy = encode.random_blocks(8, 64, seed=4)
    out = gd.dequantize(torch.from_numpy(legacy).cuda(), 8, (16, 128), torch.float16, torch.bfloat16)
    assert np.array_equal(_bits(out, BF16).ravel(), lib.dequant(legacy, 8, F16, BF16, 16 * 128))


def test_patched_dequantize_tensor_on_gpu(native, fake_gguf):
    gd = sub("enhancers.gguf_dequant")
    ops = fake_gguf
    assert gd.install(force=True)
    try:
        raw = encode.random_blocks(14, 32, seed=9)
        t = ops.GGMLTensor(torch.from_numpy(raw).cuda(), tensor_type=14, tensor_shape=torch.Size((32, 256)))
        gd.stats(reset=True)
        y = ops.dequantize_tensor(t, torch.bfloat16, None)
        torch.cuda.synchronize()
        assert gd.stats()["used"] == 1 and gd.stats()["fallback"] == 0
        assert np.array_equal(_bits(y, BF16).ravel(), lib.dequant(raw, 14, F16, BF16, 32 * 256))
        y = ops.dequantize_tensor(t, torch.bfloat16, "target")            # MID = the layer dtype
        assert np.array_equal(_bits(y, BF16).ravel(), lib.dequant(raw, 14, BF16, BF16, 32 * 256))
    finally:
        gd.uninstall()
