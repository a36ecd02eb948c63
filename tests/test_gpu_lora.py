"""GPU parity of the LoRA add (wf_dequant_add, the role of the reference's _deq_add, enhancers/gguf_dequant.py:
99-133) against the oracle, bit for bit: the first LoRA fused into the dequantisation for every format and every
MID / OUT pair, later LoRAs onto an existing weight (ragged tail included), and the drop-in Python path
(dequantize_lora, the patched get_weight) with two LoRAs whose differences come from the same torch.mm."""
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
        return t.numpy().astype(np.float32).ravel()
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).ravel()


def _same(a, b, D):
    fa, fb = np_oracle.bits_to_f32(a, D), np_oracle.bits_to_f32(b, D)
    eq = np.asarray(a).view(np.uint8).reshape(fa.size, -1) == np.asarray(b).view(np.uint8).reshape(fb.size, -1)
    ok = eq.all(axis=1) | (np.isnan(fa) & np.isnan(fb))
    return bool(ok.all()), np.nonzero(~ok)[0][:8]


@pytest.mark.parametrize("qtype", ALL_TYPES)
def test_first_lora_fused_into_dequant(native, qtype):
    nblk = 2047 if encode.PER_BLOCK[qtype] == 256 else 8191
    n = nblk * encode.PER_BLOCK[qtype]
    raw = encode.random_blocks(qtype, nblk, seed=500 + qtype, family="normal")
    diff = (np.random.default_rng(qtype).standard_normal(n) * 0.02).astype(np.float32)
    raw_dev, diff_dev = torch.from_numpy(raw).cuda(), torch.from_numpy(diff).cuda()
    for mid, out in PAIRS:
        res = torch.empty(n, dtype=TD[out], device="cuda")
        print(f"case qtype={qtype} mid={mid} out={out} n={n}", flush=True)
        rc = native.lib().wf_dequant_add(raw_dev.data_ptr(), raw_dev.numel(), qtype, mid, out, diff_dev.data_ptr(),
                                         0.4375, res.data_ptr(), n, native.stream_of(res.device))
        assert rc == 0, native.last_error()
        torch.cuda.synchronize()
        ok, where = _same(_bits(res, out), lib.dequant_add(raw, qtype, mid, out, diff, 0.4375), out)
        assert ok, (qtype, mid, out, where)


@pytest.mark.parametrize("out", [F16, BF16, F32])
@pytest.mark.parametrize("n", [8, 1_000_003, 5120 * 5120])
def test_later_lora_onto_weight(native, out, n):
    rng = np.random.default_rng(n + out)
    w = torch.from_numpy(rng.standard_normal(n).astype(np.float32) * 0.05).to(TD[out])
    diff = (rng.standard_normal(n) * 0.01).astype(np.float32)
    base = _bits(w, out)
    wd, dd = w.cuda(), torch.from_numpy(diff).cuda()
    print(f"case out={out} n={n}", flush=True)
    rc = native.lib().wf_dequant_add(None, 0, 0, 0, out, dd.data_ptr(), -1.25, wd.data_ptr(), n,
                                     native.stream_of(wd.device))
    assert rc == 0, native.last_error()
    torch.cuda.synchronize()
    ok, where = _same(_bits(wd, out), lib.dequant_add(None, 0, 0, out, diff, -1.25, base=base), out)
    assert ok, where


class LoRAAdapter:
    def __init__(self, weights):
        self.weights = weights


def _patch(up, down, alpha, strength):
    return (strength, LoRAAdapter((up, down, alpha, None, None, None)), 1.0, None, None)


def _expected(raw, qtype, mid, out, n_out, n_in, loras):
    """the oracle's chain with each difference from the same torch.mm the drop-in calls (float32 on the GPU)"""
    res = None
    for i, (up, down, sa) in enumerate(loras):
        diff = torch.mm(up.to("cuda", torch.float32), down.to("cuda", torch.float32)).cpu().numpy().ravel()
        if i == 0:
            res = lib.dequant_add(raw, qtype, mid, out, diff, sa)
        else:
            res = lib.dequant_add(None, 0, 0, out, diff, sa, base=res)
    return res


@pytest.mark.parametrize("qtype,mid", [(8, torch.float16), (12, torch.float16), (14, torch.bfloat16), (3, None)])
def test_dequantize_lora_two_loras(native, qtype, mid):
    gd = sub("enhancers.gguf_dequant")
    n_out, n_in = 384, 1024
    if qtype in encode.ENCODERS:
        raw = encode.encode(encode.weights((n_out, n_in), seed=qtype), qtype)
    else:
        raw = encode.random_blocks(qtype, n_out * n_in // encode.PER_BLOCK[qtype], seed=qtype, family="normal")
    g = torch.Generator().manual_seed(qtype)
    ups = [torch.randn((n_out, 16), generator=g).to(torch.bfloat16), torch.randn((n_out, 8), generator=g)]
    downs = [torch.randn((16, n_in), generator=g).to(torch.bfloat16), torch.randn((8, n_in), generator=g)]
    loras = gd.lora_factors([_patch(ups[0], downs[0], 8.0, 0.7), _patch(ups[1], downs[1], None, -0.3)], n_out, n_in)
    y = gd.dequantize_lora(torch.from_numpy(raw).cuda(), qtype, (n_out, n_in), mid, torch.bfloat16, loras)
    torch.cuda.synchronize()
    assert y.shape == (n_out, n_in) and y.dtype == torch.bfloat16
    m = {None: F16, torch.float16: F16, torch.bfloat16: BF16}[mid]
    expect = _expected(raw, qtype, m, BF16, n_out, n_in, loras)
    ok, where = _same(_bits(y, BF16), expect, BF16)
    assert ok, where
    # not this path's case: CPU data, no LoRA, a 1-D shape
    assert gd.dequantize_lora(torch.from_numpy(raw), qtype, (n_out, n_in), mid, torch.bfloat16, loras) is None
    assert gd.dequantize_lora(torch.from_numpy(raw).cuda(), qtype, (n_out, n_in), mid, torch.bfloat16, []) is None
    assert gd.dequantize_lora(torch.from_numpy(raw).cuda(), qtype, (n_out * n_in,), mid, torch.bfloat16, loras) is None


def test_patched_get_weight_with_lora(native, fake_gguf):
    gd = sub("enhancers.gguf_dequant")
    ops = fake_gguf
    assert gd.install(force=True)
    try:
        n_out, n_in = 256, 512
        raw = encode.encode(encode.weights((n_out, n_in), seed=3), 13)
        g = torch.Generator().manual_seed(3)
        up, down = torch.randn((n_out, 4), generator=g), torch.randn((4, n_in), generator=g)
        t = ops.GGMLTensor(torch.from_numpy(raw).cuda(), tensor_type=13, tensor_shape=torch.Size((n_out, n_in)),
                           patches=[([_patch(up, down, 2.0, 0.5)], "key")])
        gd.stats(reset=True)
        y = ops.GGMLLayer().get_weight(t, torch.bfloat16)
        torch.cuda.synchronize()
        assert gd.stats().get("lora_used") == 1
        loras = gd.lora_factors([_patch(up, down, 2.0, 0.5)], n_out, n_in)
        ok, where = _same(_bits(y, BF16), _expected(raw, 13, F16, BF16, n_out, n_in, loras), BF16)
        assert ok, where
    finally:
        gd.uninstall()


def test_inference_mode_factors_use_the_kernel(native, fake_gguf):
    # ComfyUI runs under torch.inference_mode and its LoRA factors are inference tensors (no version counter): the
    # pinned-factor path must take them (lora_used), reuse their page-locked copies on the next call, and give the
    # same bits as the oracle's chain
    gd = sub("enhancers.gguf_dequant")
    ops = fake_gguf
    assert gd.install(force=True)
    try:
        n_out, n_in = 256, 512
        raw = encode.encode(encode.weights((n_out, n_in), seed=4), 12)
        g = torch.Generator().manual_seed(4)
        with torch.inference_mode():
            up, down = torch.randn((n_out, 8), generator=g), torch.randn((8, n_in), generator=g)
            t = ops.GGMLTensor(torch.from_numpy(raw).cuda(), tensor_type=12, tensor_shape=torch.Size((n_out, n_in)),
                               patches=[([_patch(up, down, 4.0, 0.75)], "key")])
            gd.stats(reset=True)
            held_before = len(gd._PINNED)
            ys = [ops.GGMLLayer().get_weight(t, torch.bfloat16) for _ in range(2)]
            torch.cuda.synchronize()
        assert gd.stats().get("lora_used") == 2 and "lora_fallback" not in gd.stats()
        assert len(gd._PINNED) == held_before + 2          # one page-locked copy per factor, reused by the 2nd call
        loras = gd.lora_factors([_patch(up, down, 4.0, 0.75)], n_out, n_in)
        expect = _expected(raw, 12, F16, BF16, n_out, n_in, loras)
        for y in ys:
            ok, where = _same(_bits(y, BF16), expect, BF16)
            assert ok, where
    finally:
        gd.uninstall()
