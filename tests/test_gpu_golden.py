"""The gfx950 kernels against the committed golden fixtures of tests/golden/, through the C ABI, bit for bit."""
import os

import numpy as np
import pytest
import torch

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TS = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34, 10: 84, 11: 110, 12: 144, 13: 176, 14: 210}
PER_BLOCK = {2: 32, 3: 32, 6: 32, 7: 32, 8: 32, 10: 256, 11: 256, 12: 256, 13: 256, 14: 256}
TD = {0: torch.float16, 1: torch.bfloat16, 2: torch.float32}

pytestmark = pytest.mark.gpu


def _load(name):
    with np.load(os.path.join(G, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _bits(t, o):
    t = t.cpu()
    return t.numpy().astype(np.float32) if o == 2 else t.view(torch.int16).numpy().view(np.uint16)


def _same(a, b):
    if a.dtype == np.float32:
        return bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))
    return np.array_equal(a, b)


@pytest.mark.parametrize("qtype", sorted(PER_BLOCK))
def test_dequant_kernels_match_fixtures(native, qtype):
    d = _load("dequant.npz")
    raw = torch.from_numpy(d[f"raw_{qtype}"]).cuda()
    n = raw.numel() // TS[qtype] * PER_BLOCK[qtype]
    for m in range(3):
        for o in range(3):
            out = torch.empty(n, dtype=TD[o], device="cuda")
            rc = native.lib().wf_dequant(raw.data_ptr(), raw.numel(), qtype, m, o, out.data_ptr(), n,
                                         native.stream_of(raw.device))
            assert rc == 0, native.last_error()
            torch.cuda.synchronize()
            assert _same(_bits(out, o), d[f"out_{qtype}_{m}_{o}"]), (qtype, m, o)


def test_quantiser_and_int8_linear_match_fixtures(native):
    q = _load("quant_rows.npz")
    x = torch.from_numpy(q["x"].view(np.int16)).cuda()
    M, K = x.shape
    st = native.stream_of(x.device)
    for mode in (0, 1):
        xq = torch.empty((M, K), dtype=torch.int8, device="cuda")
        xs = torch.empty(M, dtype=torch.float32, device="cuda")
        rc = native.lib().wf_quant_rows_i8(x.data_ptr(), M, K, mode, xq.data_ptr(), xs.data_ptr(), st)
        assert rc == 0, native.last_error()
        torch.cuda.synchronize()
        assert np.array_equal(xq.cpu().numpy(), q[f"q_{mode}"]) and _same(xs.cpu().numpy(), q[f"s_{mode}"]), mode
    z = _load("linear_i8.npz")
    xq, wq = torch.from_numpy(z["xq"]).cuda(), torch.from_numpy(z["wq"]).cuda()
    xs, ws = torch.from_numpy(z["xs"]).cuda(), torch.from_numpy(z["ws"]).cuda()
    M, K = z["xq"].shape
    N = z["wq"].shape[0]
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    rc = native.lib().wf_linear_i8(xq.data_ptr(), wq.data_ptr(), xs.data_ptr(), ws.data_ptr(), None, y.data_ptr(), 1,
                                   M, N, K, st)
    assert rc == 0, native.last_error()
    torch.cuda.synchronize()
    assert np.array_equal(_bits(y, 1), z["y"])


def test_convrot_kernel_keeps_the_stage_sum_order(native):
    # rows whose int8 values change under any other order of a radix-4 stage's sums (tests/golden/make_golden.py)
    z = _load("convrot_order.npz")
    x = torch.from_numpy(z["x"].view(np.int16)).cuda()
    M, K = x.shape
    xq = torch.empty((M, K), dtype=torch.int8, device="cuda")
    xs = torch.empty(M, dtype=torch.float32, device="cuda")
    rc = native.lib().wf_quant_rows_i8(x.data_ptr(), M, K, 1, xq.data_ptr(), xs.data_ptr(), native.stream_of(x.device))
    assert rc == 0, native.last_error()
    torch.cuda.synchronize()
    assert np.array_equal(xq.cpu().numpy(), z["q"]) and _same(xs.cpu().numpy(), z["s"])
