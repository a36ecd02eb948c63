"""GPU parity of the int8 W8A8 path through the C ABI: wf_quant_rows_i8 (plain and ConvRot) and wf_linear_i8,
bit for bit against the oracle.

Quantiser: bf16 N(0, 1) rows at several widths (incl. the 14B-DiT width 5120), plus zero rows, a row at bf16's
largest value and rows built to hit rint ties. GEMM: ragged small shapes (tails in M, N and K) against the C oracle,
and every workload shape (M in {1024, 4096, 16384}, K = 5120, N in {5120, 13824}) on sampled rows against an exact
float64 accumulator with the epilogue in torch float32 (the same operations as the oracle's epilogue)."""
import numpy as np
import pytest
import torch

from conftest import sub
from oracle import lib

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def gpu_quant(native, x_bf16, mode):
    M, K = x_bf16.shape
    xq = torch.empty((M, K), dtype=torch.int8, device=x_bf16.device)
    xs = torch.empty(M, dtype=torch.float32, device=x_bf16.device)
    rc = native.lib().wf_quant_rows_i8(x_bf16.data_ptr(), M, K, mode, xq.data_ptr(), xs.data_ptr(),
                                       native.stream_of(x_bf16.device))
    assert rc == 0, native.last_error()
    torch.cuda.synchronize()
    return xq, xs


def gpu_linear(native, xq, wq, xs, ws, bias=None, out_dtype=torch.bfloat16):
    M, K = xq.shape
    N = wq.shape[0]
    out = torch.empty((M, N), dtype=out_dtype, device=xq.device)
    code = 1 if out_dtype == torch.bfloat16 else 0
    rc = native.lib().wf_linear_i8(xq.data_ptr(), wq.data_ptr(), xs.data_ptr(), ws.data_ptr(),
                                   bias.data_ptr() if bias is not None else None, out.data_ptr(), code, M, N, K,
                                   native.stream_of(xq.device))
    assert rc == 0, native.last_error()
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("mode,K", [(0, 512), (0, 5120), (0, 8192), (0, 48), (1, 256), (1, 1280), (1, 5120),
                                    (1, 6144),
                                    # rows wider than one wave holds: four waves per row
                                    (0, 8208), (0, 13824), (0, 20480), (0, 32768), (1, 6400), (1, 8192),
                                    (1, 13824), (1, 20480), (1, 32768)])
def test_quant_rows_random(native, mode, K):
    g = torch.Generator().manual_seed(99 + K)
    rows = 257 if K <= 8192 else 67
    x = (torch.randn((rows, K), generator=g) * 2).to(torch.bfloat16)
    # the row maximum in each of the four waves' parts in turn, so a wrong combination of partial maxima shows
    for r in range(4):
        x[r, (K // 4) * r + 3] = 40.0 + r
    xq, xs = gpu_quant(native, x.cuda(), mode)
    rq, rs = lib.quant_rows(x.view(torch.int16).numpy().view(np.uint16), mode)
    assert np.array_equal(xs.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(xq.cpu().numpy(), rq)


@pytest.mark.parametrize("mode", [0, 1])
def test_quant_rows_edges(native, mode):
    K = 512
    rows = np.zeros((6, K), dtype=np.float32)
    rows[1, 0] = 3.3895313892515355e38                     # amax clamp
    rows[1, 1:5] = [-1e38, 1e-38, -7.0, 2.5]
    rows[2, :8] = [127, 2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5]   # ties in plain mode
    rows[3] = np.linspace(-1e-20, 1e-20, K)                # tiny values: scale from amax / 127
    rows[4, ::7] = 1.0
    rows[5] = -np.arange(K) * 0.01
    x = torch.from_numpy(rows).to(torch.bfloat16)
    xq, xs = gpu_quant(native, x.cuda(), mode)
    rq, rs = lib.quant_rows(x.view(torch.int16).numpy().view(np.uint16), mode)
    assert np.array_equal(xs.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(xq.cpu().numpy(), rq)


def _rand_i8(g, shape):
    return torch.randint(-128, 128, shape, generator=g, dtype=torch.int64).to(torch.int8)


@pytest.mark.parametrize("M,N,K", [(64, 64, 128), (77, 93, 256), (130, 258, 5120), (300, 1000, 208),
                                   (512, 640, 1024)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_linear_small_against_oracle(native, M, N, K, out_dtype):
    g = torch.Generator().manual_seed(M * 7 + N)
    xq, wq = _rand_i8(g, (M, K)), _rand_i8(g, (N, K))
    xs = torch.rand(M, generator=g) * 0.05 + 1e-3
    ws = torch.rand(N, generator=g) * 0.002 + 1e-5
    out = gpu_linear(native, xq.cuda(), wq.cuda(), xs.cuda(), ws.cuda(), out_dtype=out_dtype)
    dt = lib.BF16 if out_dtype == torch.bfloat16 else lib.F16
    ref = lib.linear_i8(xq.numpy(), wq.numpy(), xs.numpy(), ws.numpy(), out_dt=dt)
    got = _bits(out)
    bad = np.argwhere(got != ref)
    assert bad.size == 0, f"{len(bad)} mismatches, first (m, n): {bad[:6].tolist()}"


def test_linear_bias(native):
    g = torch.Generator().manual_seed(5)
    M, N, K = 96, 160, 512
    xq, wq = _rand_i8(g, (M, K)), _rand_i8(g, (N, K))
    xs, ws = torch.rand(M, generator=g) * 0.05, torch.rand(N, generator=g) * 0.002
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    out = gpu_linear(native, xq.cuda(), wq.cuda(), xs.cuda(), ws.cuda(), bias=bias.cuda())
    ref = lib.linear_i8(xq.numpy(), wq.numpy(), xs.numpy(), ws.numpy(), out_dt=lib.BF16,
                        bias=bias.view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(_bits(out), ref)


@pytest.mark.parametrize("M", [1024, 4096, 16384])
@pytest.mark.parametrize("N", [5120, 13824])
def test_linear_workload_shapes_sampled_rows(native, M, N):
    K = 5120
    g = torch.Generator().manual_seed(M + N)
    xq = _rand_i8(g, (M, K))
    wq = _rand_i8(g, (N, K))
    xs = torch.rand(M, generator=g) * 0.05 + 1e-3
    ws = torch.rand(N, generator=g) * 0.002 + 1e-5
    out = gpu_linear(native, xq.cuda(), wq.cuda(), xs.cuda(), ws.cuda())
    rows = torch.unique(torch.cat([torch.arange(0, M, max(1, M // 48)), torch.tensor([M - 1, 31, 32, 255, 256])]))
    rows = rows[rows < M]
    acc = xq[rows].double() @ wq.double().T                       # exact: |acc| < 2^31
    ref = ((acc.float() * xs[rows, None]) * ws[None, :]).to(torch.bfloat16)
    got = out[rows.cuda()].cpu()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


# ------------------------------------------------------------------------------------- drop-in entry points
def test_shared_forward_qkv_share_one_quantisation(native):
    from fake_quant import FakeQT, Lin
    fi = sub("enhancers.fused_int8")
    fs = sub("enhancers.fused_state")
    fs.stats(reset=True)
    g = torch.Generator().manual_seed(11)
    K = 5120
    x = (torch.randn((2, 300, K), generator=g)).to(torch.bfloat16).cuda()
    lins, ref = [], []
    for n in (5120, 5120, 1024):
        w_q = torch.randint(-127, 128, (n, K), generator=g, dtype=torch.int64).to(torch.int8)
        ws = torch.rand(n, generator=g) * 0.01
        lins.append(Lin(FakeQT(w_q.cuda(), ws.cuda())))
        ref.append((w_q, ws))
    calls = []
    orig = fi.quantise_rows
    fi.quantise_rows = lambda *a: calls.append(1) or orig(*a)
    try:
        with fi._Overrides(lins):
            ys = [lin(x) for lin in lins]
    finally:
        fi.quantise_rows = orig
    torch.cuda.synchronize()
    assert len(calls) == 1 and fs.stats()["qkv"]["used"] == 3
    xq, xs = lib.quant_rows(x.reshape(-1, K).cpu().view(torch.int16).numpy().view(np.uint16), 1)
    for y, (w_q, ws) in zip(ys, ref):
        assert y.shape == (2, 300, w_q.shape[0])
        expect = lib.linear_i8(xq, w_q.numpy(), xs, ws.numpy(), out_dt=lib.BF16)
        assert np.array_equal(_bits(y.reshape(600, -1)), expect)


def test_residual_forward_matches_oracle(native):
    from fake_quant import FakeQT
    fi = sub("enhancers.fused_int8")
    g = torch.Generator().manual_seed(12)
    B, T, H, W, D = 2, 2, 4, 8, 1024
    x = torch.randn((B, T, H, W, D), generator=g).to(torch.bfloat16).cuda()
    w_q = torch.randint(-127, 128, (D, D), generator=g, dtype=torch.int64).to(torch.int8)
    ws = torch.rand(D, generator=g) * 0.01
    xres = torch.randn((B, T, H, W, D), generator=g).to(torch.bfloat16).cuda()
    gate = torch.randn((B, T, 1, 1, D), generator=g).to(torch.bfloat16).cuda()
    fi._tls.res = {"x": xres, "gate": gate, "done": False}
    try:
        with fi._Overrides([]):
            y = fi._residual_forward(x, FakeQT(w_q.cuda(), ws.cuda()), None)
    finally:
        fi._tls.res = None
    torch.cuda.synchronize()
    xq, xs = lib.quant_rows(x.reshape(-1, D).cpu().view(torch.int16).numpy().view(np.uint16), 1)
    expect = lib.linear_i8_residual(xq, w_q.numpy(), xs, ws.numpy(),
                                    gate.reshape(B * T, D).cpu().view(torch.int16).numpy().view(np.uint16),
                                    xres.reshape(-1, D).cpu().view(torch.int16).numpy().view(np.uint16), H * W)
    assert y.shape == xres.shape
    assert np.array_equal(_bits(y.reshape(-1, D)), expect)


@pytest.mark.parametrize("M,N", [(1024, 5120), (300, 13824)])
def test_int8_linear_plain_per_token(native, M, N):
    fi = sub("enhancers.fused_int8")
    K = 5120
    g = torch.Generator().manual_seed(M)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    w = torch.randn((N, K), generator=g) * 0.02
    ws = (w.abs().amax(dim=1) / 127).float()
    w_q = torch.clamp(torch.round(w / ws[:, None]), -127, 127).to(torch.int8)
    y = fi.int8_linear(x.cuda(), w_q.cuda(), ws.cuda(), convrot=False)
    torch.cuda.synchronize()
    xq, xs = lib.quant_rows(x.view(torch.int16).numpy().view(np.uint16), 0)
    expect = lib.linear_i8(xq, w_q.numpy(), xs, ws.numpy(), out_dt=lib.BF16)
    assert np.array_equal(_bits(y), expect)


# ------------------------------------------------------------------------------ quantiser operations (PRE)
def _gelu_table_bits():
    table = torch.nn.functional.gelu(torch.arange(65536, dtype=torch.int32, device="cuda").to(torch.int16)
                                     .view(torch.bfloat16))
    return table, _bits(table)


def gpu_quant_pre(native, x, pre, s=None, h=None, rows=1, eps=0.0):
    M, K = x.shape
    xq = torch.empty((M, K), dtype=torch.int8, device="cuda")
    xs = torch.empty(M, dtype=torch.float32, device="cuda")
    rc = native.lib().wf_quant_rows_i8_pre(x.data_ptr(), M, K, pre, s.data_ptr() if s is not None else None,
                                           h.data_ptr() if h is not None else None, rows, eps, xq.data_ptr(),
                                           xs.data_ptr(), native.stream_of(x.device))
    assert rc == 0, native.last_error()
    torch.cuda.synchronize()
    return xq, xs


@pytest.mark.parametrize("pre", [0, 1, 2, 3])
@pytest.mark.parametrize("K,groups,rows", [(1024, 3, 5), (5120, 2, 64), (6144, 1, 7), (8192, 2, 9),
                                           (13824, 3, 4), (20480, 1, 6)])
def test_quant_rows_pre_against_oracle(native, pre, K, groups, rows):
    g = torch.Generator().manual_seed(pre * 100 + K)
    x = (torch.randn((groups * rows, K), generator=g) * 1.5).to(torch.bfloat16)
    x[0] = 0.75                                         # a constant row (LayerNorm variance 0)
    scale = (torch.randn((groups, K), generator=g) * 0.3).to(torch.bfloat16)
    shift = (torch.randn((groups, K), generator=g) * 0.5).to(torch.bfloat16)
    s1 = 1 + scale
    print(f"case pre={pre} K={K} groups={groups} rows={rows}", flush=True)
    if pre == 1:
        table, tbits = _gelu_table_bits()
        xq, xs = gpu_quant_pre(native, x.cuda(), 1, table)
        rq, rs = lib.quant_rows_pre(_bits(x), 1, tbits)
    elif pre >= 2:
        xq, xs = gpu_quant_pre(native, x.cuda(), pre, s1.cuda(), shift.cuda(), rows, 1e-6)
        rq, rs = lib.quant_rows_pre(_bits(x), pre, _bits(s1), _bits(shift), rows, 1e-6)
    else:
        xq, xs = gpu_quant_pre(native, x.cuda(), 0)
        rq, rs = lib.quant_rows_pre(_bits(x), 0)
    assert np.array_equal(xs.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    bad = np.argwhere(xq.cpu().numpy() != rq)
    assert bad.size == 0, bad[:8].tolist()


@pytest.mark.parametrize("kind,K", [("mod", 5120), ("gelu", 5120), ("lnmod", 4096), ("mod", 13824),
                                    ("gelu", 20480), ("lnmod", 8192)])
def test_pending_input_quantised_with_its_operation(native, kind, K):
    from fake_quant import FakeQT, Lin
    fi = sub("enhancers.fused_int8")
    fs = sub("enhancers.fused_state")
    fs.stats(reset=True)
    g = torch.Generator().manual_seed(21)
    B, N = 2, 160
    src = (torch.randn((B, N, K), generator=g)).to(torch.bfloat16).cuda()
    scale = (torch.randn((B, 1, K), generator=g) * 0.2).to(torch.bfloat16).cuda()
    shift = (torch.randn((B, 1, K), generator=g) * 0.2).to(torch.bfloat16).cuda()
    norm = torch.nn.LayerNorm(K, elementwise_affine=False, eps=1e-6)
    w_q = torch.randint(-127, 128, (640, K), generator=g, dtype=torch.int64).to(torch.int8)
    ws = torch.rand(640, generator=g) * 0.01
    lin = Lin(FakeQT(w_q.cuda(), ws.cuda()))
    with fi._Overrides([lin]):
        if kind == "gelu":
            fi._set_pre(src, "gelu")
        else:
            fi._set_pre(src, kind, scale, shift, norm=norm if kind == "lnmod" else None)
        y = lin(src)
        fi._clear_pre()
    torch.cuda.synchronize()
    part = {"gelu": "gelu", "lnmod": "ln"}.get(kind, "modq")
    assert fs.stats()[part]["used"] == 1, fs.stats()
    xb = _bits(src.reshape(-1, K))
    if kind == "gelu":
        rq, rs = lib.quant_rows_pre(xb, 1, _gelu_table_bits()[1])
    else:
        rq, rs = lib.quant_rows_pre(xb, 2 if kind == "mod" else 3, _bits((1 + scale).reshape(B, K)),
                                    _bits(shift.reshape(B, K)), N, 1e-6)
    expect = lib.linear_i8(rq, w_q.numpy(), rs, ws.numpy(), out_dt=lib.BF16)
    assert np.array_equal(_bits(y.reshape(-1, 640)), expect)


@pytest.mark.parametrize("M,N,K", [(4000, 5000, 512), (4000, 4992, 512), (4000, 5000, 640), (4000, 4992, 128),
                                   (4000, 5000, 576), (3000, 3000, 384), (2000, 4000, 640),
                                   (1024, 5000, 512), (1000, 5120, 512),
                                   (1000, 5120, 576), (1024, 4992, 128), (1000, 5000, 640), (1024, 5120, 896),
                                   (4096, 8192, 80), (300, 1000, 208)])
def test_tilings_bias_and_residual_whole_output(native, M, N, K):
    # 4000 x N outputs take the 256 x 320 tiling (one round of 256 workgroups), 3000 x 3000 the 256 x 256 one,
    # 2000 x 4000 the 256 x 128 one, 1024 x 5000 and 1000 x 5120 the 128 x 160 one (256 tiles); N = 5000 leaves a
    # partial last tile and an odd row length (element stores), N = 4992 and 5120 whole 16-byte runs, M = 1000 a
    # partial last tile-row. With K % 128 == 0 the 256-row tilings stream whole 128-byte lines through two stage
    # buffers (K = 128: one stage; 512: two whole pairs; 384 and 640: an odd last stage) and the 128 x 160 tiling
    # 128-byte stages through its 4-stage ring (128: one stage; 512: whole rounds of the ring; 640 and 896: one and
    # three stages after them); K = 576 takes the 64-byte ring in both. K % 64 != 0 takes the register-staged
    # kernel: 256 x 256 tiles for 4096 x 8192 (512 of them), 128 x 128 for 300 x 1000. Every element of the bias and
    # the residual forms against the float32 epilogue in the kernel's order on an exact accumulator (|acc| <= 896 *
    # 127^2 < 2^24).
    G = 4
    g = torch.Generator().manual_seed(N + M)
    xq, wq = _rand_i8(g, (M, K)), _rand_i8(g, (N, K))
    xs = torch.rand(M, generator=g) * 0.05 + 1e-3
    ws = torch.rand(N, generator=g) * 0.002 + 1e-5
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    acc = (xq.double() @ wq.double().T).float()                   # exact: |acc| < 2^24 here
    t = (acc * xs[:, None]) * ws[None, :]
    out = gpu_linear(native, xq.cuda(), wq.cuda(), xs.cuda(), ws.cuda(), bias=bias.cuda()).cpu()
    ref = (t + bias.float()[None, :]).to(torch.bfloat16)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    gate = torch.randn((G, N), generator=g).to(torch.bfloat16)
    resid = torch.randn((M, N), generator=g).to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    d = {k: v.cuda() for k, v in dict(xq=xq, wq=wq, xs=xs, ws=ws, gate=gate, resid=resid).items()}
    rc = native.lib().wf_linear_i8_residual(d["xq"].data_ptr(), d["wq"].data_ptr(), d["xs"].data_ptr(),
                                            d["ws"].data_ptr(), d["gate"].data_ptr(), d["resid"].data_ptr(),
                                            y.data_ptr(), M, N, K, M // G, native.stream_of(torch.device("cuda")))
    assert rc == 0, native.last_error()
    torch.cuda.synchronize()
    gr = gate.float().repeat_interleave(M // G, dim=0)
    ref_r = (resid.float() + gr * t.to(torch.bfloat16).float()).to(torch.bfloat16)
    assert torch.equal(y.cpu().view(torch.int16), ref_r.view(torch.int16))


def test_pending_layernorm_at_a_width_that_is_not_a_power_of_two_is_materialised(native):
    # LayerNorm is fused only where torch's own kernel splits rows like the restatement (powers of two): at 5120
    # the layer quantises the real input (torch's layer_norm, then the scale-and-shift), counted as an "ln" fallback
    from fake_quant import FakeQT, Lin
    fi = sub("enhancers.fused_int8")
    fs = sub("enhancers.fused_state")
    fs.stats(reset=True)
    g = torch.Generator().manual_seed(22)
    B, N, K = 2, 96, 5120
    src = torch.randn((B, N, K), generator=g).to(torch.bfloat16).cuda()
    scale = (torch.randn((B, 1, K), generator=g) * 0.2).to(torch.bfloat16).cuda()
    shift = (torch.randn((B, 1, K), generator=g) * 0.2).to(torch.bfloat16).cuda()
    norm = torch.nn.LayerNorm(K, elementwise_affine=False, eps=1e-6)
    w_q = torch.randint(-127, 128, (256, K), generator=g, dtype=torch.int64).to(torch.int8)
    ws = torch.rand(256, generator=g) * 0.01
    lin = Lin(FakeQT(w_q.cuda(), ws.cuda()))
    with fi._Overrides([lin]):
        pre = fi._set_pre(src, "lnmod", scale, shift, norm=norm)
        y = lin(src)
        fi._clear_pre()
    torch.cuda.synchronize()
    assert pre["used"] and fs.stats()["ln"]["fallback"] == 1 and fs.stats()["qkv"]["used"] == 1
    real = norm(src) * (1 + scale) + shift
    rq, rs = lib.quant_rows(_bits(real.reshape(-1, K)), 1)
    expect = lib.linear_i8(rq, w_q.numpy(), rs, ws.numpy(), out_dt=lib.BF16)
    assert np.array_equal(_bits(y.reshape(-1, 256)), expect)
