"""GPU parity of the two-step flow's bf16 GEMM through the C ABI (wf_linear_bf16) and of its use by the GGUF linear.

wf_linear_bf16 rounds a float32 accumulation once to bf16, as torch's bf16 GEMM does; the sums run in another order
than any float32 reference, so each output is held to the bf16 rounding of a float32 reference on the GPU: within
2^-8 of its magnitude (half a bf16 ulp) plus 2^-16 of the product's scale for the float32 summation order, and equal
bit for bit to that rounding almost everywhere. Shapes reach every tiling (256 x 320, 256 x 256, 256 x 128,
128 x 160), partial last tiles in M and N, N % 8 != 0 and a 2-byte aligned output (single-value stores), and one,
two, odd and many 128-byte K stages."""
import pytest
import torch

from conftest import sub

pytestmark = pytest.mark.gpu


def gpu_bf16(native, x, w, bias=None, out=None):
    M, K = x.shape
    N = w.shape[0]
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device) if out is None else out
    rc = native.lib().wf_linear_bf16(x.data_ptr(), w.data_ptr(), bias.data_ptr() if bias is not None else None,
                                     y.data_ptr(), M, N, K, native.stream_of(x.device))
    assert rc == 0, native.last_error()
    torch.cuda.synchronize()
    return y


def check_against_f32(y, x, w, bias=None):
    ref = x.float() @ w.float().T
    if bias is not None:
        ref = ref + bias.float()[None, :]
    scale = (x.float().abs() @ w.float().abs().T).max().item()
    err = (y.float() - ref).abs()
    assert bool((err <= ref.abs() * 2.0 ** -8 + scale * 2.0 ** -16).all()), float(err.max())
    same = (y.view(torch.int16) == ref.to(torch.bfloat16).view(torch.int16)).float().mean().item()
    assert same >= 0.995, same


@pytest.mark.parametrize("M,N,K,bias", [
    (4096, 5120, 640, True),      # 256 x 320: one round of 256 tiles, 5 stages
    (4000, 5000, 128, False),     # 256 x 320: partial tiles, N % 8 != 0, one stage
    (4096, 4096, 256, True),      # 256 x 256, two stages
    (2000, 4000, 384, True),      # 256 x 128, an odd last stage
    (3000, 3000, 1024, False),    # 128 x 160
    (1000, 5120, 64, True),       # 128 x 160, half a stage (K = 64)
    (37, 100, 192, True), (1, 8, 64, False), (300, 333, 5120, True)])
def test_bf16_gemm_against_f32(native, M, N, K, bias):
    g = torch.Generator().manual_seed(M + 7 * N + K)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16).cuda()
    w = (torch.randn((N, K), generator=g) * 0.05).to(torch.bfloat16).cuda()
    b = torch.randn(N, generator=g).to(torch.bfloat16).cuda() if bias else None
    check_against_f32(gpu_bf16(native, x, w, b), x, w, b)


def test_bf16_gemm_unaligned_output(native):
    # the output 2 bytes past a 16-byte boundary: whole-run stores are off, every value goes out on its own
    M, N, K = 700, 640, 320
    g = torch.Generator().manual_seed(5)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16).cuda()
    w = torch.randn((N, K), generator=g).to(torch.bfloat16).cuda()
    buf = torch.full((M * N + 8,), float("nan"), dtype=torch.bfloat16, device="cuda")
    y = buf[1:1 + M * N].view(M, N)
    gpu_bf16(native, x, w, out=y)
    check_against_f32(y, x, w)
    assert torch.isnan(buf[0]).item() and bool(torch.isnan(buf[1 + M * N:]).all())


def test_bf16_gemm_wan_shapes_equal_hipblaslt_rounding(native):
    # the Wan-14B block's shapes at 4096 rows: the products the GGUF linear sends to this kernel
    for N, K in ((5120, 5120), (13824, 5120), (5120, 13824)):
        g = torch.Generator().manual_seed(N + K)
        x = torch.randn((4096, K), generator=g).to(torch.bfloat16).cuda()
        w = (torch.randn((N, K), generator=g) * 0.02).to(torch.bfloat16).cuda()
        y = gpu_bf16(native, x, w)
        rows = torch.tensor([0, 1, 255, 256, 2047, 4095])
        check_against_f32(y[rows.cuda()], x[rows.cuda()], w)
        # against torch's bf16 GEMM (hipBLASLt): both round a float32 sum once
        t = torch.nn.functional.linear(x, w).float()
        d = (y.float() - t).abs()
        assert bool((d <= t.abs() * 2.0 ** -7 + 1e-3).all()), float(d.max())
        del x, w, y, t


@pytest.mark.parametrize("rows,takes", [(4096, True), (2048, False)])
def test_gguf_linear_two_step_gemm(native, rows, takes):
    # mode "dequant" (and "auto" above the fused kernel's rows): wf_dequant, then wf_linear_bf16 where its 256 x 320
    # tiling gives one to three rounds of 256 workgroups, torch's GEMM otherwise
    fg = sub("enhancers.fused_gguf")
    enc = sub("gguf_encode")
    gd = sub("enhancers.gguf_dequant")
    N, K = 5120, 1024
    assert fg.hand_gemm(rows, N) is takes
    raw = torch.from_numpy(enc.encode(enc.weights((N, K), seed=3), 12)).cuda()
    x = torch.randn((rows, K), generator=torch.Generator().manual_seed(rows)).to(torch.bfloat16).cuda()
    bias = torch.randn(N, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).cuda()
    y = fg.linear(x, raw, 12, (N, K), bias, mode="dequant")
    w = gd.dequantize(raw, 12, (N, K), None, torch.bfloat16)
    hand = fg.bf16_linear(x, w, bias)
    assert hand is not None
    want = hand if takes else torch.nn.functional.linear(x, w, bias)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), want.view(torch.int16))
    check_against_f32(hand, x, w, bias)
