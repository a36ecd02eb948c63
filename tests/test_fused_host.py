"""Host logic of the GGUF linear drop-in (enhancers/fused_gguf.py): the mode "auto" choice between the fused kernel
and the two-step flow (measured crossover on MI355X), and its routing -- no GPU needed (the kernels are stubbed)."""
import torch

from conftest import sub

fg = sub("enhancers.fused_gguf")


def test_gguf_linear_holds_the_blocks_of_its_format():
    # the raw weight holds whole GGUF blocks: 34 bytes per 32 values for Q8_0, 144 / 176 / 210 per 256 for the
    # K-quants, 18 per 32 for Q4_0, 84 per 256 for Q2_K
    for q, block_bytes, per in ((8, 34, 32), (12, 144, 256), (13, 176, 256), (14, 210, 256), (2, 18, 32), (10, 84, 256)):
        layer = fg.GGUFLinear(5120, 64, q, bias=False)
        assert layer.weight.numel() == 64 * 5120 // per * block_bytes, q


def test_prefer_fused_rule_q8_0():
    # Q8_0 is fused in the library's whole-rows and few-rows forms at 1-64 rows of any width, and in its panel form
    # up to 384 rows (256 for outputs wider than K); beyond the two-step flow is faster
    for rows in (1, 2, 4, 5, 8, 9, 32, 64, 65, 128, 256):
        assert fg.prefer_fused(rows, 8, 5120, 5120) and fg.prefer_fused(rows, 8, 13824, 5120)
        assert fg.prefer_fused(rows, 8, 16353, 5120)
    assert fg.prefer_fused(384, 8, 5120, 5120) and fg.prefer_fused(384, 8, 5120, 13824)
    assert not fg.prefer_fused(384, 8, 13824, 5120)
    for rows in (385, 512, 4096):
        assert not fg.prefer_fused(rows, 8, 5120, 5120)


def test_prefer_fused_rule():
    # few activation rows: the fused kernel streams the weight once
    for rows in (1, 16, 32, 64):
        assert fg.prefer_fused(rows, 12, 5120, 5120)
        assert fg.prefer_fused(rows, 14, 13824, 5120)
    # medium rows: the panel form up to 256 rows, up to 384 for Q5_K and 512 for Q4_K
    for rows in (65, 128, 256):
        for q in (12, 13, 14):
            assert fg.prefer_fused(rows, q, 5120, 5120) and fg.prefer_fused(rows, q, 13824, 5120)
    for rows in (257, 320, 384):
        for q in (12, 13):
            assert fg.prefer_fused(rows, q, 5120, 5120) and fg.prefer_fused(rows, q, 5120, 13824)
            assert not fg.prefer_fused(rows, q, 13824, 5120)            # wide outputs: two-step above 256 rows
        assert not fg.prefer_fused(rows, 14, 5120, 5120)
    for rows in (385, 448, 512):
        assert fg.prefer_fused(rows, 12, 5120, 5120) and fg.prefer_fused(rows, 12, 5120, 13824)
        assert not fg.prefer_fused(rows, 12, 13824, 5120)
        assert not fg.prefer_fused(rows, 13, 5120, 5120) and not fg.prefer_fused(rows, 14, 5120, 5120)
    # from there on the two-step flow is faster for every format and shape
    for rows in (513, 1024, 4096, 8192, 32768):
        for q in (12, 13, 14):
            assert not fg.prefer_fused(rows, q, 5120, 5120) and not fg.prefer_fused(rows, q, 5120, 13824)


def test_auto_routes_by_rows(monkeypatch):
    calls = []

    def fake_fused(x, data, qtype, oshape, bias=None, mid_dtype=None):
        calls.append("fused")
        return torch.zeros(*x.shape[:-1], oshape[0])

    def fake_dequant(data, qtype, oshape, mid_dtype=None, out_dtype=None):
        calls.append("dequant")
        return torch.zeros(oshape, dtype=out_dtype)

    monkeypatch.setattr(fg, "fused_linear", fake_fused)
    monkeypatch.setattr(fg.gguf_dequant, "dequantize", fake_dequant)
    data = torch.zeros(16, dtype=torch.uint8)
    fg.linear(torch.zeros(2, 8, 256, dtype=torch.bfloat16), data, 12, (32, 256))           # 16 rows
    fg.linear(torch.zeros(1, 1024, 256, dtype=torch.bfloat16), data, 12, (32, 256))        # 1024 rows
    fg.linear(torch.zeros(1, 1024, 256, dtype=torch.bfloat16), data, 12, (32, 256), mode="fused")
    fg.linear(torch.zeros(4, 256, dtype=torch.bfloat16), data, 12, (32, 256), mode="dequant")
    assert calls == ["fused", "dequant", "fused", "dequant"]
    layer = fg.GGUFLinear(256, 32, 12, bias=False)
    assert layer.mode == "auto"


def test_hand_gemm_rule():
    # the library's bf16 GEMM takes products whose 256 x 320 tiling gives one to three rounds of 256 workgroups
    assert fg.hand_gemm(4096, 5120) and fg.hand_gemm(4096, 13824) and fg.hand_gemm(8192, 5120)
    assert fg.hand_gemm(4096, 15360)                       # 768 tiles: three rounds
    assert not fg.hand_gemm(2048, 5120)                    # 128 tiles: half the chip idle
    assert not fg.hand_gemm(4096, 16000)                   # 800 tiles
    assert not fg.hand_gemm(16384, 5120) and not fg.hand_gemm(8192, 13824)


def test_bf16_linear_declines_what_its_kernel_does_not_take():
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    w = torch.zeros(8, 64, dtype=torch.bfloat16)
    assert fg.bf16_linear(x, w) is None                    # CPU tensors
    assert fg.bf16_linear(x.float(), w) is None
    assert fg.bf16_linear(x, w.half()) is None


def test_two_step_routes_its_gemm(monkeypatch):
    calls = []

    def fake_dequant(data, qtype, oshape, mid_dtype=None, out_dtype=None):
        return torch.zeros(oshape, dtype=out_dtype)

    def fake_hand(x, w, bias=None):
        calls.append("hand")
        return torch.zeros(*x.shape[:-1], w.shape[0], dtype=x.dtype)

    def fake_torch(x, w, bias=None):
        calls.append("torch")
        return torch.zeros(*x.shape[:-1], w.shape[0], dtype=x.dtype)

    monkeypatch.setattr(fg.gguf_dequant, "dequantize", fake_dequant)
    monkeypatch.setattr(fg, "bf16_linear", fake_hand)
    monkeypatch.setattr(fg.torch.nn.functional, "linear", fake_torch)
    data = torch.zeros(16, dtype=torch.uint8)
    fg.linear(torch.zeros(1, 4096, 256, dtype=torch.bfloat16), data, 12, (5120, 256), mode="dequant")
    fg.linear(torch.zeros(1, 2048, 256, dtype=torch.bfloat16), data, 12, (5120, 256), mode="dequant")
    assert calls == ["hand", "torch"]
