"""GPU check of wf_linear_gguf (fused K-quant dequant + bf16 MFMA GEMM) through the C ABI.

Reference: a float64 GEMM of the same bf16 activations with the oracle's bit-exact dequantised bf16 weight (the
reference path: dequantize, then F.linear in bf16). The tolerance is the task's bound for bf16 GEMMs, max relative error
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
@pytest.mark.parametrize("M,N,K", [(77, 300, 512), (256, 256, 256), (512, 768, 5120), (2100, 300, 512)])
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


@pytest.mark.parametrize("qtype,N,K", [(13, 5120, 5120), (14, 5120, 5120), (13, 5120, 13824), (14, 13824, 5120),
                                        (12, 5120, 13824)])
def test_wan_block_shapes_whole_output(native, qtype, N, K):
    # every one of the 4096 x N outputs of a Wan block layer at full K (random blocks of realistic scales), against a
    # float32 GEMM on the GPU of the same bf16 activations with the oracle's dequantised bf16 weight; the same bounds
    # as check()
    M = 4096
    raw = encode.random_blocks(qtype, N * K // 256, seed=N + K + qtype, family="normal")
    g = torch.Generator().manual_seed(99)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16).cuda()
    print(f"case wan whole output qtype={qtype} M={M} N={N} K={K}", flush=True)
    y = fused(native, x, torch.from_numpy(raw).cuda(), qtype, N)
    w = weight_bf16(raw, qtype, 0, N, K).cuda()
    torch.backends.cuda.matmul.allow_tf32 = False
    ref = x.float() @ w.T
    del w
    scale = ref.abs().max().item()
    err = (y.float() - ref).abs()
    assert err.max().item() / scale <= 1e-2
    over = err - (ref.abs() * 2.0 ** -8 + 1e-3 * scale)
    assert over.max().item() <= 0, (over.max().item(), torch.nonzero(over > 0)[:4].tolist())


def check_gpu(y, x, w, bias=None):
    """check()'s bounds against a float32 GEMM on the GPU (for outputs too large for a CPU float64 reference)"""
    torch.backends.cuda.matmul.allow_tf32 = False
    ref = x.float() @ w.cuda().T
    if bias is not None:
        ref = ref + bias.float()[None, :]
    scale = ref.abs().max().item()
    err = (y.float() - ref).abs()
    assert err.max().item() / scale <= 1e-2
    over = err - (ref.abs() * 2.0 ** -8 + 1e-3 * scale)
    assert over.max().item() <= 0, (over.max().item(), torch.nonzero(over > 0)[:4].tolist())


@pytest.mark.parametrize("M,N,K,with_bias,mid,offset", [(2048, 8999, 768, False, 0, 0), (2100, 8000, 256, True, 2, 0),
                                                        (4100, 8000, 512, True, 1, 1), (3333, 5120, 1280, False, 0, 0),
                                                        (4096, 5120, 512, False, 0, 1)])
def test_q6k_tall_form_whole_output(native, M, N, K, with_bias, mid, offset):
    # Q6_K from 1024 rows, where 512 x 160 tiles take no more modelled rounds than 256-row tiles, goes to the tall form
    # (each dequantised weight value feeds 512 rows; activations as whole 128-byte lines): ragged M past a 512-row
    # tile, ragged N past a 160-row tile and N % 8 != 0 (element stores), bias, every MID, and an output view one
    # element past an aligned start (element stores); every output element checked
    qtype = 14
    raw = encode.random_blocks(qtype, N * K // 256, seed=M + N + K, family="normal")
    g = torch.Generator().manual_seed(M * 3 + N)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16).cuda()
    bias = torch.randn(N, generator=g).to(torch.bfloat16).cuda() if with_bias else None
    flat = torch.empty(M * N + 8, dtype=torch.bfloat16, device="cuda")
    y = flat[offset:offset + M * N].view(M, N)
    print(f"case tall qtype=14 M={M} N={N} K={K} mid={mid} offset={offset}", flush=True)
    rd = torch.from_numpy(raw).cuda()
    rc = native.lib().wf_linear_gguf(x.data_ptr(), M, K, rd.data_ptr(), rd.numel(), qtype, N,
                                     bias.data_ptr() if bias is not None else None, y.data_ptr(), mid,
                                     native.stream_of(x.device))
    assert rc == 0, native.last_error()
    torch.cuda.synchronize()
    check_gpu(y, x, weight_bf16(raw, qtype, mid, N, K), bias=bias)


@pytest.mark.parametrize("qtype", [12, 13, 14, 8])
@pytest.mark.parametrize("mid", [0, 2])
@pytest.mark.parametrize("M,N,K,with_bias", [(1, 300, 256, True), (5, 5120, 5120, False), (16, 61, 512, True),
                                             (17, 1000, 1024, False), (33, 300, 2048, True), (64, 5120, 512, False),
                                             (48, 777, 1280, True), (65, 256, 768, False),
                                             (4, 777, 1280, False), (12, 777, 1280, True)])
def test_few_rows_whole_output(native, qtype, mid, M, N, K, with_bias):
    # up to 64 activation rows take the few-rows kernel (32 weight rows per workgroup, K split over its 8 waves,
    # 1 to 4 row tiles of 16; K = 256 and 512 leave waves with no super-block); 65 rows the panel kernel: ragged M
    # and N, every output element checked. 777 x 1280: the last workgroup's last weight row ends with a Q6_K block
    # that starts on a dword (the buffer range check ends at that row). Q8_0 takes the few-rows kernel from 5 rows (1-4
    # rows of outputs narrower than 16384: the whole-rows form), the panel form at 65
    raw = encode.random_blocks(qtype, nblocks(qtype, N, K), seed=qtype * 7 + M, family="normal")
    g = torch.Generator().manual_seed(M * 31 + N)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    bias = torch.randn(N, generator=g).to(torch.bfloat16) if with_bias else None
    y = fused(native, x.cuda(), torch.from_numpy(raw).cuda(), qtype, N, bias=bias.cuda() if with_bias else None,
              mid=mid)
    check(y, x, weight_bf16(raw, qtype, mid, N, K), bias=bias)


def nblocks(qtype, N, K):
    return N * K // (32 if qtype == 8 else 256)


@pytest.mark.parametrize("qtype,mid", [(12, 0), (13, 0), (14, 0), (8, 0), (12, 2), (13, 1), (14, 2), (8, 1)])
@pytest.mark.parametrize("M,N,K,with_bias", [(1, 5120, 5120, True), (2, 5120, 13824, False), (1, 8000, 5120, True),
                                             (2, 4101, 1280, True), (1, 61, 256, False), (2, 1, 768, True),
                                             (1, 1000, 2304, False), (1, 13824, 5120, True), (2, 9001, 512, False),
                                             (3, 5120, 1280, True), (4, 13000, 768, False), (1, 16400, 512, True)])
def test_whole_rows_form_whole_output(native, qtype, mid, M, N, K, with_bias):
    # K-quants at one to three rows of an output narrower than 8192 (Q6_K and Q8_0: up to four rows and 16384 wide,
    # on 512 workgroups from 8192; the other shapes, and 16400 rows, take the few-rows kernel): each
    # workgroup takes whole quads of 4 weight rows, the MFMA's 16 columns holding 4 rows x 4 parts of K. The Wan
    # shapes (5120 rows: 20 per CU; 13824: 54 super-blocks in parts of 14, the last part 12; 13824 rows: Q6_K's
    # 512-workgroup grid, Q4_K / Q5_K's few-rows kernel), 8000 rows (7-8 quads per workgroup), ragged N (4101, 61, 1,
    # 9001: quads past N), K with empty parts (1280: parts of 2, 2, 1, 0; 256, 512, 768: one super-block per part,
    # some parts empty); every output element checked, and a second call gives the same bits
    raw = encode.random_blocks(qtype, nblocks(qtype, N, K), seed=qtype * 3 + M + N, family="normal")
    g = torch.Generator().manual_seed(M * 13 + N + K)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    bias = torch.randn(N, generator=g).to(torch.bfloat16) if with_bias else None
    print(f"case whole-rows qtype={qtype} mid={mid} M={M} N={N} K={K}", flush=True)
    xd, rd = x.cuda(), torch.from_numpy(raw).cuda()
    bd = bias.cuda() if with_bias else None
    y = fused(native, xd, rd, qtype, N, bias=bd, mid=mid)
    check(y, x, weight_bf16(raw, qtype, mid, N, K), bias=bias)
    assert torch.equal(y.view(torch.int16), fused(native, xd, rd, qtype, N, bias=bd, mid=mid).view(torch.int16))


@pytest.mark.parametrize("qtype,mid", [(12, 0), (13, 0), (13, 2), (14, 0), (14, 1), (8, 0), (8, 2)])
def test_whole_rows_form_one_hot_rows_are_the_weight_bits(native, qtype, mid):
    # activation rows that are unit vectors e_k make every output the dequantised weight value w[n, k] itself (one
    # nonzero product, exact float32 sums, a bf16 value rounded to bf16 again): the whole-rows form's dequantisation
    # equals the oracle's bit for bit, columns at part and super-block edges and random ones, scales of realistic
    # size and blocks with d in [1, 8); and so do the panel form's (65 rows, one slice: the 32 unit rows, then rows of
    # zeros) and, for Q8_0, the few-rows kernel's
    N, K = 1000, 5120
    raw = encode.random_blocks(qtype, nblocks(qtype, N, K), seed=qtype, family="normal").reshape(N * K // 256, -1)
    rng = np.random.default_rng(qtype)
    big = rng.random(raw.shape[0]) < 0.1
    d = 208 if qtype == 14 else 0                        # a block's float16 scale d (Q8_0: the first of 8 blocks)
    raw[big, d:d + 2] = np.float16(rng.uniform(1.0, 8.0, size=int(big.sum()))).view(np.uint8).reshape(-1, 2)
    raw = raw.ravel()
    w = weight_bf16(raw, qtype, mid, N, K)
    assert np.isfinite(w.numpy()).all()
    rd = torch.from_numpy(raw).cuda()
    ks = np.concatenate([[0, 31, 32, 255, 256, 1279, 1280, 2559, 2560, 3839, 3840, K - 1], rng.integers(0, K, 20)])
    per = {12: 3, 13: 3, 14: 4, 8: 4}[qtype]             # the most rows the whole-rows form takes (ragged last call)
    calls = [ks[i:i + per] for i in range(0, len(ks), per)]
    if qtype == 8:
        calls += [ks[:16], ks[16:]]                      # and Q8_0 through the few-rows kernel
    for sel in calls:
        x = torch.zeros((len(sel), K), dtype=torch.bfloat16)
        x[torch.arange(len(sel)), torch.from_numpy(sel)] = 1.0
        y = fused(native, x.cuda(), rd, qtype, N, mid=mid).cpu().float()
        assert torch.equal(y, w[:, torch.from_numpy(sel)].T), sel
    x = torch.zeros((65, K), dtype=torch.bfloat16)
    x[torch.arange(len(ks)), torch.from_numpy(ks)] = 1.0
    y = fused(native, x.cuda(), rd, qtype, N, mid=mid).cpu().float()
    assert torch.equal(y[:len(ks)], w[:, torch.from_numpy(ks)].T) and not y[len(ks):].any()


def test_q8_0_drop_in_fuses_few_rows_and_falls_back_elsewhere(native):
    # the GGUF linear with a Q8_0 weight: at 1-4 rows the library's whole-rows form, at 5-64 its few-rows kernel, then
    # its panel form (up to 256 rows for this output, wider than K), beyond the two-step flow (wf_dequant, then the
    # bf16 GEMM) -- the fused kernel itself takes up to 512 rows and declines more; all against the float32 product of
    # the oracle's bf16 weight
    fg = sub("enhancers.fused_gguf")
    N, K = 5120, 2048
    raw = encode.random_blocks(8, nblocks(8, N, K), seed=8, family="normal")
    rd = torch.from_numpy(raw).cuda()
    w = weight_bf16(raw, 8, 0, N, K)
    for rows, fused in ((1, True), (4, True), (5, True), (64, True), (65, True), (256, True), (257, False),
                        (513, False)):
        x = torch.randn((rows, K), generator=torch.Generator().manual_seed(rows)).to(torch.bfloat16)
        assert fg.prefer_fused(rows, 8, N, K) is fused
        assert (fg.fused_linear(x.cuda(), rd, 8, (N, K)) is not None) is (rows <= 512)
        y = fg.linear(x.cuda(), rd, 8, (N, K))
        torch.cuda.synchronize()
        check(y, x, w)


def test_rejects_what_it_does_not_handle(native):
    lib_ = native.lib()
    assert lib_.wf_linear_gguf(None, 4, 300, None, 0, 12, 4, None, None, 0, None) == native.EUNSUPPORTED   # K
    assert lib_.wf_linear_gguf(None, 4, 256, None, 144 * 4, 8, 4, None, None, 0, None) == native.EUNSUPPORTED
    assert lib_.wf_linear_gguf(None, 4, 256, None, 144 * 3, 12, 4, None, None, 0, None) == native.EUNSUPPORTED


def fused_ws(native, x, raw_dev, qtype, N, bias=None, mid=0, ws=None):
    """wf_linear_gguf_ws with a workspace of the size wf_linear_gguf_workspace asks for (zeroed here unless given)"""
    import ctypes
    M, K = x.shape
    need = ctypes.c_int64()
    assert native.lib().wf_linear_gguf_workspace(M, N, K, ctypes.byref(need)) == 0
    if ws is None:
        ws = torch.zeros(max(16384, need.value), dtype=torch.uint8, device=x.device)
    assert ws.numel() >= need.value
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    rc = native.lib().wf_linear_gguf_ws(x.data_ptr(), M, K, raw_dev.data_ptr(), raw_dev.numel(), qtype, N,
                                        bias.data_ptr() if bias is not None else None, y.data_ptr(), mid,
                                        ws.data_ptr(), ws.numel(), native.stream_of(x.device))
    assert rc == 0, native.last_error()
    torch.cuda.synchronize()
    return y, ws, need.value


@pytest.mark.parametrize("qtype", [12, 13, 14])
@pytest.mark.parametrize("mid", [0, 2])
@pytest.mark.parametrize("M,N,K,with_bias", [(1, 300, 8192, True), (5, 2048, 8192, False), (8, 61, 8448, True),
                                             (3, 1000, 13824, False), (7, 384, 9728, True), (8, 640, 8192, False),
                                             (2, 130, 13824, True), (9, 320, 8192, True), (4, 2048, 5120, False),
                                             (6, 1000, 5120, True), (1, 4100, 8192, False)])
def test_split_k_whole_output(native, qtype, mid, M, N, K, with_bias):
    # up to 8 activation rows of a narrow, deep product (N <= 2048, K >= 8192, K >= 2 N) take the split-K form (128
    # weight rows per workgroup, K in slices of 1-4 super-blocks, partial sums added by the last workgroup of each
    # column tile): ragged M, N and slices, every output element checked; 9 rows, N > 2048 or K < 8192 go to the
    # few-rows kernel without the workspace
    raw = encode.random_blocks(qtype, N * K // 256, seed=qtype * 5 + M, family="normal")
    g = torch.Generator().manual_seed(M * 17 + N)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    bias = torch.randn(N, generator=g).to(torch.bfloat16) if with_bias else None
    print(f"case split-K qtype={qtype} mid={mid} M={M} N={N} K={K}", flush=True)
    y, ws, need = fused_ws(native, x.cuda(), torch.from_numpy(raw).cuda(), qtype, N,
                           bias=bias.cuda() if with_bias else None, mid=mid)
    assert (need > 0) == (M <= 8 and N <= 2048 and K >= 8192 and K >= 2 * N)
    check(y, x, weight_bf16(raw, qtype, mid, N, K), bias=bias)
    assert not ws[:16384].any()                          # the counters are back to zero


def test_split_k_reuses_its_workspace_and_repeats_bits(native):
    # two calls on one workspace (the second with fewer rows and another width), then the first again: the same
    # bits as its first run -- the partial sums are added in slice order whichever workgroup arrives last
    qtype, K = 12, 13824
    raws = {N: torch.from_numpy(encode.random_blocks(qtype, N * K // 256, seed=N, family="normal")).cuda()
            for N in (2048, 1280)}
    g = torch.Generator().manual_seed(3)
    x = torch.randn((8, K), generator=g).to(torch.bfloat16).cuda()
    y1, ws, n1 = fused_ws(native, x, raws[2048], qtype, 2048)
    y2, ws, n2 = fused_ws(native, x[:3].contiguous(), raws[1280], qtype, 1280, ws=ws)
    y3, ws, _ = fused_ws(native, x, raws[2048], qtype, 2048, ws=ws)
    assert n1 > 0 and n2 > 0
    assert torch.equal(y1.view(torch.int16), y3.view(torch.int16))
    check(y2, x[:3].cpu(), weight_bf16(raws[1280].cpu().numpy(), qtype, 0, 1280, K))


def test_split_k_rejects_a_short_workspace(native):
    import ctypes
    M, N, K = 8, 256, 8192
    need = ctypes.c_int64()
    assert native.lib().wf_linear_gguf_workspace(M, N, K, ctypes.byref(need)) == 0 and need.value > 0
    x = torch.zeros((M, K), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(N * K // 256 * 144, dtype=torch.uint8, device="cuda")
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    ws = torch.zeros(need.value, dtype=torch.uint8, device="cuda")
    st = native.stream_of(x.device)
    assert native.lib().wf_linear_gguf_ws(x.data_ptr(), M, K, w.data_ptr(), w.numel(), 12, N, None, y.data_ptr(), 0,
                                          ws.data_ptr(), need.value - 1, st) == native.EINVAL
    assert native.lib().wf_linear_gguf_ws(x.data_ptr(), M, K, w.data_ptr(), w.numel(), 12, N, None, y.data_ptr(), 0,
                                          None, 0, st) == native.EINVAL


def noalloc(native, x, raw_dev, qtype, N, bias=None, mid=0):
    M, K = x.shape
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    rc = native.lib().wf_linear_gguf_noalloc(x.data_ptr(), M, K, raw_dev.data_ptr(), raw_dev.numel(), qtype, N,
                                             bias.data_ptr() if bias is not None else None, y.data_ptr(), mid,
                                             native.stream_of(x.device))
    assert rc == 0, native.last_error()
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("qtype", [12, 13, 14, 8])
@pytest.mark.parametrize("M,N,K,with_bias,mid", [(65, 300, 512, True, 0), (128, 256, 2048, False, 2),
                                                 (129, 1002, 1024, True, 0), (300, 520, 5120, False, 0),
                                                 (512, 130, 768, True, 2), (257, 384, 1024, False, 1),
                                                 (17, 300, 1024, True, 0), (24, 640, 1024, False, 1),
                                                 (33, 520, 2048, False, 2), (64, 130, 5120, True, 0),
                                                 (40, 384, 512, True, 0)])
def test_panel_whole_output(native, qtype, M, N, K, with_bias, mid):
    # 65 to 512 activation rows take the panel form (128 weight rows x 16 MT activation rows per workgroup): through
    # wf_linear_gguf in one K slice; through wf_linear_gguf_ws in as many slices as give 256 workgroups (two
    # super-blocks at least), their float32 partial sums added in slice order by a second kernel; allocation-free
    # with the slices its scratch holds. With the workspace it also takes 33-64 rows (MT = 4) and 17-32 rows (MT = 2)
    # of a deep product (K >= 2 N), when K gives more than one slice (else the few-rows kernel: 40 x 512, and the
    # shallow 24 x 640 x 1024); wf_linear_gguf keeps the few-rows kernel up to 64 rows. Ragged M and N (N % 4 != 0
    # takes the reduction's element path), every output element checked; the three agree bit for bit where they run
    # the same slices. Q8_0 takes the panel form from 65 rows only (64-row panels), its few-rows forms below
    raw = encode.random_blocks(qtype, nblocks(qtype, N, K), seed=qtype * 3 + M, family="normal")
    g = torch.Generator().manual_seed(M * 7 + N)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    bias = torch.randn(N, generator=g).to(torch.bfloat16) if with_bias else None
    xd, rd, bd = x.cuda(), torch.from_numpy(raw).cuda(), bias.cuda() if with_bias else None
    print(f"case panel qtype={qtype} mid={mid} M={M} N={N} K={K}", flush=True)
    w = weight_bf16(raw, qtype, mid, N, K)
    y1 = fused(native, xd, rd, qtype, N, bias=bd, mid=mid)
    check(y1, x, w, bias=bias)
    y2, _, need = fused_ws(native, xd, rd, qtype, N, bias=bd, mid=mid)
    check(y2, x, w, bias=bias)
    nsb = K // 256
    assert (need > 0) == (nsb >= 4 and (M > 32 or K >= 2 * N))     # two super-blocks per slice at least
    if need:                                         # the split form's 16 KiB of counters, then the slices
        part = need - 16384
        assert part % (M * N * 4) == 0 and part // (M * N * 4) >= 2
    if not need:
        assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))     # the same form, the same slices
    y3 = noalloc(native, xd, rd, qtype, N, bias=bd, mid=mid)
    if need <= 16 << 20:
        assert torch.equal(y3.view(torch.int16), y2.view(torch.int16))
    check(y3, x, w, bias=bias)


def test_panel_then_split_share_one_workspace(native):
    # one workspace per stream serves every shape: a panel call in K slices leaves the split form's counters at zero,
    # so a split call after it on the same workspace still finds its last workgroup and writes every output
    qtype = 12
    g = torch.Generator().manual_seed(11)
    xp = torch.randn((128, 2048), generator=g).to(torch.bfloat16)
    rp = encode.random_blocks(qtype, 256 * 2048 // 256, seed=5, family="normal")
    xs = torch.randn((4, 8192), generator=g).to(torch.bfloat16)
    rs = encode.random_blocks(qtype, 512 * 8192 // 256, seed=6, family="normal")
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    yp, ws, need_p = fused_ws(native, xp.cuda(), torch.from_numpy(rp).cuda(), qtype, 256, ws=ws)
    assert need_p > 16384                            # the panel form in slices, with partial sums
    assert not ws[:16384].any()
    ys, ws, need_s = fused_ws(native, xs.cuda(), torch.from_numpy(rs).cuda(), qtype, 512, ws=ws)
    assert need_s > 0                                # the split form
    check(yp, xp, weight_bf16(rp, qtype, 0, 256, 2048))
    check(ys, xs, weight_bf16(rs, qtype, 0, 512, 8192))
    assert not ws[:16384].any()


def test_panel_workspace_is_checked(native):
    import ctypes
    M, N, K = 128, 256, 2048
    need = ctypes.c_int64()
    assert native.lib().wf_linear_gguf_workspace(M, N, K, ctypes.byref(need)) == 0 and need.value > 0
    x = torch.zeros((M, K), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(N * K // 256 * 144, dtype=torch.uint8, device="cuda")
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    ws = torch.zeros(need.value, dtype=torch.uint8, device="cuda")
    st = native.stream_of(x.device)
    assert native.lib().wf_linear_gguf_ws(x.data_ptr(), M, K, w.data_ptr(), w.numel(), 12, N, None, y.data_ptr(), 0,
                                          ws.data_ptr(), need.value - 1, st) == native.EINVAL


@pytest.mark.parametrize("qtype", [12, 14])
@pytest.mark.parametrize("rows", [1, 40, 130])
def test_fused_linear_input_layouts(native, qtype, rows):
    # the drop-in takes the weight as ComfyUI-GGUF holds it (1-D or [N, bytes per row] uint8), activations of any
    # leading shape or strides, and a strided bias: every layout gives the bits of the plain 2-D contiguous call,
    # which is itself checked against float64 on the dequantised weight
    fg = sub("enhancers.fused_gguf")
    N, K = 384, 1024
    raw = encode.random_blocks(qtype, N * K // 256, seed=rows + qtype, family="normal")
    g = torch.Generator().manual_seed(rows)
    x = torch.randn((rows, K), generator=g).to(torch.bfloat16)
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    rd, xd, bd = torch.from_numpy(raw).cuda(), x.cuda(), bias.cuda()
    print(f"case fused_linear layouts qtype={qtype} rows={rows}", flush=True)
    ref = fg.fused_linear(xd, rd, qtype, (N, K), bias=bd)
    torch.cuda.synchronize()
    check(ref.cpu(), x, weight_bf16(raw, qtype, 0, N, K), bias=bias)
    bits = ref.view(torch.int16)
    as_rows = rd.view(N, -1)                                            # [N, bytes per row]
    x3 = xd.view(1, rows, K)
    x_strided = torch.empty((rows, 2 * K), dtype=torch.bfloat16, device="cuda")[:, ::2]
    x_strided.copy_(xd)
    b_strided = torch.empty(2 * N, dtype=torch.bfloat16, device="cuda")[::2]
    b_strided.copy_(bd)
    for what, y in (("2-D weight", fg.fused_linear(xd, as_rows, qtype, (N, K), bias=bd)),
                    ("3-D activations", fg.fused_linear(x3, rd, qtype, (N, K), bias=bd)),
                    ("strided activations", fg.fused_linear(x_strided, rd, qtype, (N, K), bias=bd)),
                    ("strided bias", fg.fused_linear(xd, rd, qtype, (N, K), bias=b_strided))):
        torch.cuda.synchronize()
        assert y is not None, what
        assert torch.equal(y.reshape(rows, N).view(torch.int16), bits), what
    assert fg.fused_linear(x3, rd, qtype, (N, K), bias=bd).shape == (1, rows, N)
    # operands off x's device are not the kernel's case (the two-step flow takes them)
    assert fg.fused_linear(xd, rd, qtype, (N, K), bias=bias) is None
    assert fg.fused_linear(xd, torch.from_numpy(raw), qtype, (N, K), bias=bd) is None
    # nor is a 0-dimensional x (no row of K values)
    assert fg.fused_linear(xd[0, 0], rd, qtype, (N, K)) is None
