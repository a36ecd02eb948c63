"""wf_linear_gguf_noalloc, the entry point that allocates nothing, through the C ABI against the entry point it is a
variant of (wf_linear_gguf_ws with a caller's workspace): two split-form calls in a row on the library's scratch,
the second smaller than the first, each bit-identical to wf_linear_gguf_ws; a shape that takes no scratch; a shape
whose scratch would exceed the library's 16 MiB, refused before anything runs."""
import ctypes

import pytest
import torch

from conftest import sub

pytestmark = pytest.mark.gpu

encode = sub("gguf_encode")


def _run(native, fn, x, raw, qtype, N, bias=None, ws=None):
    M, K = x.shape
    y = torch.full((M, N), -7.0, dtype=torch.bfloat16, device=x.device)
    args = [x.data_ptr(), M, K, raw.data_ptr(), raw.numel(), qtype, N, None if bias is None else bias.data_ptr(),
            y.data_ptr(), 0]
    if ws is not None:
        args += [ws.data_ptr(), ws.numel()]
    rc = getattr(native.lib(), fn)(*args, native.stream_of(x.device))
    assert rc == 0, native.last_error()
    torch.cuda.synchronize()
    return y


def _workspace(native, M, N, K):
    need = ctypes.c_int64()
    assert native.lib().wf_linear_gguf_workspace(M, N, K, ctypes.byref(need)) == 0
    return need.value, torch.zeros(max(16384, need.value), dtype=torch.uint8, device="cuda")


@pytest.mark.parametrize("qtype", [12, 14])
def test_noalloc_equals_the_workspace_entry_point(native, qtype):
    g = torch.Generator().manual_seed(qtype)
    K = 13824
    cases = [(8, 2048, True), (3, 1280, False)]          # the second call smaller than the first
    for M, N, with_bias in cases:
        print(f"case noalloc qtype={qtype} M={M} N={N} K={K}", flush=True)
        raw = torch.from_numpy(encode.random_blocks(qtype, N * K // 256, seed=N + qtype, family="normal")).cuda()
        x = torch.randn((M, K), generator=g).to(torch.bfloat16).cuda()
        bias = torch.randn(N, generator=g).to(torch.bfloat16).cuda() if with_bias else None
        need, ws = _workspace(native, M, N, K)
        assert need > 0                                  # the split form: the scratch is used
        ref = _run(native, "wf_linear_gguf_ws", x, raw, qtype, N, bias, ws)
        got = _run(native, "wf_linear_gguf_noalloc", x, raw, qtype, N, bias)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), (M, N)


def test_noalloc_without_split_is_the_plain_entry_point(native):
    g = torch.Generator().manual_seed(5)
    M, N, K = 16, 5120, 5120
    raw = torch.from_numpy(encode.random_blocks(12, N * K // 256, seed=9, family="normal")).cuda()
    x = torch.randn((M, K), generator=g).to(torch.bfloat16).cuda()
    assert _workspace(native, M, N, K)[0] == 0
    ref = _run(native, "wf_linear_gguf", x, raw, 12, N)
    got = _run(native, "wf_linear_gguf_noalloc", x, raw, 12, N)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_noalloc_refuses_a_shape_beyond_its_scratch(native):
    # 8 rows of a 2048 x 307200 Q4_K weight: 300 slices x 8 x 2048 float32 partial sums = 18.75 MiB > 16 MiB
    M, N, K = 8, 2048, 307200
    need, _ = _workspace(native, M, N, K)
    assert need > 16 << 20
    raw = torch.empty(N * K // 256 * 144, dtype=torch.uint8, device="cuda")
    x = torch.zeros((M, K), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    rc = native.lib().wf_linear_gguf_noalloc(x.data_ptr(), M, K, raw.data_ptr(), raw.numel(), 12, N, None,
                                             y.data_ptr(), 0, native.stream_of(x.device))
    assert rc == native.EUNSUPPORTED and "scratch" in native.last_error()
