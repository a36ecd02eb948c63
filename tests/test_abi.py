"""The C ABI library loads and exports every function include/weightferry.h declares, the Python binding knows
each of them, and the argument checks answer without touching a GPU (CPU-only: no kernel is launched)."""
import ctypes
import os
import re

import pytest

from conftest import ROOT, sub

HEADER = os.path.join(ROOT, "include", "weightferry.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wf_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_and_library_exports_everything():
    native = sub("_native")
    declared = _declared()
    assert declared, "no declarations found"
    assert sorted(native.EXPORTS) == declared
    lib = native.lib()
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.wf_abi_version() >= 1


def test_argument_checks_without_gpu():
    native = sub("_native")
    lib = native.lib()
    buf = ctypes.create_string_buffer(4096)
    p = ctypes.addressof(buf)
    p16 = (p + 15) // 16 * 16
    # unknown GGML type: "not my case"
    assert lib.wf_dequant(p16, 144, 99, 0, 1, p16, 256, None) == native.EUNSUPPORTED
    assert "99" in native.last_error()
    # dtype codes outside 0..2
    assert lib.wf_dequant(p16, 144, 12, 3, 1, p16, 256, None) == native.EUNSUPPORTED
    # bytes not a whole number of blocks / values that do not match
    assert lib.wf_dequant(p16, 143, 12, 0, 1, p16, 256, None) == native.EUNSUPPORTED
    assert lib.wf_dequant(p16, 144, 12, 0, 1, p16, 255, None) == native.EUNSUPPORTED
    # misaligned pointers
    assert lib.wf_dequant(p16 + 2, 144, 12, 0, 1, p16, 256, None) == native.EUNSUPPORTED
    assert "aligned" in native.last_error()
    # null pointers
    assert lib.wf_dequant(None, 144, 12, 0, 1, None, 256, None) == native.EINVAL
    # nothing to do
    assert lib.wf_dequant(p16, 0, 12, 0, 1, p16, 0, None) == native.OK


def test_dequant_add_argument_checks_without_gpu():
    native = sub("_native")
    lib = native.lib()
    buf = ctypes.create_string_buffer(8192)
    p16 = (ctypes.addressof(buf) + 15) // 16 * 16
    # the same block checks as wf_dequant when the weight is dequantised first
    assert lib.wf_dequant_add(p16, 144, 99, 0, 1, p16, 0.5, p16, 256, None) == native.EUNSUPPORTED
    assert lib.wf_dequant_add(p16, 144, 12, 0, 1, p16, 0.5, p16, 255, None) == native.EUNSUPPORTED
    assert lib.wf_dequant_add(p16, 144, 12, 0, 1, None, 0.5, p16, 256, None) == native.EINVAL
    assert lib.wf_dequant_add(p16, 144, 12, 0, 1, p16 + 4, 0.5, p16, 256, None) == native.EUNSUPPORTED
    assert "aligned" in native.last_error()
    # a later LoRA (no blocks): only the output dtype, the pointers and their alignment matter
    assert lib.wf_dequant_add(None, 0, 0, 0, 3, p16, 0.5, p16, 8, None) == native.EUNSUPPORTED
    assert lib.wf_dequant_add(None, 0, 0, 0, 1, None, 0.5, p16, 8, None) == native.EINVAL
    assert lib.wf_dequant_add(None, 0, 0, 0, 1, p16, 0.5, p16 + 2, 8, None) == native.EUNSUPPORTED
    assert lib.wf_dequant_add(None, 0, 0, 0, 1, p16, 0.5, p16, -1, None) == native.EINVAL
    assert lib.wf_dequant_add(None, 0, 0, 0, 1, None, 0.5, None, 0, None) == native.OK


def test_bf16_gemm_argument_checks_without_gpu():
    native = sub("_native")
    lib = native.lib()
    buf = ctypes.create_string_buffer(4096)
    p16 = (ctypes.addressof(buf) + 15) // 16 * 16
    # K a whole number of 64-value stages, 16-byte aligned operands: else "not my case" (the caller's GEMM runs)
    assert lib.wf_linear_bf16(p16, p16, None, p16, 4, 4, 96, None) == native.EUNSUPPORTED
    assert "64" in native.last_error()
    assert lib.wf_linear_bf16(p16 + 2, p16, None, p16, 4, 4, 64, None) == native.EUNSUPPORTED
    assert lib.wf_linear_bf16(p16, p16 + 8, None, p16, 4, 4, 64, None) == native.EUNSUPPORTED
    assert lib.wf_linear_bf16(p16, p16, None, p16 + 1, 4, 4, 64, None) == native.EUNSUPPORTED
    # operands past the buffer resources' byte range
    assert lib.wf_linear_bf16(p16, p16, None, p16, 1 << 24, 4, 64, None) == native.EUNSUPPORTED
    assert lib.wf_linear_bf16(p16, p16, None, p16, 4, 1 << 24, 64, None) == native.EUNSUPPORTED
    # malformed sizes, null pointers; nothing to do
    assert lib.wf_linear_bf16(p16, p16, None, p16, -1, 4, 64, None) == native.EINVAL
    assert lib.wf_linear_bf16(p16, p16, None, p16, 4, 4, 0, None) == native.EINVAL
    assert lib.wf_linear_bf16(None, p16, None, p16, 4, 4, 64, None) == native.EINVAL
    assert lib.wf_linear_bf16(p16, p16, None, p16, 0, 4, 64, None) == native.OK


def test_check_maps_codes():
    native = sub("_native")
    assert native.check(native.OK, "x") is True
    assert native.check(native.EUNSUPPORTED, "x") is False
    with pytest.raises(native.NativeError):
        native.check(native.EHIP, "x")


def test_probe_is_a_separate_library_with_its_own_checks():
    # the benchmark's byte mover lives in libwf_probe.so: the product library does not export it
    native = sub("_native")
    assert not hasattr(native.lib(), "wf_hbm_stream") and not hasattr(native.lib(), "wfp_hbm_stream")
    probe = ctypes.CDLL(os.path.join(ROOT, "comfyui-weightferry_amd", "lib", "libwf_probe.so"))
    probe.wfp_hbm_stream.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_void_p]
    probe.wfp_last_error.restype = ctypes.c_char_p
    buf = ctypes.create_string_buffer(4096)
    p16 = (ctypes.addressof(buf) + 15) // 16 * 16
    assert probe.wfp_hbm_stream(p16, p16, 0, 1, 2, None) == -1
    assert probe.wfp_hbm_stream(p16, None, 4, 1, 0, None) == -1
    assert probe.wfp_hbm_stream(None, p16, 4, 1, 2, None) == -1
    assert probe.wfp_hbm_stream(p16 + 4, p16, 4, 1, 2, None) == -1
    assert probe.wfp_hbm_stream(p16, p16, 4, 3, 5, None) == -2
    assert b"3:5" in probe.wfp_last_error()


def test_fused_gemm_q8_0_checks_without_gpu():
    # Q8_0 (8 blocks of 34 bytes per 256 values) is the library's case only at 1-512 rows;
    # elsewhere it answers "not my case" before any launch, so the caller's two-step flow runs
    native = sub("_native")
    lib = native.lib()
    buf = ctypes.create_string_buffer(64)
    p16 = (ctypes.addressof(buf) + 15) // 16 * 16
    N, K = 4, 256
    for M, n in ((513, N), (1024, N), (4096, 16353)):
        rc = lib.wf_linear_gguf(p16, M, K, p16, n * (K // 256) * 272, 8, n, None, p16, 0, None)
        assert rc == native.EUNSUPPORTED and "Q8_0" in native.last_error(), (M, n)
    # a block count that is not 34 bytes per 32 values
    assert lib.wf_linear_gguf(p16, 1, K, p16, N * (K // 256) * 256, 8, N, None, p16, 0, None) == native.EUNSUPPORTED
    # rows longer than the kernels' buffer ranges address (any format)
    Kl = (1 << 20) + 256
    for qt, ts in ((8, 272), (12, 144)):
        rc = lib.wf_linear_gguf(p16, 1, Kl, p16, N * (Kl // 256) * ts, qt, N, None, p16, 0, None)
        assert rc == native.EUNSUPPORTED
        assert "1048576" in native.last_error()
    # nothing to do
    assert lib.wf_linear_gguf(p16, 0, K, p16, N * (K // 256) * 272, 8, N, None, p16, 0, None) == native.OK


def test_fused_gemm_workspace_sizes_without_gpu():
    # wf_linear_gguf_workspace is host logic: which form takes a shape with a workspace, and how many float32 partial
    # sums (or split counters) it needs -- the rules the library's header states
    import ctypes as ct
    native = sub("_native")
    lib = native.lib()

    def need(M, N, K):
        v = ct.c_int64(-1)
        assert lib.wf_linear_gguf_workspace(M, N, K, ct.byref(v)) == native.OK
        return v.value
    # 1-16 rows of a shallow or wide product: the few-rows kernel, no workspace
    for M in (1, 8, 16):
        assert need(M, 5120, 5120) == 0 and need(M, 13824, 5120) == 0
    # up to 8 rows of a narrow deep product: the split form (16 KiB of counters, then the partial sums)
    assert need(1, 2048, 8192) > 16384 and need(8, 2048, 8192) > need(1, 2048, 8192)
    # 17-32 rows of a deep product (K >= 2 N) and 33-512 rows of any: the panel form's slices, S * M * N * 4 bytes with
    # S >= 2 (the largest need over the formats), past the split form's 16 KiB of counters (one workspace serves both)
    for M, N, K in ((17, 5120, 13824), (32, 5120, 13824), (33, 5120, 5120), (64, 5120, 13824), (128, 5120, 5120),
                    (512, 13824, 5120)):
        n = need(M, N, K) - 16384
        assert n > 0 and n % (M * N * 4) == 0 and n // (M * N * 4) >= 2, (M, N, K, n)
    # 17-32 rows of a shallow product: the few-rows kernel, no workspace
    for M, N, K in ((17, 5120, 5120), (32, 13824, 5120), (32, 5120, 5120)):
        assert need(M, N, K) == 0, (M, N, K)
    # too shallow for two slices of two super-blocks, or past the panel form: nothing
    assert need(128, 5120, 768) == 0 and need(513, 5120, 5120) == 0 and need(4096, 5120, 5120) == 0
    # bad shapes are refused
    v = ct.c_int64()
    assert lib.wf_linear_gguf_workspace(4, 64, 300, ct.byref(v)) == native.EINVAL
