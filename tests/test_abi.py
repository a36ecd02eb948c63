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
