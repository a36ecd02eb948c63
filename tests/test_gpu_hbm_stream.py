"""The byte-moving kernel the benchmark sets beside the dequantisation (wfp_hbm_stream, in the measurement-only
library libwf_probe.so) moves exactly the bytes it claims: every output chunk of every supported read:write mix holds (xor of the thread's input words, chunk index,
thread index, 0), and nothing past the output is touched."""
import numpy as np
import pytest
import torch

from conftest import ROOT, PKG_NAME, sub

pytestmark = pytest.mark.gpu


def _probe():
    import ctypes
    import os
    sub("_native").lib()                 # torch's HIP runtime first, as for the product library
    lib = ctypes.CDLL(os.path.join(ROOT, PKG_NAME, "lib", "libwf_probe.so"))
    p, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.wfp_hbm_stream.argtypes, lib.wfp_hbm_stream.restype = [p, p, i64, i32, i32, p], i32
    lib.wfp_last_error.restype = ctypes.c_char_p
    return lib


@pytest.mark.parametrize("reads,writes", [(1, 0), (0, 1), (1, 1), (1, 2), (2, 7)])
@pytest.mark.parametrize("items", [1, 255, 4097])
def test_stream_writes_every_chunk(reads, writes, items):
    native = sub("_native")
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(items * 10 + reads)
    src = rng.integers(0, 1 << 32, size=(max(1, reads) * items, 4), dtype=np.uint64).astype(np.uint32)
    inp = torch.from_numpy(src.view(np.int32)).to(dev)
    guard = 64                                                   # chunks after the output that must stay untouched
    out = torch.full(((max(1, writes) * items + guard) * 4,), -7, dtype=torch.int32, device=dev)
    probe = _probe()
    rc = probe.wfp_hbm_stream(inp.data_ptr(), out.data_ptr(), items, reads, writes, native.stream_of(dev))
    assert rc == 0, probe.wfp_last_error()
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32).reshape(-1, 4)
    acc = np.zeros(items, dtype=np.uint32)
    for r in range(reads):
        c = src[r * items:(r + 1) * items]
        acc ^= c[:, 0] ^ c[:, 1] ^ c[:, 2] ^ c[:, 3]
    t = np.arange(items, dtype=np.uint32)
    for w in range(writes):
        chunk = got[w * items:(w + 1) * items]
        assert np.array_equal(chunk[:, 0], acc)
        assert (chunk[:, 1] == w).all()
        assert np.array_equal(chunk[:, 2], t)
        assert (chunk[:, 3] == 0).all()
    untouched = got[writes * items:].view(np.int32)
    if writes == 0:
        # the read-only form may store its sum in the first word only when it equals the kernel's key
        untouched = untouched[1:] if untouched.size else untouched
    assert (untouched == -7).all()
