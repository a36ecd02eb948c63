"""GGUF model files: the native header reader (wf_gguf_*) against files assembled byte by byte from the published
GGUF specification, the package's writer against the same bytes, round trips over every metadata value type and
the tensor types the reader sizes, and malformed files (each must be rejected with an error, never a crash or a
read out of bounds). No GPU is needed."""
import os
import struct

import numpy as np
import pytest

from conftest import sub

gf = sub("core.tiers.gguf_file")
native = sub("_native")


def s(x):
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def by_hand(alignment=None, version=3):
    """A GGUF file spelled out field by field: KV general.architecture = "cosmos" (string), optional
    general.alignment (u32); tensors "a" (F32, dims [3]) then "b" (Q8_0, dims [32, 2] innermost first)."""
    kvs = s("general.architecture") + struct.pack("<I", 8) + s("cosmos")
    n_kv = 1
    al = 32
    if alignment is not None:
        kvs += s("general.alignment") + struct.pack("<II", 4, alignment)
        n_kv += 1
        al = alignment
    a = np.arange(3, dtype=np.float32).tobytes()                       # 12 bytes
    b = bytes(range(68))                                               # 2 rows of one Q8_0 block (34 bytes)
    off_b = (len(a) + al - 1) // al * al
    infos = s("a") + struct.pack("<I", 1) + struct.pack("<Q", 3) + struct.pack("<IQ", 0, 0)
    infos += s("b") + struct.pack("<I", 2) + struct.pack("<QQ", 32, 2) + struct.pack("<IQ", 8, off_b)
    head = b"GGUF" + struct.pack("<IQQ", version, 2, n_kv) + kvs + infos
    data_start = (len(head) + al - 1) // al * al
    body = a + b"\0" * (off_b - len(a)) + b
    return head + b"\0" * (data_start - len(head)) + body, data_start, off_b, a, b


def write(tmp_path, data, name="m.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


@pytest.mark.parametrize("alignment", [None, 64, 4096])
def test_reader_on_a_file_spelled_out_by_hand(tmp_path, alignment):
    data, data_start, off_b, a, b = by_hand(alignment)
    r = gf.GGUFReader(write(tmp_path, data))
    assert r.version == 3 and r.alignment == (alignment or 32) and r.data_offset == data_start
    assert r.file_bytes == len(data)
    assert r.metadata["general.architecture"] == "cosmos"
    assert list(r.tensors) == ["a", "b"]
    ta, tb = r.tensors["a"], r.tensors["b"]
    assert (ta.qtype, ta.shape, ta.offset, ta.nbytes) == (0, (3,), data_start, 12)
    assert (tb.qtype, tb.shape, tb.offset, tb.nbytes) == (8, (2, 32), data_start + off_b, 68)
    assert r.read("a").tobytes() == a and r.read("b").tobytes() == b


@pytest.mark.parametrize("alignment", [32, 64, 4096])
def test_writer_produces_the_same_bytes(tmp_path, alignment):
    data, *_ , a, b = by_hand(None if alignment == 32 else alignment)
    p = str(tmp_path / "w.gguf")
    gf.write_gguf(p, [("a", 0, (3,), a), ("b", 8, (2, 32), b)], {"general.architecture": "cosmos"}, alignment=alignment)
    assert open(p, "rb").read() == data


def test_round_trip_every_value_type_and_tensor_type(tmp_path):
    V = gf.GGUFValue
    meta = {
        "u8": V(gf.UINT8, 200), "i8": V(gf.INT8, -100), "u16": V(gf.UINT16, 60000), "i16": V(gf.INT16, -30000),
        "u32": V(gf.UINT32, 4000000000), "i32": V(gf.INT32, -2000000000), "f32": V(gf.FLOAT32, 0.5),
        "bool": True, "str": "héllo", "u64": V(gf.UINT64, 2 ** 63 + 5), "i64": V(gf.INT64, -(2 ** 40)),
        "f64": V(gf.FLOAT64, 1.0 / 3.0), "arr_i": [1, 2, 3], "arr_s": ["x", "yz", ""], "empty": V(gf.ARRAY, [], gf.INT32),
    }
    rng = np.random.default_rng(0)
    tensors = []
    for k, (name, qt) in enumerate(gf.GGML_TYPES.items()):
        block, size = gf.GGML_GEOMETRY[qt]
        shape = (3, block * 2) if k % 2 else (2, 1, block)
        n = gf.tensor_nbytes(qt, shape)
        assert n == np.prod(shape) // block * size
        tensors.append((f"t.{name}", qt, shape, rng.integers(0, 256, n, dtype=np.uint8)))
    p = str(tmp_path / "rt.gguf")
    gf.write_gguf(p, tensors, meta, alignment=128)
    r = gf.GGUFReader(p)
    assert r.alignment == 128
    for k in ("u8", "i8", "u16", "i16", "u32", "i32", "u64", "i64"):
        assert r.metadata[k] == meta[k].value, k
    assert r.metadata["f32"] == 0.5 and r.metadata["f64"] == 1.0 / 3.0
    assert r.metadata["bool"] is True and r.metadata["str"] == "héllo"
    assert r.metadata["arr_i"] == (gf.UINT32, 3) and r.metadata["arr_s"] == (gf.STRING, 3)
    assert r.metadata["empty"] == (gf.INT32, 0)
    assert list(r.tensors) == [t[0] for t in tensors]
    for name, qt, shape, data in tensors:
        t = r.tensors[name]
        assert t.qtype == qt and t.shape == shape and t.nbytes == data.size
        assert (t.offset - r.data_offset) % 128 == 0
        assert np.array_equal(r.read(name), data)


def rejects(tmp_path, data, fragment):
    p = write(tmp_path, data, "bad.gguf")
    with pytest.raises(native.NativeError) as e:
        gf.GGUFReader(p)
    assert fragment in str(e.value), str(e.value)


def test_every_truncation_is_rejected(tmp_path):
    data, data_start, *_ = by_hand(64)
    for n in list(range(0, data_start, 3)) + [data_start, len(data) - 1]:
        p = write(tmp_path, data[:n], "cut.gguf")
        with pytest.raises(native.NativeError):
            gf.GGUFReader(p)


def test_malformed_headers(tmp_path):
    data, data_start, off_b, *_ = by_hand()
    rejects(tmp_path, b"GGUX" + data[4:], "magic")
    rejects(tmp_path, data[:4] + struct.pack("<I", 1) + data[8:], "version")
    rejects(tmp_path, data[:4] + struct.pack("<I", 4) + data[8:], "version")
    rejects(tmp_path, data[:8] + struct.pack("<Q", 1 << 40) + data[16:], "limit")
    # a string longer than the file
    kv0 = 24
    rejects(tmp_path, data[:kv0] + struct.pack("<Q", 1 << 20) + data[kv0 + 8:], "truncated")
    # unknown value type of the first key/value
    key_end = kv0 + 8 + len("general.architecture")
    rejects(tmp_path, data[:key_end] + struct.pack("<I", 13) + data[key_end + 4:], "value type")


def tensor_file(dims, qtype=8, offset=0, n_dims=None, alignment=None, payload=68):
    kv = b""
    n_kv = 0
    if alignment is not None:
        kv = s("general.alignment") + struct.pack("<II", 4, alignment)
        n_kv = 1
    nd = len(dims) if n_dims is None else n_dims
    info = s("w") + struct.pack("<I", nd) + b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", qtype, offset)
    head = b"GGUF" + struct.pack("<IQQ", 3, 1, n_kv) + kv + info
    al = alignment or 32
    start = (len(head) + al - 1) // al * al
    return head + b"\0" * (start - len(head)) + bytes(payload)


def test_malformed_tensor_infos(tmp_path):
    assert gf.GGUFReader(write(tmp_path, tensor_file([32, 2]))).tensors["w"].nbytes == 68
    rejects(tmp_path, tensor_file([32, 2], payload=67), "beyond the file")
    rejects(tmp_path, tensor_file([32, 2], offset=16, payload=200), "not a multiple")
    rejects(tmp_path, tensor_file([32, 0]), "dimension")
    rejects(tmp_path, tensor_file([33, 2]), "whole number of blocks")
    rejects(tmp_path, tensor_file([32, 2], qtype=99), "GGML type")
    rejects(tmp_path, tensor_file([32, 1, 1, 1, 2]), "dimension count")
    rejects(tmp_path, tensor_file([32, 2], alignment=48), "power-of-two")
    rejects(tmp_path, tensor_file([1 << 40, 1 << 30], qtype=0), "overflows")
    # 2^62 elements pass the element-count check; their bytes (F32: 2^64, F16: 2^63) do not fit in 64 bits and
    # must not wrap to a small or negative size that would pass the end-of-file check
    rejects(tmp_path, tensor_file([1 << 31, 1 << 31], qtype=0), "byte count overflows")
    rejects(tmp_path, tensor_file([1 << 31, 1 << 31], qtype=1), "byte count overflows")
    rejects(tmp_path, tensor_file([1 << 31, 1 << 30], qtype=0), "byte count overflows")


def test_missing_file_and_directory(tmp_path):
    with pytest.raises(native.NativeError):
        gf.GGUFReader(str(tmp_path / "nope.gguf"))
    with pytest.raises(native.NativeError):
        gf.GGUFReader(str(tmp_path))
