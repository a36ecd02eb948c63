"""GGUF model files: the tensor table through the native reader (wf_gguf_*), and a writer.

The reference reads GGUF files through ComfyUI-GGUF / gguf-py (not vendored) and writes them with gguf-py's
GGUFWriter (tools/convert_to_gguf.py:45-75: architecture "cosmos", general.quantization_version,
general.file_type, each tensor padded to the alignment). The SSD tier needs each tensor's absolute byte range to
read streamed blocks straight from the model file; ``GGUFReader`` gives it. ``write_gguf`` writes a GGUF version 3
file of raw tensor bytes (the synthetic models of the tests and the benchmark, and a converter's output side).

GGUF dimensions are innermost first; ``GGUFTensor.shape`` is the torch order (outermost first), as ComfyUI-GGUF's
``tensor_shape``."""
import ctypes
import os
import struct
from dataclasses import dataclass

import numpy as np

from ... import _native

# GGML type ids and block geometry (values per block, bytes per block) of the types the reader sizes
GGML_TYPES = {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8, "Q2_K": 10, "Q3_K": 11,
              "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "BF16": 30}
GGML_GEOMETRY = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
                 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 30: (1, 2)}

# GGUF metadata value types
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALAR_FMT = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
               BOOL: "<?", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}


def tensor_nbytes(qtype, shape):
    """Bytes of a tensor of GGML type ``qtype`` and torch shape ``shape`` (the innermost dimension in whole blocks)."""
    block, size = GGML_GEOMETRY[qtype]
    n = 1
    for d in shape:
        n *= int(d)
    if int(shape[-1]) % block:
        raise ValueError(f"row length {shape[-1]} is not a multiple of the type's {block}-value blocks")
    return n // block * size


@dataclass(frozen=True)
class GGUFTensor:
    name: str
    qtype: int
    shape: tuple      # torch order, outermost first
    offset: int       # absolute byte offset in the file
    nbytes: int


class GGUFReader:
    """The header of a GGUF file: ``metadata`` (key -> value; arrays as (element type, count)), ``tensors``
    (name -> GGUFTensor, in file order), ``version``, ``alignment``, ``data_offset``, ``file_bytes``."""

    def __init__(self, path):
        self.path = os.fspath(path)
        lib = _native.lib()
        h = ctypes.c_void_p()
        _native.call("wf_gguf_open", self.path.encode(), ctypes.byref(h))
        try:
            ver, nt, nkv, al, doff, fb = ctypes.c_int(), *(ctypes.c_int64() for _ in range(5))
            _native.call("wf_gguf_info", h, ctypes.byref(ver), ctypes.byref(nt), ctypes.byref(nkv), ctypes.byref(al),
                         ctypes.byref(doff), ctypes.byref(fb))
            self.version, self.alignment = ver.value, al.value
            self.data_offset, self.file_bytes = doff.value, fb.value
            self.metadata = {}
            for i in range(nkv.value):
                self._kv(lib, h, i)
            self.tensors = {}
            name = ctypes.create_string_buffer(1 << 16)
            typ, nd = ctypes.c_int(), ctypes.c_int()
            dims = (ctypes.c_int64 * 4)()
            off, nb = ctypes.c_int64(), ctypes.c_int64()
            for i in range(nt.value):
                _native.call("wf_gguf_tensor", h, i, name, len(name), ctypes.byref(typ), ctypes.byref(nd), dims,
                             ctypes.byref(off), ctypes.byref(nb))
                key = name.value.decode("utf-8", errors="replace")
                shape = tuple(int(dims[d]) for d in range(nd.value))[::-1]
                self.tensors[key] = GGUFTensor(key, typ.value, shape, off.value, nb.value)
        finally:
            lib.wf_gguf_close(h)

    def _kv(self, lib, h, i):
        key = ctypes.create_string_buffer(1 << 16)
        typ, et = ctypes.c_int(), ctypes.c_int()
        cnt, iv = ctypes.c_int64(), ctypes.c_int64()
        fv = ctypes.c_double()
        # first call sizes a string value, the second (if needed) fetches it
        _native.call("wf_gguf_kv", h, i, key, len(key), ctypes.byref(typ), ctypes.byref(et), ctypes.byref(cnt),
                     ctypes.byref(iv), ctypes.byref(fv), None, 0)
        k = key.value.decode("utf-8", errors="replace")
        t = typ.value
        if t == STRING:
            sval = ctypes.create_string_buffer(cnt.value + 1)
            _native.call("wf_gguf_kv", h, i, key, len(key), ctypes.byref(typ), ctypes.byref(et), ctypes.byref(cnt),
                         ctypes.byref(iv), ctypes.byref(fv), sval, len(sval))
            v = sval.raw[:cnt.value].decode("utf-8", errors="replace")
        elif t == ARRAY:
            v = (et.value, cnt.value)
        elif t == BOOL:
            v = bool(iv.value)
        elif t in (FLOAT32, FLOAT64):
            v = fv.value
        else:
            v = iv.value if t != UINT64 else iv.value & 0xFFFFFFFFFFFFFFFF
        self.metadata[k] = v

    def read(self, name):
        """The raw bytes of tensor ``name`` (numpy uint8), read from the file."""
        t = self.tensors[name]
        with open(self.path, "rb") as f:
            f.seek(t.offset)
            data = f.read(t.nbytes)
        if len(data) != t.nbytes:
            raise EOFError(f"{self.path}: tensor {name} is cut short")
        return np.frombuffer(data, dtype=np.uint8)


def _pack_string(s):
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _infer_type(v):
    if isinstance(v, bool):
        return BOOL
    if isinstance(v, int):
        return UINT32 if 0 <= v < 2 ** 32 else INT64
    if isinstance(v, float):
        return FLOAT32
    if isinstance(v, str):
        return STRING
    if isinstance(v, (list, tuple)):
        return ARRAY
    raise TypeError(f"no GGUF type for {type(v).__name__}")


@dataclass(frozen=True)
class GGUFValue:
    """A metadata value with an explicit GGUF type (arrays: type ARRAY, a list value and its element type)."""
    type: int
    value: object
    elem_type: int = UINT32


def _pack_value(t, v, et=None):
    if t == STRING:
        return _pack_string(v)
    if t == ARRAY:
        return struct.pack("<IQ", et, len(v)) + b"".join(_pack_value(et, x) for x in v)
    return struct.pack(_SCALAR_FMT[t], v)


def write_gguf(path, tensors, metadata=None, alignment=32, version=3):
    """Write a GGUF file. ``tensors``: iterable of (name, qtype, shape (torch order), data: bytes-like / numpy / torch
    uint8 of the tensor's exact size). ``metadata``: key -> value (type inferred: bool, u32 or i64, f32, string,
    list = array of the first element's type) or key -> GGUFValue. A non-default ``alignment`` is written as
    general.alignment (u32). Tensors are laid out in the given order, each at the next multiple of the alignment.
    Returns the data section's offset."""
    metadata = dict(metadata or {})
    if alignment != 32:
        metadata["general.alignment"] = GGUFValue(UINT32, int(alignment))
    items = []
    for k, v in metadata.items():
        if not isinstance(v, GGUFValue):
            t = _infer_type(v)
            v = GGUFValue(t, list(v), _infer_type(v[0]) if v else UINT32) if t == ARRAY else GGUFValue(t, v)
        items.append((k, v))
    infos, datas, offset = [], [], 0
    for name, qtype, shape, data in tensors:
        buf = _as_buffer(data)
        need = tensor_nbytes(qtype, shape)
        if buf.nbytes != need:
            raise ValueError(f"tensor {name}: {buf.nbytes} bytes for {need}")
        offset = (offset + alignment - 1) // alignment * alignment
        infos.append((name, qtype, tuple(int(d) for d in shape)[::-1], offset))
        datas.append((offset, buf))
        offset += buf.nbytes
    head = b"GGUF" + struct.pack("<IQQ", version, len(infos), len(items))
    for k, v in items:
        head += _pack_string(k) + struct.pack("<I", v.type) + _pack_value(v.type, v.value, v.elem_type)
    for name, qtype, dims, off in infos:
        head += _pack_string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", qtype, off)
    data_start = (len(head) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * (data_start - len(head)))
        pos = 0
        for off, buf in datas:
            f.write(b"\0" * (off - pos))
            f.write(memoryview(buf))
            pos = off + buf.nbytes
    return data_start


def _as_buffer(data):
    """Contiguous uint8 numpy view of a tensor's bytes (no copy for contiguous CPU data)."""
    if isinstance(data, (bytes, bytearray, memoryview)):
        return np.frombuffer(data, dtype=np.uint8)
    if isinstance(data, np.ndarray):
        return np.ascontiguousarray(data).reshape(-1).view(np.uint8)
    try:
        import torch
        if isinstance(data, torch.Tensor):
            return data.detach().contiguous().cpu().reshape(-1).view(torch.uint8).numpy()
    except ImportError:
        pass
    raise TypeError(f"tensor data of type {type(data).__name__}")
