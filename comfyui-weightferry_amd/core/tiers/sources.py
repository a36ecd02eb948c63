"""Block sources of the SSD tier and the reader ring (core/tiers/sources.py of the reference: FileBlockSource
:87-110, PieceFileSource :113-152, DiskRing :165-355).

A source says where each SSD-tier block's bytes lie in a file: ``FileBlockSource`` one range per block,
``PieceFileSource`` a list of (file offset, bytes, offset in the packed block) per block. ``gguf_block_source`` builds
the pieces of streamed blocks from a GGUF model file's tensor table, each parameter at its offset in the block's flat
layout, with file-adjacent pieces merged (a file written in the flat layout's order and alignment gives one read per
block). ``DiskRing`` is the native ring (wf_ring_*): reader threads fill ``depth`` pinned buffers in cyclic block
order; the streaming state copies out of them with submit / wait, host code with acquire / release."""
import ctypes
import os

import numpy as np
import torch

from ... import _native
from .gguf_file import GGUFReader


class FileBlockSource:
    """Blocks read straight from a file: block i is the byte range ranges[i] = (absolute offset, size)."""

    is_model_file = True

    def __init__(self, path, ranges):
        self.path = str(path)
        self.ranges = [(int(o), int(n)) for o, n in ranges]
        self.n_blocks = len(self.ranges)
        self.block_bytes = max(n for _, n in self.ranges)

    def pieces(self):
        return [[(o, n, 0)] for o, n in self.ranges]


class PieceFileSource:
    """Blocks read from a file when each is several ranges: pieces[i] = list of (absolute offset, bytes, offset in the
    packed block)."""

    is_model_file = True

    def __init__(self, path, pieces):
        self.path = str(path)
        self._pieces = [[(int(o), int(n), int(d)) for o, n, d in blk] for blk in pieces]
        self.n_blocks = len(self._pieces)
        self.block_bytes = max(max(d + n for _, n, d in blk) for blk in self._pieces)

    def pieces(self):
        return self._pieces


def merge_pieces(pieces):
    """Merge consecutive pieces whose file gap equals their block gap (the padding between them is read along)."""
    out = []
    for o, n, d in sorted(pieces, key=lambda p: p[2]):
        if out:
            po, pn, pd = out[-1]
            if o - po == d - pd and o >= po + pn:
                out[-1] = (po, o + n - po, pd)
                continue
        out.append((o, n, d))
    return out


def gguf_block_source(path, block_param_names, offsets, reader=None):
    """PieceFileSource of streamed blocks stored in a GGUF file: block_param_names[i] lists the tensor names of
    block i's parameters (in parameters() order), ``offsets`` their offsets in the block's flat layout. Checks that
    every tensor exists and that all blocks have the same per-parameter sizes."""
    reader = reader or GGUFReader(path)
    blocks = []
    sizes0 = None
    for names in block_param_names:
        if len(names) != len(offsets):
            raise ValueError(f"{len(names)} tensor names for {len(offsets)} parameters")
        pcs, sizes = [], []
        for name, off in zip(names, offsets):
            t = reader.tensors.get(name)
            if t is None:
                raise KeyError(f"{path}: no tensor {name}")
            pcs.append((t.offset, t.nbytes, off))
            sizes.append(t.nbytes)
        if sizes0 is None:
            sizes0 = sizes
        elif sizes != sizes0:
            raise ValueError(f"block of {names[0]} has other tensor sizes than the first streamed block")
        blocks.append(merge_pieces(pcs))
    return PieceFileSource(path, blocks), sizes0


def read_packed(source, d, off, n, out):
    """Bytes [off, off + n) of block d's packed bytes, read from the source's file with ordinary reads into ``out``
    (a writable buffer of n bytes); bytes no piece covers (padding) are zero. For the few reads outside the ring's
    order (layers called before a forward's first block)."""
    mv = memoryview(out).cast("B")
    if mv.nbytes != n:
        raise ValueError(f"a {mv.nbytes}-byte buffer for {n} bytes")
    mv[:] = bytes(n)
    with open(source.path, "rb", buffering=0) as f:
        for fo, ln, po in source.pieces()[d]:
            a, b = max(off, po), min(off + n, po + ln)
            done = 0
            while a + done < b:
                got = os.preadv(f.fileno(), [mv[a - off + done:b - off]], fo + a - po + done)
                if got <= 0:
                    raise OSError(f"{source.path}: short read at {fo + a - po + done}")
                done += got


class DiskRing:
    """The native reader ring over a source. pin=True allocates page-locked buffers (needed for submit); direct=True
    reads with O_DIRECT where the file system allows (no page cache)."""

    def __init__(self, source, depth=2, pin=True, threads=1, direct=True, device=None):
        pieces = source.pieces()
        starts = np.zeros(len(pieces) + 1, dtype=np.int64)
        flat = [p for blk in pieces for p in blk]
        starts[1:] = np.cumsum([len(b) for b in pieces])
        arr = np.array(flat, dtype=np.int64).reshape(-1, 3)
        self._keep = [np.ascontiguousarray(arr[:, k]) for k in range(3)] + [starts]
        flags = (1 if pin else 0) | (2 if direct else 0)
        dev = 0 if device is None else (torch.device(device).index or 0)
        h = ctypes.c_void_p()
        _native.call("wf_ring_open", source.path.encode(), len(pieces), starts.ctypes.data,
                     self._keep[0].ctypes.data, self._keep[1].ctypes.data, self._keep[2].ctypes.data, int(depth),
                     int(threads), flags, dev, ctypes.byref(h))
        self.handle = h.value
        self.n = len(pieces)
        self.depth = depth
        self.block_bytes = source.block_bytes
        self.pinned = pin

    def acquire(self, d):
        """(uint8 CPU tensor viewing block d's bytes in its ring buffer, slot); valid until release(slot)."""
        ptr, n, slot = ctypes.c_void_p(), ctypes.c_int64(), ctypes.c_int()
        _native.call("wf_ring_acquire", self.handle, int(d), ctypes.byref(ptr), ctypes.byref(n), ctypes.byref(slot))
        buf = (ctypes.c_uint8 * n.value).from_address(ptr.value)
        return torch.frombuffer(buf, dtype=torch.uint8), slot.value

    def release(self, slot, stream=None):
        """Return the buffer; with a stream, it is refilled only after the work queued on that stream (its copy)."""
        _native.call("wf_ring_release", self.handle, int(slot), stream)

    def submit(self, d, dst, wait_event, done_event, stream):
        """Copy block d into the device tensor ``dst`` on ``stream`` after ``wait_event`` (a _native.Event or None);
        ``done_event`` is recorded after the copy. Returns the ticket for wait()."""
        t = ctypes.c_int64()
        _native.call("wf_ring_submit", self.handle, int(d), dst.data_ptr(), dst.numel() * dst.element_size(),
                     wait_event.handle if wait_event is not None else None,
                     done_event.handle if done_event is not None else None, stream, ctypes.byref(t))
        return t.value

    def wait(self, ticket):
        _native.call("wf_ring_wait", self.handle, int(ticket))

    def resync(self):
        _native.call("wf_ring_resync", self.handle)

    def stats(self):
        rs, ws = ctypes.c_double(), ctypes.c_double()
        b, r = ctypes.c_int64(), ctypes.c_int64()
        _native.call("wf_ring_stats", self.handle, ctypes.byref(rs), ctypes.byref(ws), ctypes.byref(b), ctypes.byref(r))
        return {"read_s": rs.value, "wait_s": ws.value, "bytes": b.value, "reads": r.value,
                "read_gbps": b.value / rs.value / 1e9 if rs.value > 0 else None}

    def close(self):
        if self.handle is not None:
            h, self.handle = self.handle, None
            _native.call("wf_ring_close", h)

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 -- interpreter shutdown
            pass
