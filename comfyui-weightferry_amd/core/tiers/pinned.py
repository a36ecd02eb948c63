"""Page-locked (pinned) host memory of exactly the requested size: the drop-in for the reference's PinnedHost
(core/tiers/pinned.py:74-149).

The reference registers an ordinary allocation with cudaHostRegister. Here the buffer is allocated page-locked by
the library (wf_host_alloc = hipHostMalloc): also exact-size, also returned to the OS at release(). When that fails
the buffer falls back to torch's pinned allocator, and where no GPU exists at all, to pageable memory (registered is
False then, as in the reference's fallback: correct, slower DMA)."""
import ctypes
import threading

import torch

from ... import _native

_REGISTERED = {"bytes": 0, "count": 0}
_LOCK = threading.RLock()


class PinnedHost:
    """Page-locked host buffer of exactly ``nbytes`` (plus optional alignment); ``.tensor`` is a uint8 CPU tensor
    over it. Call release() when done (also done on garbage collection); no copy may still read it then."""

    def __init__(self, nbytes, align=0):
        self.nbytes = int(nbytes)
        total = self.nbytes + int(align)
        self._held = 0                 # bytes counted in registered_bytes() for this buffer
        self._ptr = None
        self._base = None
        self.registered = False
        if total > 0:
            try:
                p = ctypes.c_void_p()
                _native.call("wf_host_alloc", total, ctypes.byref(p))
                self._ptr = p.value
                self._base = torch.frombuffer((ctypes.c_uint8 * total).from_address(self._ptr), dtype=torch.uint8)
                self.registered = True
            except Exception:  # noqa: BLE001 -- not page-locked by the library: torch's pinned allocator, or pageable
                self._ptr = None
        if self._base is None:
            try:
                self._base = torch.empty(total, dtype=torch.uint8, device="cpu", pin_memory=True)
                self.registered = False
            except Exception:  # noqa: BLE001 -- no GPU runtime at all
                self._base = torch.empty(total, dtype=torch.uint8, device="cpu")
        if self.registered:
            self._held = total
            with _LOCK:
                _REGISTERED["bytes"] += total
                _REGISTERED["count"] += 1
        addr = self._base.data_ptr()
        off = (-addr) % align if align else 0
        self.tensor = self._base[off:off + self.nbytes]

    @property
    def ptr(self):
        return self.tensor.data_ptr() if self.tensor is not None else None

    def release(self):
        if self._base is None:
            return
        self.tensor = None
        base, self._base = self._base, None
        del base
        if self._ptr is not None:
            ptr, self._ptr = self._ptr, None
            try:
                _native.lib().wf_host_free(ptr)
            except Exception:  # noqa: BLE001 -- releasing at shutdown: nothing left to do
                pass
            with _LOCK:
                _REGISTERED["bytes"] -= self._held
                _REGISTERED["count"] -= 1
            self._held = 0
        self.registered = False

    def __del__(self):
        try:
            self.release()
        except Exception:  # noqa: BLE001 -- __del__ must not raise
            pass


def release_all(holders):
    for h in holders or ():
        if h is not None:
            h.release()


def registered_bytes():
    with _LOCK:
        return dict(_REGISTERED)
