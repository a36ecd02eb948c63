"""ctypes binding of libweightferry_hip.so, the gfx950 kernels behind the C ABI of ``include/weightferry.h``.

The library is built in-tree by ``csrc/Makefile`` into ``lib/libweightferry_hip.so``. There is no other
implementation: when the library is missing every GPU entry point raises ``NativeMissing`` (the drop-in never
falls back to a CPU or torch computation of its own).

torch is imported before the library is loaded so that the library binds to torch's HIP runtime (both carry the
SONAME libamdhip64.so.7): one runtime per process, and torch's stream handles are valid in every call.
"""
import contextlib
import ctypes
import os
import threading

import torch  # noqa: F401  -- first: the library must bind to torch's HIP runtime

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libweightferry_hip.so")

OK, EINVAL, EUNSUPPORTED, EHIP = 0, -1, -2, -3

_p, _i64, _int, _sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t

# every symbol of include/weightferry.h: name -> (restype, argtypes)
EXPORTS = {
    "wf_abi_version": (_int, []),
    "wf_last_error": (ctypes.c_char_p, []),
    "wf_dequant": (_int, [_p, _i64, _int, _int, _int, _p, _i64, _p]),
    "wf_dequant_add": (_int, [_p, _i64, _int, _int, _int, _p, ctypes.c_float, _p, _i64, _p]),
    "wf_quant_rows_i8": (_int, [_p, _i64, _i64, _int, _p, _p, _p]),
    "wf_quant_rows_i8_pre": (_int, [_p, _i64, _i64, _int, _p, _p, _i64, ctypes.c_float, _p, _p, _p]),
    "wf_linear_i8": (_int, [_p, _p, _p, _p, _p, _p, _int, _i64, _i64, _i64, _p]),
    "wf_linear_bf16": (_int, [_p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "wf_linear_i8_residual": (_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p]),
    "wf_linear_gguf": (_int, [_p, _i64, _i64, _p, _i64, _int, _i64, _p, _p, _int, _p]),
    "wf_linear_gguf_workspace": (_int, [_i64, _i64, _i64, ctypes.POINTER(_i64)]),
    "wf_linear_gguf_ws": (_int, [_p, _i64, _i64, _p, _i64, _int, _i64, _p, _p, _int, _p, _i64, _p]),
    "wf_linear_gguf_noalloc": (_int, [_p, _i64, _i64, _p, _i64, _int, _i64, _p, _p, _int, _p]),
    "wf_host_alloc": (_int, [_sz, ctypes.POINTER(ctypes.c_void_p)]),
    "wf_host_free": (_int, [_p]),
    "wf_h2d_async": (_int, [_p, _p, _sz, _p]),
    "wf_stream_create": (_int, [ctypes.POINTER(ctypes.c_void_p)]),
    "wf_stream_destroy": (_int, [_p]),
    "wf_stream_synchronize": (_int, [_p]),
    "wf_event_create": (_int, [ctypes.POINTER(ctypes.c_void_p), _int]),
    "wf_event_destroy": (_int, [_p]),
    "wf_event_record": (_int, [_p, _p]),
    "wf_stream_wait_event": (_int, [_p, _p]),
    "wf_event_query": (_int, [_p]),
    "wf_event_synchronize": (_int, [_p]),
    "wf_event_elapsed_ms": (_int, [_p, _p, ctypes.POINTER(ctypes.c_float)]),
    "wf_gguf_open": (_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)]),
    "wf_gguf_close": (_int, [_p]),
    "wf_gguf_info": (_int, [_p, ctypes.POINTER(_int)] + [ctypes.POINTER(_i64)] * 5),
    "wf_gguf_tensor": (_int, [_p, _i64, ctypes.c_char_p, _i64, ctypes.POINTER(_int), ctypes.POINTER(_int),
                              ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "wf_gguf_kv": (_int, [_p, _i64, ctypes.c_char_p, _i64, ctypes.POINTER(_int), ctypes.POINTER(_int),
                          ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(ctypes.c_double),
                          ctypes.c_char_p, _i64]),
    "wf_ring_open": (_int, [ctypes.c_char_p, _i64, _p, _p, _p, _p, _int, _int, _int, _int,
                            ctypes.POINTER(ctypes.c_void_p)]),
    "wf_ring_acquire": (_int, [_p, _i64, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(_i64),
                               ctypes.POINTER(_int)]),
    "wf_ring_release": (_int, [_p, _int, _p]),
    "wf_ring_submit": (_int, [_p, _i64, _p, _i64, _p, _p, _p, ctypes.POINTER(_i64)]),
    "wf_ring_wait": (_int, [_p, _i64]),
    "wf_ring_resync": (_int, [_p]),
    "wf_ring_stats": (_int, [_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                             ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "wf_ring_close": (_int, [_p]),
}

_lib = None
_lock = threading.Lock()


class NativeMissing(RuntimeError):
    """libweightferry_hip.so is not built (or does not load): the HIP path cannot run."""


def available():
    try:
        lib()
        return True
    except NativeMissing:
        return False


def lib():
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise NativeMissing(f"{LIB_PATH} is not built: run `make -C {os.path.join(_HERE, 'csrc')}` "
                                    "(or __graft_entry__.build()) first")
            try:
                handle = ctypes.CDLL(LIB_PATH)
            except OSError as exc:
                raise NativeMissing(f"{LIB_PATH} does not load: {exc}") from exc
            for name, (res, args) in EXPORTS.items():
                fn = getattr(handle, name, None)
                if fn is None:
                    raise NativeMissing(f"{LIB_PATH} does not export {name}")
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def last_error():
    msg = lib().wf_last_error()
    return msg.decode(errors="replace") if msg else ""


class NativeError(RuntimeError):
    pass


def check(rc, what):
    """True on WF_OK, False on WF_EUNSUPPORTED ("not my case": the caller returns None), raises otherwise."""
    if rc == OK:
        return True
    if rc == EUNSUPPORTED:
        return False
    raise NativeError(f"{what} failed ({rc}): {last_error()}")


def call(fn_name, *args):
    """lib().<fn_name>(*args), raising NativeError on any non-zero return."""
    rc = getattr(lib(), fn_name)(*args)
    if rc != OK:
        raise NativeError(f"{fn_name} failed ({rc}): {last_error()}")
    return rc


class Stream:
    """A HIP stream of the library (non-blocking, default priority); .handle is the hipStream_t."""

    def __init__(self):
        h = ctypes.c_void_p()
        call("wf_stream_create", ctypes.byref(h))
        self.handle = h.value

    def synchronize(self):
        call("wf_stream_synchronize", self.handle)

    def close(self):
        if self.handle is not None:
            lib().wf_stream_destroy(self.handle)
            self.handle = None


class Event:
    """A HIP event of the library; timing=True keeps timestamps for elapsed_ms."""

    def __init__(self, timing=False):
        h = ctypes.c_void_p()
        call("wf_event_create", ctypes.byref(h), 1 if timing else 0)
        self.handle = h.value

    def record(self, stream):
        call("wf_event_record", self.handle, stream)

    def query(self):
        rc = lib().wf_event_query(self.handle)
        if rc < 0:
            raise NativeError(f"wf_event_query failed ({rc}): {last_error()}")
        return rc == 0

    def synchronize(self):
        call("wf_event_synchronize", self.handle)

    def elapsed_ms(self, end):
        ms = ctypes.c_float()
        call("wf_event_elapsed_ms", self.handle, end.handle, ctypes.byref(ms))
        return float(ms.value)

    def close(self):
        if self.handle is not None:
            lib().wf_event_destroy(self.handle)
            self.handle = None


def stream_wait(stream, event):
    call("wf_stream_wait_event", stream, event.handle)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_no_guard = contextlib.nullcontext()


def on_device(device):
    """``torch.cuda.device(device)`` when ``device`` is not the current device, else a no-op context: the library's
    kernels run on the current device, and the guard costs a few microseconds per call when it changes nothing."""
    if device.index is None or device.index == torch.cuda.current_device():
        return _no_guard
    return torch.cuda.device(device)


def stream_of(device):
    """Raw hipStream_t of torch's current stream on ``device`` (the convention of the reference's int8 path,
    enhancers/fused_int8.py:151). torch's raw-stream query when it has one (a fraction of the cost of building the
    Stream object: this runs once per layer call)."""
    if _raw_stream is not None:
        if not isinstance(device, torch.device):
            device = torch.device(device)
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream
