"""Shared state of the int8 linear path: the per-thread pending input / shared quantisation / pending residual, and
the per-part used / fallback counters (the reference's enhancers/fused_state.py)."""
import threading

_state = {"parts": ("modq",), "orig": None}
_stats = {}   # part -> {"used": n, "fallback": n, "why": first fallback reason}
_tls = threading.local()


def _count(part, used, why=None):
    st = _stats.setdefault(part, {"used": 0, "fallback": 0, "why": None})
    if used:
        st["used"] += 1
    else:
        st["fallback"] += 1
        if st["why"] is None:
            st["why"] = why


def stats(reset=False):
    out = {k: dict(v) for k, v in _stats.items()}
    if reset:
        _stats.clear()
    return out
