"""State shared by the int8 linear path (fused_int8) and its block adapter (int8_block): the installed parts and
the methods they replaced, the per-thread pending input / shared quantisation / pending residual (``_tls.pre``,
``_tls.qkv``, ``_tls.res``), and per-part counters of calls served here ("used") or left to ComfyUI ("fallback", with
the first reason seen). The counters' shape is what ``stats()`` reports (the reference's enhancers/fused_state.py).
"""
import threading

_state = {"parts": (), "orig": None}
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
