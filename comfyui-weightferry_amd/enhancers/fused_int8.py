"""The int8 W8A8 linear on gfx950: the drop-in for the reference's enhancers/fused_int8.py.

ComfyUI's int8 ConvRot linear (a QuantizedTensor weight in TensorWiseINT8Layout: int8 [N, K] + a weight scale)
calls ``lin._forward(input, weight, bias)``; inside ``_Overrides`` that is ``_shared_forward`` /
``_residual_forward``, which quantise the bf16 input per row (wf_quant_rows_i8, ConvRot 256-groups) -- once per input
tensor, shared by q / k / v -- and run the int8 MFMA GEMM with the scale epilogue (wf_linear_i8) or the gated
residual epilogue (wf_linear_i8_residual). Anything else returns None and the layer runs
torch.nn.functional.linear, as in the reference (:279-292,295-308).

Eligibility follows the reference's ``_int8_quantised`` (:123-188): bias None, weight a TensorWiseINT8Layout
QuantizedTensor, not transposed, ConvRot with group size 256, bf16 CUDA input with m > 2 and k % 256 == 0,
k == the weight's K, k within the quantiser's width (<= 6144). The comfy_kitchen device-capability decisions have
no counterpart here. ``int8_linear`` is the direct entry (plain per-token or ConvRot activations, optional bias)."""
import torch

from .. import _native
from .fused_kernels import PRE_GELU, PRE_LNMOD, PRE_MOD, QUANT_MODES
from .fused_state import _count, _state, _tls

_QUANT_MAX_K = {0: 8192, 1: 6144}


# ------------------------------------------------------------------------------------------------ pending inputs
def _key2d(t):
    return (t.data_ptr(), t.numel(), t.shape[-1])


def _set_pre(marker, kind, scale=None, shift=None, norm=None):
    """Register a pending input: the layer that receives ``marker`` quantises kind(marker) itself (modq / gelu;
    lnmod: marker is the block input, norm its LayerNorm) (enhancers/fused_int8.py:28-39)."""
    pre = {"key": _key2d(marker), "kind": kind, "src": marker, "used": False, "mat": None, "norm": norm,
           "scale5": scale, "shift5": shift}
    if kind in ("mod", "lnmod"):
        D = marker.shape[-1]
        groups = scale.numel() // D
        pre["s1"] = (1 + scale).contiguous().view(groups, D)
        pre["shift"] = shift.contiguous().view(groups, D)
        pre["rows_per_group"] = marker.numel() // D // groups
    _tls.pre = pre
    return pre


def _clear_pre():
    pre = getattr(_tls, "pre", None)
    _tls.pre = None
    return pre


def _materialise(pre):
    """The pending input's real value (enhancers/fused_int8.py:48-57): GELU, or x * (1 + scale) + shift after an
    optional LayerNorm, in the input dtype as torch computes them."""
    if pre["mat"] is None:
        src = pre["src"]
        if pre["kind"] == "gelu":
            pre["mat"] = torch.nn.functional.gelu(src)
        else:
            x = pre["norm"](src) if pre["kind"] == "lnmod" else src
            pre["mat"] = x * (1 + pre["scale5"]) + pre["shift5"]
    return pre["mat"]


def _pending_for(input):
    """(the pending input, whether ``input`` is it) (enhancers/fused_int8.py:271-276)."""
    pre = getattr(_tls, "pre", None)
    is_pre = (pre is not None and torch.is_tensor(input) and input.dim() >= 2
              and pre["key"] == _key2d(input.reshape(-1, input.shape[-1])))
    return pre, is_pre


_PRE_CODE = {"gelu": PRE_GELU, "mod": PRE_MOD, "lnmod": PRE_LNMOD}
_gelu_tables = {}


def _gelu_table(device):
    """torch's GELU (erf) of every bfloat16 value, indexed by its 16 bits (enhancers/fused_int8.py:94-105): the
    quantiser's GELU looks its results up here, so they are torch's own on this device."""
    key = str(device)
    tab = _gelu_tables.get(key)
    if tab is None:
        xs = torch.arange(65536, dtype=torch.int32, device=device).to(torch.int16).view(torch.bfloat16)
        tab = torch.nn.functional.gelu(xs).contiguous()
        _gelu_tables[key] = tab
    return tab


def _pre_fusable(pre, k):
    """Whether the pending operation can run inside the quantiser at width k (LNMOD: a LayerNorm without affine
    weights, k % 512 == 0)."""
    if pre["kind"] == "lnmod":
        norm = pre["norm"]
        return (k % 512 == 0 and getattr(norm, "weight", None) is None and getattr(norm, "bias", None) is None
                and isinstance(getattr(norm, "eps", None), float))
    return pre["kind"] in _PRE_CODE


def quantise_pre(pre, x_2d):
    """(x_q, x_s) of kind(x_2d) for the pending input ``pre`` with its operation inside the ConvRot quantiser
    (wf_quant_rows_i8_pre; the reference's _quantise_pre, enhancers/fused_int8.py:60-75), or None when declined."""
    m, k = x_2d.shape
    dev = x_2d.device
    x_q = torch.empty((m, k), dtype=torch.int8, device=dev)
    x_s = torch.empty((m, 1), dtype=torch.float32, device=dev)
    code = _PRE_CODE[pre["kind"]]
    if code == PRE_GELU:
        s, h, rows, eps = _gelu_table(dev), None, 1, 0.0
    else:
        s, h, rows = pre["s1"], pre["shift"], pre["rows_per_group"]
        eps = float(pre["norm"].eps) if code == PRE_LNMOD else 0.0
    with torch.cuda.device(dev):
        rc = _native.lib().wf_quant_rows_i8_pre(x_2d.data_ptr(), m, k, code, s.data_ptr(),
                                                h.data_ptr() if h is not None else None, rows, eps,
                                                x_q.data_ptr(), x_s.data_ptr(), _native.stream_of(dev))
    if not _native.check(rc, "wf_quant_rows_i8_pre"):
        return None
    return x_q, x_s


# ------------------------------------------------------------------------------------------------- the weight
def _plain_weight(weight):
    """(w_q int8 [N, K], w_scale, params) of a TensorWiseINT8Layout QuantizedTensor, or None. Uses ComfyUI's
    quant_ops when importable, else the tensor's own fields (_qdata, _params.scale)."""
    if getattr(weight, "_layout_cls", None) != "TensorWiseINT8Layout":
        return None
    params = getattr(weight, "_params", None)
    try:
        from comfy.quant_ops import TensorWiseINT8Layout
        w_q, w_scale = TensorWiseINT8Layout.get_plain_tensors(weight)
    except ImportError:
        w_q, w_scale = getattr(weight, "_qdata", None), getattr(params, "scale", None)
    if w_q is None or w_scale is None:
        return None
    return w_q, w_scale, params


def _is_quantized(t):
    try:
        from comfy.quant_ops import QuantizedTensor
        return isinstance(t, QuantizedTensor)
    except ImportError:
        return hasattr(t, "_layout_cls") and hasattr(t, "_qdata")


def _weight_scale(w_scale, n, dev):
    ws = torch.as_tensor(w_scale, dtype=torch.float32, device=dev).reshape(-1)
    return ws if ws.numel() == n else ws.expand(n).contiguous()


# ----------------------------------------------------------------------------------------------- entry points
def quantise_rows(x_2d, mode):
    """(x_q int8 [m, k], x_s float32 [m, 1]) of a contiguous bf16 [m, k] CUDA tensor; mode 0 plain, 1 ConvRot."""
    m, k = x_2d.shape
    x_q = torch.empty((m, k), dtype=torch.int8, device=x_2d.device)
    x_s = torch.empty((m, 1), dtype=torch.float32, device=x_2d.device)
    with torch.cuda.device(x_2d.device):
        rc = _native.lib().wf_quant_rows_i8(x_2d.data_ptr(), m, k, mode, x_q.data_ptr(), x_s.data_ptr(),
                                            _native.stream_of(x_2d.device))
    if not _native.check(rc, "wf_quant_rows_i8"):
        return None
    return x_q, x_s


def gemm(x_q, x_s, w_q, ws, out_dtype=torch.bfloat16, bias=None):
    """(float(x_q @ w_q.T) * x_s) * ws (+ bias), rounded once to out_dtype; None when the library declines."""
    m, k = x_q.shape
    n = w_q.shape[0]
    out = torch.empty((m, n), dtype=out_dtype, device=x_q.device)
    code = 1 if out_dtype == torch.bfloat16 else 0
    with torch.cuda.device(x_q.device):
        rc = _native.lib().wf_linear_i8(x_q.data_ptr(), w_q.data_ptr(), x_s.data_ptr(), ws.data_ptr(),
                                        bias.data_ptr() if bias is not None else None, out.data_ptr(), code, m, n, k,
                                        _native.stream_of(x_q.device))
    return out if _native.check(rc, "wf_linear_i8") else None


def int8_linear(x, w_q, w_scale, bias=None, convrot=False):
    """The whole W8A8 linear on bf16 / f16 activations x [..., K]: per-row dynamic int8 activations (plain
    per-token, or ConvRot), int8 weight [N, K] with per-channel (or per-tensor) float32 scale, int32 accumulation,
    output in x's dtype. None when not this path's case."""
    if not x.is_cuda or x.dtype not in (torch.bfloat16, torch.float16) or w_q.dtype != torch.int8:
        return None
    k = x.shape[-1]
    mode = QUANT_MODES["convrot" if convrot else "plain"]
    if w_q.shape[1] != k or k > _QUANT_MAX_K[mode] or (convrot and k % 256) or k % 16:
        return None
    if x.dtype != torch.bfloat16:
        return None
    x_2d = x.reshape(-1, k).contiguous()
    q = quantise_rows(x_2d, mode)
    if q is None:
        return None
    n = w_q.shape[0]
    out = gemm(q[0], q[1], w_q.contiguous(), _weight_scale(w_scale, n, x.device), x.dtype, bias)
    return None if out is None else out.reshape(*x.shape[:-1], n)


def _int8_quantised(x, weight, bias):
    """The quantised input of ComfyUI's int8 ConvRot linear, reused while the same input tensor comes back
    (q / k / v); None when ComfyUI would take any other path for this call (enhancers/fused_int8.py:123-188)."""
    cache = getattr(_tls, "qkv", None)
    if cache is None or bias is not None or not _is_quantized(weight) or _is_quantized(x):
        return None
    plain = _plain_weight(weight)
    if plain is None:
        return None
    w_q, w_scale, params = plain
    if getattr(params, "transposed", False) or not getattr(params, "convrot", False):
        return None
    gs = getattr(params, "convrot_groupsize", 256)
    x = x.contiguous()
    x_2d = x if x.dim() == 2 else x.reshape(-1, x.shape[-1])
    m, k = x_2d.shape
    w_q = w_q.contiguous()
    n = w_q.shape[0]
    if (x.dtype != torch.bfloat16 or not x.is_cuda or m <= 2 or gs != 256 or k % 256 != 0
            or not 256 <= k <= _QUANT_MAX_K[1] or w_q.shape[1] != k):
        return None
    pre, is_pre = _pending_for(x_2d)
    part = {"gelu": "gelu", "lnmod": "ln"}.get(pre["kind"], "modq") if is_pre else None
    if is_pre and not _pre_fusable(pre, k):
        # quantise the real input instead, as ComfyUI does (q / k / v still share it)
        _count(part, False, f"{pre['kind']} at width {k} is not fused")
        x_2d = _materialise(pre).reshape(-1, k).contiguous()
        is_pre = False
    key = (x_2d.data_ptr(), tuple(x_2d.shape), tuple(x_2d.stride()), gs, is_pre)
    if cache.get("key") == key:
        x_q, x_s = cache["q"]
    else:
        # the pending operation inside the quantiser: the same bits as quantising its real value
        q = quantise_pre(pre, x_2d) if is_pre else quantise_rows(x_2d, QUANT_MODES["convrot"])
        if q is None:
            return None
        if is_pre:
            _count(part, True)
        x_q, x_s = q
        cache["key"], cache["q"] = key, (x_q, x_s)
    ws = _weight_scale(w_scale, n, x.device)
    return {"x_q": x_q, "x_s": x_s, "w_q": w_q, "ws": ws, "m": m, "n": n, "dev": x.device, "dtype": x.dtype,
            "shape": x.shape}


def _int8_linear_shared(x, weight, bias):
    """ComfyUI's int8 ConvRot linear with _int8_quantised's input; None when ComfyUI would take another path
    (enhancers/fused_int8.py:191-206)."""
    q = _int8_quantised(x, weight, bias)
    if q is None:
        return None
    out = gemm(q["x_q"], q["x_s"], q["w_q"], q["ws"], q["dtype"])
    if out is None:
        return None
    return out if x.dim() == 2 else out.reshape(*x.shape[:-1], q["n"])


_VERIFY_GATES = False  # tests: check every merged call's gate rows


def _residual_gemm(q, gate2d, resid, out, rows):
    with torch.cuda.device(q["dev"]):
        rc = _native.lib().wf_linear_i8_residual(q["x_q"].data_ptr(), q["w_q"].data_ptr(), q["x_s"].data_ptr(),
                                                 q["ws"].data_ptr(), gate2d.data_ptr(), resid.data_ptr(),
                                                 out.data_ptr(), q["m"], q["n"], q["w_q"].shape[1], rows,
                                                 _native.stream_of(q["dev"]))
    return _native.check(rc, "wf_linear_i8_residual")


def _int8_linear_residual(x, weight, bias, res):
    """x_res + gate * linear(x) for the block's residual x_res (B, T, H, W, D) with gate (B, T, 1, 1D), or the row
    path's (B, N, D) with gate (B, 1, D): one GEMM with the residual epilogue over every (batch, frame) group of
    rows (enhancers/fused_int8.py:212-268). None when not possible."""
    xr, gate = res["x"], res["gate"]
    q = _int8_quantised(x, weight, bias)
    if q is None:
        return None
    m, n = q["m"], q["n"]
    D = xr.shape[-1]
    if xr.dim() == 5:
        B, T, H, W, _ = xr.shape
        if not xr.is_contiguous() or tuple(gate.shape) != (B, T, 1, 1, D):
            return None
        groups, rows = B * T, H * W
    elif xr.dim() == 3:
        groups, rows, _ = xr.shape
        if xr.stride(2) != 1 or xr.stride(1) != D or tuple(gate.shape) != (groups, 1, D):
            return None
    else:
        return None
    if n != D or m != groups * rows or xr.dtype != q["dtype"] or gate.dtype != q["dtype"] or xr.dtype != torch.bfloat16:
        return None
    g2 = gate.reshape(groups, D).contiguous()
    resid = xr.contiguous().view(groups * rows, D)
    out = torch.empty((groups * rows, D), dtype=xr.dtype, device=xr.device)
    if res.get("same") and groups > 1:
        # every group has the same gate: one GEMM over all rows with group 0's gate (the same bits)
        if _VERIFY_GATES:
            _count("resmerge_gate", bool(torch.equal(g2, g2[:1].expand_as(g2))), "gate rows differ")
        used = _residual_gemm(q, g2[:1].contiguous(), resid, out, groups * rows)
        _count("resmerge", bool(used), None if used else "declined")
    else:
        used = _residual_gemm(q, g2, resid, out, rows)
    if not used:
        return None
    return out.view(*q["shape"][:-1], n) if xr.dim() == 3 else out.view(xr.shape)


def _shared_forward(input, weight, bias):
    """The _forward of a linear layer under _Overrides (enhancers/fused_int8.py:279-292)."""
    pre, is_pre = _pending_for(input)
    if is_pre:
        pre["used"] = True
    out = _int8_linear_shared(input, weight, bias)
    if out is None:
        _count("qkv", False, f"weight {type(weight).__name__} {getattr(weight, '_layout_cls', None)}, "
                             f"input {type(input).__name__} {getattr(input, 'dtype', None)}")
        if is_pre:
            input = _materialise(pre).reshape(input.shape)
        return torch.nn.functional.linear(input, weight, bias)
    _count("qkv", True)
    return out


def _residual_forward(input, weight, bias):
    """The _forward of a sub-layer's output projection with the block's residual pending
    (enhancers/fused_int8.py:295-308)."""
    res = getattr(_tls, "res", None)
    if res is not None and not res["done"]:
        pre, is_pre = _pending_for(input)
        out = _int8_linear_residual(input, weight, bias, res)
        if out is not None:
            if is_pre:
                pre["used"] = True
            res["done"] = True
            _count("res", True)
            return out
        _count("res", False, f"input {tuple(input.shape)} {input.dtype}")
    return _shared_forward(input, weight, bias)


class _Overrides:
    """_shared_forward (or the given function) on some linear layers for the duration of a call, as an instance
    attribute over the class method (enhancers/fused_int8.py:311-332)."""

    def __init__(self, layers):
        pairs = [x if isinstance(x, tuple) else (x, _shared_forward) for x in layers]
        self.layers = [(lin, fn) for lin, fn in pairs if "_forward" not in lin.__dict__]

    def __enter__(self):
        self.outer = getattr(_tls, "qkv", None) is not None
        if not self.outer:
            _tls.qkv = {}
        for lin, fn in self.layers:
            lin._forward = fn
        return self

    def __exit__(self, *exc):
        for lin, _fn in self.layers:
            lin.__dict__.pop("_forward", None)
        if not self.outer:
            _tls.qkv = None
        return False


__all__ = ["quantise_pre", "_gelu_table", "_int8_quantised", "_int8_linear_shared", "_int8_linear_residual", "_shared_forward",
           "_residual_forward", "_Overrides", "int8_linear", "quantise_rows", "gemm", "_state"]
