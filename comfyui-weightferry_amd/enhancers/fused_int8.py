"""Int8 W8A8 linears of ComfyUI's ConvRot-quantised models on the gfx950 kernels.

How a call arrives. ComfyUI's quantised Linear computes ``self._forward(input, weight, bias)``. A caller that sees
the whole block (``int8_block``, the Cosmos / Anima block adapter) sets ``_forward`` on chosen layers for one
sub-layer with ``_Overrides``: ``_shared_forward`` for input projections, ``_residual_forward`` for the projection
whose output is added to the block's residual stream. Each of them either produces the layer's output here or
returns ComfyUI's own result (``torch.nn.functional.linear`` on the QuantizedTensor), counting which through
``fused_state._count``.

What a call here computes, for a bf16 input x [m, k] and an int8 ConvRot weight w_q [n, k] with scale ws:

* the input's per-row ConvRot int8 quantisation (``wf_quant_rows_i8`` / ``_pre``), *once* per input tensor while
  ``_Overrides`` is active: q, k and v projections of the same input share it (the ``qkv`` cache);
* an input may arrive *pending*: the block registered that the real input is op(marker) -- a scale-and-shift
  (``mod``), LayerNorm then scale-and-shift (``lnmod``), or GELU (``gelu``) -- and the layer receives ``marker``;
  the operation then runs inside the quantiser and the real input is never written;
* the int8 GEMM with the scale epilogue (``wf_linear_i8``), or with the gated residual ``x_res + gate * out``
  (``wf_linear_i8_residual``) when the block left its residual pending.

The per-thread state lives in ``fused_state._tls``: ``qkv`` (the shared quantisation, a dict while ``_Overrides``
is active), ``pre`` (the pending input), ``res`` (the pending residual). The names of this module's functions and
of those three fields are the reference's protocol between its block and its linear path (enhancers/fused_int8.py,
enhancers/fused_block.py); the eligibility rules follow enhancers/fused_int8.py:108-147.
"""
import atexit
from collections import namedtuple

import torch

from .. import _native
from .fused_state import _count, _state, _tls  # noqa: F401 -- _state is part of this module's public surface

# the operation wf_quant_rows_i8_pre applies to a row before its rotation (the reference's codes,
# enhancers/fused_kernels.py:14-18): GELU of the bf16 input; the scale-and-shift bf16(bf16(x * (1 + scale)) + shift);
# LayerNorm without affine, then that scale-and-shift. Rows with no operation go through wf_quant_rows_i8.
PRE_GELU, PRE_MOD, PRE_LNMOD = 1, 2, 3
QUANT_MODES = {"plain": 0, "convrot": 1}

# widest rows the quantiser takes (wf_quant_rows_i8: four waves per row beyond 6144 / 8192 values)
_QUANT_MAX_K = {QUANT_MODES["plain"]: 32768, QUANT_MODES["convrot"]: 32768}
_CONVROT_GROUP = 256


# ------------------------------------------------------------------------------------------------ kernels
def _stream(dev):
    return _native.stream_of(dev)


def quantise_rows(x_2d, mode):
    """(x_q int8 [m, k], x_s float32 [m, 1]) of a contiguous bf16 CUDA tensor [m, k]: per-row int8 of the values
    themselves (mode 0) or of their 256-group ConvRot rotation (mode 1). None when the library declines."""
    m, k = x_2d.shape
    dev = x_2d.device
    x_q = torch.empty((m, k), dtype=torch.int8, device=dev)
    x_s = torch.empty((m, 1), dtype=torch.float32, device=dev)
    with _native.on_device(dev):
        rc = _native.lib().wf_quant_rows_i8(x_2d.data_ptr(), m, k, mode, x_q.data_ptr(), x_s.data_ptr(), _stream(dev))
    return (x_q, x_s) if _native.check(rc, "wf_quant_rows_i8") else None


def gemm(x_q, x_s, w_q, ws, out_dtype=torch.bfloat16, bias=None):
    """out[m, n] = out_dtype((float(sum_k x_q[m, k] w_q[n, k]) * x_s[m]) * ws[n] (+ bias[n])), the sum exact in
    int32; None when the library declines."""
    m, k = x_q.shape
    n = w_q.shape[0]
    dev = x_q.device
    out = torch.empty((m, n), dtype=out_dtype, device=dev)
    code = 1 if out_dtype == torch.bfloat16 else 0
    with _native.on_device(dev):
        rc = _native.lib().wf_linear_i8(x_q.data_ptr(), w_q.data_ptr(), x_s.data_ptr(), ws.data_ptr(),
                                        None if bias is None else bias.data_ptr(), out.data_ptr(), code, m, n, k,
                                        _stream(dev))
    return out if _native.check(rc, "wf_linear_i8") else None


def _gemm_residual(q, gate_2d, resid_2d, out_2d, rows_per_gate):
    """wf_linear_i8_residual: out = bf16(resid + gate[row // rows_per_gate] * linear) over q's rows."""
    with _native.on_device(q.device):
        rc = _native.lib().wf_linear_i8_residual(q.x_q.data_ptr(), q.w_q.data_ptr(), q.x_s.data_ptr(),
                                                 q.ws.data_ptr(), gate_2d.data_ptr(), resid_2d.data_ptr(),
                                                 out_2d.data_ptr(), q.m, q.n, q.w_q.shape[1], rows_per_gate,
                                                 _stream(q.device))
    return _native.check(rc, "wf_linear_i8_residual")


# ------------------------------------------------------------------------------------- a direct entry point
def _channel_scales(w_scale, n, dev):
    """The weight scale as float32 [n] on ``dev`` (a per-tensor scalar is repeated)."""
    ws = torch.as_tensor(w_scale, dtype=torch.float32, device=dev).reshape(-1)
    return ws if ws.numel() == n else ws.expand(n).contiguous()


def int8_linear(x, w_q, w_scale, bias=None, convrot=False):
    """The W8A8 linear of bf16 activations x [..., k]: dynamic per-row int8 activations (plain, or ConvRot),
    weight w_q int8 [n, k] with a float32 per-channel (or per-tensor) scale, exact int32 sums, output bf16
    [..., n]. None when this is not the kernels' case."""
    if not x.is_cuda or x.dtype != torch.bfloat16 or w_q.dtype != torch.int8 or w_q.device != x.device:
        return None
    if bias is not None and bias.device != x.device:
        return None
    k = x.shape[-1]
    mode = QUANT_MODES["convrot" if convrot else "plain"]
    if w_q.shape[1] != k or k % 16 or k > _QUANT_MAX_K[mode] or (convrot and k % _CONVROT_GROUP):
        return None
    q = quantise_rows(x.reshape(-1, k).contiguous(), mode)
    if q is None:
        return None
    n = w_q.shape[0]
    out = gemm(q[0], q[1], w_q.contiguous(), _channel_scales(w_scale, n, x.device), x.dtype, bias)
    return None if out is None else out.reshape(*x.shape[:-1], n)


# ------------------------------------------------------------------------------------------ pending inputs
class _Pending:
    """An input left pending by the block: the layer that receives ``src`` (recognised by ``key``) quantises
    ``kind``(src) instead. Read by dict access too (``pre["used"]``), the form the reference's block uses."""

    __slots__ = ("key", "kind", "src", "norm", "scale", "shift", "s1", "shift2d", "rows_per_group", "used", "_real")

    def __init__(self, src, kind, scale=None, shift=None, norm=None):
        self.key, self.kind, self.src, self.norm = _key2d(src), kind, src, norm
        self.scale, self.shift, self.used, self._real = scale, shift, False, None
        self.s1 = self.shift2d = None
        self.rows_per_group = 1
        if kind in ("mod", "lnmod"):
            width = src.shape[-1]
            groups = scale.numel() // width          # (batch x frames) of the block, batch of the row path
            self.s1 = (1 + scale).contiguous().view(groups, width)
            self.shift2d = shift.contiguous().view(groups, width)
            self.rows_per_group = src.numel() // width // groups

    def __getitem__(self, name):
        return getattr(self, name)

    def __setitem__(self, name, value):
        setattr(self, name, value)

    def real(self):
        """The real input, computed as ComfyUI computes it (torch ops in the input dtype), once."""
        if self._real is None:
            if self.kind == "gelu":
                self._real = torch.nn.functional.gelu(self.src)
            else:
                base = self.norm(self.src) if self.kind == "lnmod" else self.src
                self._real = base * (1 + self.scale) + self.shift
        return self._real

    def fusable(self, k):
        """Whether the quantiser can apply the operation at row width k. The LayerNorm is restated for
        LayerNorms without affine parameters, on rows PyTorch's own kernel splits the same way: widths that are
        multiples of 512 and powers of two (the reference's rule, enhancers/fused_block.py:509-520)."""
        if self.kind != "lnmod":
            return self.kind in _PRE_CODES
        norm = self.norm
        return (k % 512 == 0 and not k & (k - 1) and getattr(norm, "weight", None) is None
                and getattr(norm, "bias", None) is None and isinstance(getattr(norm, "eps", None), float))


_PRE_CODES = {"gelu": PRE_GELU, "mod": PRE_MOD, "lnmod": PRE_LNMOD}
_PRE_PART = {"gelu": "gelu", "lnmod": "ln", "mod": "modq"}   # the counter each kind is reported under


def _key2d(t):
    """How a pending input recognises its tensor: storage address, size and row width (reshapes keep them)."""
    return t.data_ptr(), t.numel(), t.shape[-1]


def _set_pre(marker, kind, scale=None, shift=None, norm=None):
    """Leave ``kind``(marker) pending for the layer that receives ``marker`` (enhancers/fused_int8.py:28-39):
    kind "mod" -- marker * (1 + scale) + shift; "lnmod" -- the same after ``norm`` (marker is then the block
    input); "gelu" -- GELU of marker. Returns the pending record; its ``used`` says whether a layer took it."""
    _tls.pre = _Pending(marker, kind, scale, shift, norm)
    return _tls.pre


def _clear_pre():
    """Drop the pending input (returns it, or None)."""
    pre, _tls.pre = getattr(_tls, "pre", None), None
    return pre


def _materialise(pre):
    """The pending input's real value (computed once)."""
    return pre.real()


def _pending_for(input):
    """(the pending input, whether ``input`` is the tensor it is pending on) (enhancers/fused_int8.py:271-276)."""
    pre = getattr(_tls, "pre", None)
    if pre is None or not torch.is_tensor(input) or input.dim() < 2:
        return pre, False
    return pre, pre.key == _key2d(input.reshape(-1, input.shape[-1]))


_gelu_tables = {}


def _gelu_table(device):
    """torch's GELU (erf form) of all 65536 bfloat16 values on ``device``, indexed by the value's bits: the
    quantiser's GELU reads its results from here, so they are torch's own bits on this device."""
    key = str(device)
    if key not in _gelu_tables:
        every_bf16 = torch.arange(65536, dtype=torch.int32, device=device).to(torch.int16).view(torch.bfloat16)
        _gelu_tables[key] = torch.nn.functional.gelu(every_bf16).contiguous()
    return _gelu_tables[key]


def _release_gpu_caches():
    """Drop the GPU tensors this module holds (GELU tables; a leftover pending input, shared quantisation or
    pending residual of this thread) at interpreter exit, before the modules and torch's allocator are torn down
    (the reference does the same at exit, enhancers/fused_int8.py:81-91)."""
    _gelu_tables.clear()
    for name in ("pre", "qkv", "res"):
        if getattr(_tls, name, None) is not None:
            setattr(_tls, name, None)


atexit.register(_release_gpu_caches)


def quantise_pre(pre, x_2d):
    """(x_q, x_s) of the pending operation applied to x_2d, the operation inside the ConvRot quantiser
    (wf_quant_rows_i8_pre); the same bits as quantising the real input. None when the library declines."""
    m, k = x_2d.shape
    dev = x_2d.device
    code = _PRE_CODES[pre.kind]
    if code == PRE_GELU:
        table, shift, rows, eps = _gelu_table(dev), None, 1, 0.0
    else:
        table, shift, rows = pre.s1, pre.shift2d, pre.rows_per_group
        eps = float(pre.norm.eps) if code == PRE_LNMOD else 0.0
    x_q = torch.empty((m, k), dtype=torch.int8, device=dev)
    x_s = torch.empty((m, 1), dtype=torch.float32, device=dev)
    with _native.on_device(dev):
        rc = _native.lib().wf_quant_rows_i8_pre(x_2d.data_ptr(), m, k, code, table.data_ptr(),
                                                None if shift is None else shift.data_ptr(), rows, eps,
                                                x_q.data_ptr(), x_s.data_ptr(), _stream(dev))
    return (x_q, x_s) if _native.check(rc, "wf_quant_rows_i8_pre") else None


# ----------------------------------------------------------------------------------------------- the weight
def _is_quantized(t):
    """Whether t is ComfyUI's QuantizedTensor (by class when ComfyUI is importable, else by its fields)."""
    try:
        from comfy.quant_ops import QuantizedTensor
    except ImportError:
        return hasattr(t, "_layout_cls") and hasattr(t, "_qdata")
    return isinstance(t, QuantizedTensor)


def _int8_weight(weight):
    """(w_q int8 [n, k], scale, layout parameters) of a TensorWiseINT8Layout QuantizedTensor, else None."""
    if getattr(weight, "_layout_cls", None) != "TensorWiseINT8Layout":
        return None
    params = getattr(weight, "_params", None)
    try:
        from comfy.quant_ops import TensorWiseINT8Layout
    except ImportError:
        w_q, scale = getattr(weight, "_qdata", None), getattr(params, "scale", None)
    else:
        w_q, scale = TensorWiseINT8Layout.get_plain_tensors(weight)
    return None if w_q is None or scale is None else (w_q, scale, params)


def _quant_algos():
    """ComfyUI's table of quantisation formats (comfy.quant_ops.QUANT_ALGOS), or None without ComfyUI."""
    try:
        from comfy.quant_ops import QUANT_ALGOS
    except ImportError:
        return None
    return QUANT_ALGOS


def _int8_proj_ok(lin):
    """Whether the layer passes its input unchanged to ``_forward``: a ComfyUI quantised linear (it has
    ``_forward`` and no forward of its own on the instance) with an int8 TensorWiseINT8Layout weight, no AWQ
    pre-quantisation scale, and a format that does not quantise the input itself (enhancers/fused_int8.py:108-115).
    False without ComfyUI's format table."""
    algos = _quant_algos()
    if algos is None or not hasattr(lin, "_forward") or "forward" in getattr(lin, "__dict__", {}):
        return False
    if getattr(lin, "pre_quant_scale", None) is not None:
        return False
    fmt = algos.get(getattr(lin, "quant_format", None), {})
    return (fmt.get("quantize_input", True) is False
            and getattr(getattr(lin, "weight", None), "_layout_cls", None) == "TensorWiseINT8Layout")


# ---------------------------------------------------------------------------------- the shared quantisation
_Quantised = namedtuple("_Quantised", "x_q x_s w_q ws m n device dtype shape")


def _eligible_weight(x, weight, bias, cache):
    """(w_q, scale, params) when ComfyUI would run its int8 ConvRot path for this call and the kernels take it,
    else None (enhancers/fused_int8.py:129-147): inside _Overrides, no bias, a non-transposed ConvRot
    TensorWiseINT8Layout weight with 256-groups, a bf16 CUDA input that is not quantised itself, more than two
    rows, a width that is whole groups, within the quantiser's range and equal to the weight's."""
    if cache is None or bias is not None or _is_quantized(x) or not _is_quantized(weight):
        return None
    plain = _int8_weight(weight)
    if plain is None:
        return None
    w_q, scale, params = plain
    if getattr(params, "transposed", False) or not getattr(params, "convrot", False):
        return None
    if getattr(params, "convrot_groupsize", _CONVROT_GROUP) != _CONVROT_GROUP:
        return None
    k = x.shape[-1] if x.dim() else 0
    m = x.numel() // k if k else 0
    if x.dtype != torch.bfloat16 or not x.is_cuda or m <= 2 or k % _CONVROT_GROUP:
        return None
    if not _CONVROT_GROUP <= k <= _QUANT_MAX_K[QUANT_MODES["convrot"]] or w_q.shape[1] != k:
        return None
    if w_q.device != x.device:
        return None                 # the kernels read the weight on x's device (the scales are moved there)
    return plain


def _int8_quantised(x, weight, bias):
    """The int8 form of ``x`` for this linear (the input quantised, the weight as int8 rows and channel scales),
    or None when ComfyUI would take another path for this call. While one ``_Overrides`` is active, an input seen
    before (the same tensor: q / k / v) reuses its quantisation; a pending input is quantised with its operation
    inside the quantiser, or -- when that operation cannot be fused at this width -- from its real value, which
    the projections then share (enhancers/fused_int8.py:123-188)."""
    cache = getattr(_tls, "qkv", None)
    plain = _eligible_weight(x, weight, bias, cache)
    if plain is None:
        return None
    w_q, scale, _params = plain
    x = x.contiguous()
    x_2d = x.reshape(-1, x.shape[-1])
    m, k = x_2d.shape
    pre, pending = _pending_for(x_2d)
    if pending and not pre.fusable(k):
        _count(_PRE_PART[pre.kind], False, f"{pre.kind} at width {k} is not fused")
        x_2d = pre.real().reshape(-1, k).contiguous()
        pending = False
    key = (x_2d.data_ptr(), tuple(x_2d.shape), tuple(x_2d.stride()), _CONVROT_GROUP, pending)
    if cache.get("key") == key:
        x_q, x_s = cache["q"]
    else:
        q = quantise_pre(pre, x_2d) if pending else quantise_rows(x_2d, QUANT_MODES["convrot"])
        if q is None:
            return None
        if pending:
            _count(_PRE_PART[pre.kind], True)
        x_q, x_s = q
        cache["key"], cache["q"] = key, q
    w_q = w_q.contiguous()
    n = w_q.shape[0]
    return _Quantised(x_q, x_s, w_q, _channel_scales(scale, n, x.device), m, n, x.device, x.dtype, x.shape)


def _int8_linear_shared(x, weight, bias):
    """ComfyUI's int8 ConvRot linear of x through the kernels, with ``_int8_quantised``'s input; None when ComfyUI
    would take another path (enhancers/fused_int8.py:191-206)."""
    q = _int8_quantised(x, weight, bias)
    if q is None:
        return None
    out = gemm(q.x_q, q.x_s, q.w_q, q.ws, q.dtype)
    if out is None or x.dim() == 2:
        return out
    return out.reshape(*x.shape[:-1], q.n)


_VERIFY_GATES = False  # tests set it: every merged residual call checks that its gate rows are really equal


def _residual_layout(xr, gate):
    """(groups, rows per group) of the pending residual when the epilogue can read it in place: the block's
    (B, T, H, W, D) contiguous residual with gate (B, T, 1, 1, D), or the row path's (B, N, D) residual with
    unit-stride rows and gate (B, 1, D); else None."""
    width = xr.shape[-1]
    if xr.dim() == 5:
        b, t, h, w, _ = xr.shape
        ok = xr.is_contiguous() and tuple(gate.shape) == (b, t, 1, 1, width)
        return (b * t, h * w) if ok else None
    if xr.dim() == 3:
        groups, rows, _ = xr.shape
        ok = xr.stride(2) == 1 and xr.stride(1) == width and tuple(gate.shape) == (groups, 1, width)
        return (groups, rows) if ok else None
    return None


def _int8_linear_residual(x, weight, bias, res):
    """``x_res + gate * linear(x)`` for the pending residual ``res`` ({"x": x_res, "gate": gate, "same": bool}),
    with the sum inside the GEMM's epilogue: one launch over every (batch, frame) group of rows, each group with
    its own gate row -- or group 0's gate for all of them when ``res["same"]`` says the gate rows are equal.
    None when not possible (enhancers/fused_int8.py:212-268)."""
    xr, gate = res["x"], res["gate"]
    q = _int8_quantised(x, weight, bias)
    if q is None:
        return None
    layout = _residual_layout(xr, gate)
    if layout is None:
        return None
    groups, rows = layout
    width = xr.shape[-1]
    if q.n != width or q.m != groups * rows:
        return None
    if not xr.dtype == gate.dtype == q.dtype == torch.bfloat16:
        return None
    gates = gate.reshape(groups, width).contiguous()
    resid = xr.contiguous().view(groups * rows, width)
    out = torch.empty((groups * rows, width), dtype=xr.dtype, device=xr.device)
    merged = bool(res.get("same")) and groups > 1
    if merged:
        if _VERIFY_GATES:
            _count("resmerge_gate", bool(torch.equal(gates, gates[:1].expand_as(gates))), "gate rows differ")
        ok = _gemm_residual(q, gates[:1].contiguous(), resid, out, groups * rows)
        _count("resmerge", ok, None if ok else "declined")
    else:
        ok = _gemm_residual(q, gates, resid, out, rows)
    if not ok:
        return None
    return out.view(xr.shape) if xr.dim() == 5 else out.view(*q.shape[:-1], q.n)


# -------------------------------------------------------------------------------------- the _forward overrides
def _fallback(input, weight, bias, pre, pending, why):
    """ComfyUI's own linear on the real input, counted as a fallback of the shared path."""
    _count("qkv", False, why)
    if pending:
        input = pre.real().reshape(input.shape)
    return torch.nn.functional.linear(input, weight, bias)


def _shared_forward(input, weight, bias):
    """``_forward`` of an input projection under ``_Overrides`` (enhancers/fused_int8.py:279-292)."""
    pre, pending = _pending_for(input)
    if pending:
        pre.used = True
    out = _int8_linear_shared(input, weight, bias)
    if out is None:
        why = (f"weight {type(weight).__name__} {getattr(weight, '_layout_cls', None)}, "
               f"input {type(input).__name__} {getattr(input, 'dtype', None)}")
        return _fallback(input, weight, bias, pre, pending, why)
    _count("qkv", True)
    return out


def _residual_forward(input, weight, bias):
    """``_forward`` of the projection whose output joins the residual stream: ``x_res + gate * linear(input)``
    inside the GEMM while the block's residual is pending and not yet added (it is then marked done), else the
    plain shared path (enhancers/fused_int8.py:295-308)."""
    res = getattr(_tls, "res", None)
    if res is None or res["done"]:
        return _shared_forward(input, weight, bias)
    pre, pending = _pending_for(input)
    out = _int8_linear_residual(input, weight, bias, res)
    if out is None:
        _count("res", False, f"input {tuple(input.shape)} {input.dtype}")
        return _shared_forward(input, weight, bias)
    if pending:
        pre.used = True
    res["done"] = True
    _count("res", True)
    return out


class _Overrides:
    """A context in which the given linear layers compute through this module: each entry is a layer (it gets
    ``_shared_forward``) or a (layer, function) pair; the function is set as an instance attribute ``_forward`` over
    the class method and removed on exit. A layer that already has an instance ``_forward`` is left alone. The
    outermost active context owns the shared-quantisation cache (enhancers/fused_int8.py:311-332)."""

    def __init__(self, layers):
        chosen = [item if isinstance(item, tuple) else (item, _shared_forward) for item in layers]
        self.layers = [(lin, fn) for lin, fn in chosen if "_forward" not in lin.__dict__]
        self.outer = False

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


__all__ = ["quantise_rows", "quantise_pre", "gemm", "int8_linear", "_gelu_table", "_int8_proj_ok", "_int8_quantised",
           "_int8_linear_shared", "_int8_linear_residual", "_shared_forward", "_residual_forward", "_Overrides",
           "_set_pre", "_clear_pre", "_materialise", "_pending_for", "_state"]
