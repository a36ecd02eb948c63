"""Linear layers whose weight is GGUF K-quant blocks, with the dequantisation inside the GEMM (wf_linear_gguf).

The reference dequantises the weight (enhancers/gguf_dequant.py:296-326, one kernel into a bf16 weight in HBM)
and ComfyUI-GGUF then runs torch.nn.functional.linear on it. ``linear`` does both in one kernel launch for bf16
activations and a Q4_K / Q5_K / Q6_K weight, with the same dequantised values (dequant dtype MID, then the layer
dtype) and float32 accumulation; mode="dequant" keeps the reference's two-step flow (wf_dequant, then the bf16 GEMM:
the library's wf_linear_bf16 where it is the faster one, ``hand_gemm``, else torch.nn.functional.linear);
mode="auto" (the default of GGUFLinear) picks whichever measured faster on MI355X for the layer's shape
(``prefer_fused``). Anything else -- other formats, dtypes, CPU tensors -- returns None from ``fused_linear`` and
``linear`` takes the two-step flow."""
import ctypes

import torch

from .. import _native
from . import gguf_dequant

_FUSED_TYPES = {12: 144, 13: 176, 14: 210, 8: 272}   # weight bytes per 256 values (Q8_0: 8 blocks of 34)
Q8_0_ROWS = 512              # Q8_0 is fused at 1-512 rows (the library's whole-rows, few-rows and panel forms)
_MID = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
_workspaces = {}             # (device index, stream) -> uint8 workspace whose counter words are zero between calls
_needs = {}                  # (rows, n_out, k) -> the workspace bytes wf_linear_gguf_workspace gives


def _workspace(device, stream, nbytes):
    """The split-K workspace of this device and stream, at least ``nbytes``: allocated zeroed once (its counters
    must be zero on entry, and every call leaves them zero) and grown when a larger product needs more. Calls on one
    stream are ordered, so they can share it."""
    key = (device.index, stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


def _workspace_bytes(rows, n_out, k):
    """wf_linear_gguf_workspace for this shape, asked once per shape (the answer depends on the shape only)."""
    key = (rows, n_out, k)
    need = _needs.get(key)
    if need is None:
        v = ctypes.c_int64()
        _native.call("wf_linear_gguf_workspace", rows, n_out, k, ctypes.byref(v))
        if len(_needs) > 4096:
            _needs.clear()
        need = _needs[key] = v.value
    return need


def _launch(x2, raw, q, n_out, k, b, y, mid):
    rows = x2.shape[0]
    stream = _native.stream_of(x2.device)
    args = (x2.data_ptr(), rows, k, raw.data_ptr(), raw.numel(), q, n_out, b.data_ptr() if b is not None else None,
            y.data_ptr(), mid)
    need = _workspace_bytes(rows, n_out, k)
    if need:                        # the split or panel form (K in slices) with its workspace
        ws = _workspace(x2.device, stream, need)
        return _native.lib().wf_linear_gguf_ws(*args, ws.data_ptr(), ws.numel(), stream)
    return _native.lib().wf_linear_gguf(*args, stream)


def fused_linear(x, data, qtype, oshape, bias=None, mid_dtype=None):
    """y = x @ dequantize(W).T (+ bias) in one kernel, or None when this is not that case."""
    q = int(qtype) if qtype is not None else None
    if q not in _FUSED_TYPES or not x.is_cuda or x.dim() == 0 or data.device != x.device or x.dtype != torch.bfloat16:
        return None                 # (one device: the kernel reads every operand on x's device)
    if bias is not None and bias.device != x.device:
        return None
    n_out, k = int(oshape[0]), int(oshape[1])
    if x.shape[-1] != k or k % 256 or (bias is not None and (bias.dtype != torch.bfloat16 or bias.numel() != n_out)):
        return None
    mid = torch.float16 if mid_dtype is None else mid_dtype
    if mid not in _MID:
        return None
    if not data.is_contiguous():
        return None
    # (the reshapes only where needed: this runs once per layer call, and with few rows its host time is the layer's)
    raw = data if data.dim() == 1 and data.dtype == torch.uint8 else data.reshape(-1).view(torch.uint8)
    if raw.numel() != n_out * (k // 256) * _FUSED_TYPES[q]:
        return None
    if q == 8 and x.numel() // k > Q8_0_ROWS:
        return None                 # (the library's answer for these Q8_0 shapes: not its case)
    x2 = x if x.dim() == 2 and x.is_contiguous() else x.reshape(-1, k).contiguous()
    y = torch.empty((x2.shape[0], n_out), dtype=torch.bfloat16, device=x.device)
    b = bias if bias is None or bias.is_contiguous() else bias.contiguous()
    with _native.on_device(x.device):
        rc = _launch(x2, raw, q, n_out, k, b, y, _MID[mid])
    if not _native.check(rc, "wf_linear_gguf"):
        return None
    return y if x.dim() == 2 else y.reshape(*x.shape[:-1], n_out)


# Where the fused kernel beats the two-step flow (one dequantisation, then hipBLASLt), measured on MI355X over the
# Wan-14B shapes (5120 x 5120, 13824 x 5120, 5120 x 13824), µs per block of six layers:
#   * up to 64 rows, its few-rows form (the weight streamed through the chip once): 32 rows 124-134 µs against
#     269-334 two-step (Q4_K); with the workspace the library runs the panel form in K slices from 33 rows, and from
#     17 rows for deep products (K >= 2 N) (Wan shapes at 64 rows: 5120 x 13824 Q4_K 45 against 70 µs);
#   * 65-256 rows, its panel form (128 x 128 panels, K in slices): Q4_K 183 against 367 µs at 128 rows, 290 against
#     496 at 256; Q5_K 198 / 306 against 363 / 500; Q6_K 269 / 451 against 364 / 502; and up to 384 rows for Q4_K /
#     Q5_K (three 128-row panels): Q4_K 375 / 380 against 411 / 417 at 320 / 384 rows, Q5_K 408 / 412 against
#     415 / 421 (Q6_K 607 against 413 at 320) -- except the wide ffn_up (n_out > k: 13824 x 5120, 102 against 85 µs
#     at 320 rows, 324 panels on 256 CUs), which keeps the two-step flow above 256 rows; Q4_K up to 512 rows (with
#     512 workgroups of K slices there): 5120 x 5120 58 against 61 µs at 512 rows, 5120 x 13824 122 against 137;
#   * above that the two-step flow is faster: Q5_K 515 / 524 against 467 / 490 µs per block at 448 / 512 rows, Q6_K
#     737 against 491 at 512; Q5_K 1.80 against 1.72 ms at 4096; at 8192 the tiled form wins only 5120 x 5120, by
#     5 % (Q4_K).
# mode "fused" still takes the tiled form at any row count.
FEW_ROWS = 64
# Q8_0 (64-row panels): 243 / 252 / 437 µs against 339 / 424 / 553 at 65 / 128 / 256 rows; at 384 rows its ffn_up
# 150 against 114 µs, the other layers 56 / 131 against 59 / 136; at 512 rows 721 against 540 per block. At 1-64 rows
# (whole-rows and few-rows forms) 87-273 µs against 257-337.
PANEL_ROWS = {12: 512, 13: 384, 14: 256, 8: 384}


def prefer_fused(rows, qtype, n_out, k):
    """mode "auto": True when the fused kernel is the faster way to compute this layer on MI355X."""
    if rows <= FEW_ROWS:
        return True
    limit = PANEL_ROWS.get(int(qtype), 0)
    if n_out > k:
        limit = min(limit, 256)
    return rows <= limit


# The two-step flow's GEMM: the library's wf_linear_bf16 (whole 128-byte lines through two LDS stage buffers, 256 x 320
# tiles at these sizes) against hipBLASLt's (torch.nn.functional.linear), ms per Wan-14B shape on MI355X:
#   4096 rows: 5120 x 5120 0.165 against 0.176, 5120 x 13824 0.432 against 0.449, 13824 x 5120 0.459 against 0.404
#              (704 tiles: 2.75 rounds of 256 workgroups) -- the block's six linears 1.546 against 1.549;
#   2048 rows and fewer: 0.104-0.114 against 0.095 (5120 x 5120) -- 128 or fewer 256 x 320 tiles leave CUs idle;
#   16384 rows: 0.640 against 0.562 (5120 x 5120), 6.07 against 5.47 per block -- hipBLASLt's stream-K kernel keeps
#              its MFMA 83 % busy against 73 % here.
# So wf_linear_bf16 takes the products whose 256 x 320 tiling gives one to three rounds of 256 workgroups.
HAND_GEMM_TILES = (256, 768)


def hand_gemm(rows, n_out):
    """True when wf_linear_bf16 is the faster GEMM for a [rows, k] x [n_out, k]^T product on MI355X."""
    tiles = -(-rows // 256) * -(-n_out // 320)
    return HAND_GEMM_TILES[0] <= tiles <= HAND_GEMM_TILES[1]


def bf16_linear(x, w, bias=None):
    """y = x @ w.T (+ bias) by wf_linear_bf16 (bf16 in and out, float32 accumulation), or None when that kernel does
    not take the case (dtypes, devices, K % 64, alignment)."""
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16 or not x.is_cuda or w.device != x.device or w.dim() != 2:
        return None
    n_out, k = w.shape
    if x.dim() == 0 or x.shape[-1] != k or not w.is_contiguous():
        return None
    if bias is not None and (bias.dtype != torch.bfloat16 or bias.device != x.device or bias.numel() != n_out):
        return None
    x2 = x if x.dim() == 2 and x.is_contiguous() else x.reshape(-1, k).contiguous()
    b = bias if bias is None or bias.is_contiguous() else bias.contiguous()
    y = torch.empty((x2.shape[0], n_out), dtype=torch.bfloat16, device=x.device)
    with _native.on_device(x.device):
        rc = _native.lib().wf_linear_bf16(x2.data_ptr(), w.data_ptr(), b.data_ptr() if b is not None else None,
                                          y.data_ptr(), x2.shape[0], n_out, k, _native.stream_of(x.device))
    if not _native.check(rc, "wf_linear_bf16"):
        return None
    return y if x.dim() == 2 else y.reshape(*x.shape[:-1], n_out)


def linear(x, data, qtype, oshape, bias=None, mid_dtype=None, mode="auto"):
    """The layer's forward: the fused kernel when it takes the case (mode "fused", or "auto" where it is the faster
    one), else the reference's flow -- the weight dequantised to x's dtype (wf_dequant), then the bf16 GEMM
    (wf_linear_bf16 where ``hand_gemm`` says it is the faster one, else torch.nn.functional.linear)."""
    rows = x.numel() // max(1, x.shape[-1]) if x.dim() else 0
    if mode == "auto":
        mode = "fused" if prefer_fused(rows, qtype, oshape[0], oshape[1]) else "dequant"
    if mode == "fused":
        y = fused_linear(x, data, qtype, oshape, bias, mid_dtype)
        if y is not None:
            return y
    w = gguf_dequant.dequantize(data, qtype, oshape, mid_dtype, x.dtype)
    if w is None:
        raise ValueError(f"GGML type {qtype} with shape {tuple(oshape)} is not handled on this path")
    if hand_gemm(rows, int(oshape[0])):
        y = bf16_linear(x, w, bias)
        if y is not None:
            return y
    return torch.nn.functional.linear(x, w, bias)


class GGUFLinear(torch.nn.Module):
    """A linear layer with a GGUF-quantised weight held as raw uint8 blocks (the form ComfyUI-GGUF keeps), so that
    block streaming moves the quantised bytes."""

    def __init__(self, in_features, out_features, qtype=12, bias=True, mode="auto", mid_dtype=None):
        super().__init__()
        q = int(qtype)
        per = 256 if q in gguf_dequant._KFORMATS else 32                 # values per block
        ts = (gguf_dequant._KFORMATS if q in gguf_dequant._KFORMATS else gguf_dequant._FORMATS).get(q, (None, None))[1]
        if ts is None or in_features % per:
            raise ValueError(f"GGML type {qtype} with {in_features} inputs")
        self.in_features, self.out_features, self.qtype = in_features, out_features, q
        self.mode, self.mid_dtype = mode, mid_dtype
        self.weight = torch.nn.Parameter(torch.zeros(out_features * in_features // per * ts, dtype=torch.uint8),
                                         requires_grad=False)
        self.bias = (torch.nn.Parameter(torch.zeros(out_features, dtype=torch.bfloat16), requires_grad=False)
                     if bias else None)

    def forward(self, x):
        return linear(x, self.weight, self.qtype, (self.out_features, self.in_features), self.bias,
                      self.mid_dtype, self.mode)
