"""ORACLE / CPU BASELINE (test infrastructure only): torch-CPU restatement of ComfyUI-GGUF's dequantisation op chain.

This is the path the reference takes for CPU tensors: its ``dequantize`` returns None when the data is not on the
GPU (enhancers/gguf_dequant.py:300,308), so ComfyUI-GGUF's own torch code (``dequant.py`` of city96/ComfyUI-GGUF,
checkout 6ea2651; not vendored in the reference) runs. The reference's kernel is documented as the same operations,
dtypes and roundings as that chain (enhancers/gguf_dequant.py:3-7,16-23): each torch op on float16 / bfloat16 tensors
computes in float32 and rounds to the tensor dtype, then ``.to(out)``.

Written in the vectorised tensor form ComfyUI-GGUF uses (split the block bytes, view, shift by a broadcast tensor,
mask, multiply, subtract), a third formulation next to ``wf_oracle.c`` and ``np_oracle``. Only Q8_0 and the
K-quants Q4_K / Q5_K / Q6_K (the hot-path formats) are restated here.
"""
import torch

QK_K = 256
K_SCALE_SIZE = 12
TYPE_SIZE = {8: 34, 12: 144, 13: 176, 14: 210}
BLOCK_SIZE = {8: 32, 12: 256, 13: 256, 14: 256}


def _split(blocks, *sizes):
    n_max = blocks.shape[1]
    rest = n_max - sum(sizes)
    return torch.split(blocks, list(sizes) + [rest], dim=1)


def _f16(t, dtype):
    return t.contiguous().view(torch.float16).to(dtype)


def _scale_min(scales):
    n = scales.shape[0]
    s = scales.view(torch.uint8).reshape((n, 3, 4))
    d, m, m_d = torch.split(s, 1, dim=-2)
    sc = torch.cat([d & 0x3F, (m_d & 0x0F) | ((d >> 2) & 0x30)], dim=-1)
    mn = torch.cat([m & 0x3F, (m_d >> 4) | ((m >> 2) & 0x30)], dim=-1)
    return sc.reshape((n, 8)), mn.reshape((n, 8))


def _q8_0(blocks, dtype):
    d, x = _split(blocks, 2)
    d = _f16(d, dtype)
    x = x.contiguous().view(torch.int8)
    return d * x


def _q4_k(blocks, dtype):
    n = blocks.shape[0]
    d, dmin, scales, qs = _split(blocks, 2, 2, K_SCALE_SIZE)
    d = _f16(d, dtype)
    dmin = _f16(dmin, dtype)
    sc, m = _scale_min(scales)
    d = (d * sc).reshape((n, -1, 1))
    dm = (dmin * m).reshape((n, -1, 1))
    qs = qs.reshape((n, -1, 1, 32)) >> torch.tensor([0, 4], dtype=torch.uint8).reshape((1, 1, 2, 1))
    qs = (qs & 0x0F).reshape((n, -1, 32))
    return (d * qs - dm).reshape((n, QK_K))


def _q5_k(blocks, dtype):
    n = blocks.shape[0]
    d, dmin, scales, qh, qs = _split(blocks, 2, 2, K_SCALE_SIZE, QK_K // 8)
    d = _f16(d, dtype)
    dmin = _f16(dmin, dtype)
    sc, m = _scale_min(scales)
    d = (d * sc).reshape((n, -1, 1))
    dm = (dmin * m).reshape((n, -1, 1))
    ql = qs.reshape((n, -1, 1, 32)) >> torch.tensor([0, 4], dtype=torch.uint8).reshape((1, 1, 2, 1))
    qh = qh.reshape((n, -1, 1, 32)) >> torch.arange(8, dtype=torch.uint8).reshape((1, 1, 8, 1))
    ql = (ql & 0x0F).reshape((n, -1, 32))
    qh = (qh & 0x01).reshape((n, -1, 32))
    q = ql | (qh << 4)
    return (d * q - dm).reshape((n, QK_K))


def _q6_k(blocks, dtype):
    n = blocks.shape[0]
    ql, qh, scales, d = _split(blocks, QK_K // 2, QK_K // 4, QK_K // 16)
    scales = scales.contiguous().view(torch.int8).to(dtype)
    d = _f16(d, dtype)
    d = (d * scales).reshape((n, QK_K // 16, 1))
    ql = ql.reshape((n, -1, 1, 64)) >> torch.tensor([0, 4], dtype=torch.uint8).reshape((1, 1, 2, 1))
    ql = (ql & 0x0F).reshape((n, -1, 32))
    qh = qh.reshape((n, -1, 1, 32)) >> torch.tensor([0, 2, 4, 6], dtype=torch.uint8).reshape((1, 1, 4, 1))
    qh = (qh & 0x03).reshape((n, -1, 32))
    q = (ql | (qh << 4)).to(torch.int8) - 32
    q = q.reshape((n, QK_K // 16, -1))
    return (d * q).reshape((n, QK_K))


_CHAIN = {8: _q8_0, 12: _q4_k, 13: _q5_k, 14: _q6_k}


def dequantize(raw_u8, qtype, oshape, mid_dtype=None, out_dtype=None):
    """ComfyUI-GGUF ``dequantize(data, qtype, oshape, dtype=mid).to(out)`` on CPU: raw uint8 tensor of blocks ->
    tensor of shape ``oshape``. MID defaults to float16 and OUT to MID, as in enhancers/gguf_dequant.py:302-303."""
    q = int(qtype)
    mid = mid_dtype if mid_dtype is not None else torch.float16
    out = out_dtype if out_dtype is not None else mid
    ts = TYPE_SIZE[q]
    blocks = raw_u8.reshape(-1).view(torch.uint8).reshape(-1, ts)
    y = _CHAIN[q](blocks, mid)
    return y.reshape(tuple(oshape)).to(out)


def linear_bf16(x, w, bias=None):
    """The CPU F.linear ComfyUI-GGUF runs after the dequantisation (bf16 in, bf16 out)."""
    return torch.nn.functional.linear(x, w, bias)
