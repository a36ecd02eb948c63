"""ORACLE (test infrastructure only): numpy restatement of the GGUF dequantisation in the block-loop form of the
GGML formats (sub-block pairs of 64 values for Q4_K / Q5_K, 128-value halves for Q6_K / Q3_K / Q2_K), with the
reference's rounding chain: every product and sum rounded to the dequant dtype MID, then the cast to OUT
(enhancers/gguf_dequant.py:16-23,136-256).

It computes the same bits as ``wf_oracle.c`` through a different index formulation, so an index slip in either
shows up when the two are compared. Rounding: float16 through numpy's own IEEE conversion, bfloat16 through the
reference's bit rule (enhancers/gguf_dequant.py:78-81), float32 the identity.
"""
import numpy as np

F16, BF16, F32 = 0, 1, 2
LEGACY = {2: ("Q4_0", 18), 3: ("Q4_1", 20), 6: ("Q5_0", 22), 7: ("Q5_1", 24), 8: ("Q8_0", 34)}
KQUANT = {10: ("Q2_K", 84), 11: ("Q3_K", 110), 12: ("Q4_K", 144), 13: ("Q5_K", 176), 14: ("Q6_K", 210)}


def block_bytes(qtype):
    q = int(qtype)
    if q in LEGACY:
        return LEGACY[q][1], 32
    if q in KQUANT:
        return KQUANT[q][1], 256
    raise KeyError(qtype)


def bf16_bits_rule(x):
    """(u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000 on float32 bits -> float32 (enhancers/gguf_dequant.py:78-81)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def R(x, D):
    x = np.asarray(x, dtype=np.float32)
    if D == F16:
        with np.errstate(over="ignore"):
            return x.astype(np.float16).astype(np.float32)
    if D == BF16:
        return bf16_bits_rule(x)
    return x


def to_out_bits(x, D):
    """Rounded float32 values -> the stored representation (uint16 bits for f16/bf16, float32 for f32)."""
    if D == F16:
        with np.errstate(over="ignore"):
            return x.astype(np.float16).view(np.uint16)
    if D == BF16:
        return (bf16_bits_rule(x).view(np.uint32) >> 16).astype(np.uint16)
    return x.astype(np.float32)


def _f16(blocks, off):
    return blocks[:, off:off + 2].copy().view(np.float16).astype(np.float32)[:, 0]


def _mul(a, b):
    with np.errstate(over="ignore", invalid="ignore"):
        return np.multiply(a, b, dtype=np.float32)


def _sub(a, b):
    with np.errstate(over="ignore", invalid="ignore"):
        return np.subtract(a, b, dtype=np.float32)


def _add(a, b):
    with np.errstate(over="ignore", invalid="ignore"):
        return np.add(a, b, dtype=np.float32)


def _scale_min_k4(s, j):
    """GGML get_scale_min_k4 (j = sub-block 0..7) over a [nb, 12] byte array: (sc, m) as int arrays."""
    s = s.astype(np.int32)
    if j < 4:
        return s[:, j] & 63, s[:, j + 4] & 63
    return (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 6) << 4), (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)


def dequant(raw, qtype, mid, out):
    """Flat dequantised values of dtype ``out`` (as from to_out_bits) of the blocks in ``raw`` (uint8)."""
    q = int(qtype)
    ts, per = block_bytes(q)
    raw = np.asarray(raw, dtype=np.uint8).ravel()
    assert raw.size % ts == 0
    b = raw.reshape(-1, ts)
    nb = b.shape[0]
    y = np.empty((nb, per), dtype=np.float32)
    bi = b.astype(np.int32)
    if q in LEGACY:
        d = R(_f16(b, 0), mid)[:, None]
        if q == 8:
            qv = b[:, 2:34].view(np.int8).astype(np.float32)
        else:
            qs_off = {2: 2, 3: 4, 6: 6, 7: 8}[q]
            qs = bi[:, qs_off:qs_off + 16]
            nib = np.concatenate([qs & 0xF, qs >> 4], axis=1)           # value j < 16: low nibble of byte j
            if q in (6, 7):
                qh_off = {6: 2, 7: 4}[q]
                qh = (bi[:, qh_off] | (bi[:, qh_off + 1] << 8) | (bi[:, qh_off + 2] << 16)
                      | (bi[:, qh_off + 3] << 24)).astype(np.int64)  # 32-bit little-endian qh
                bits = (qh[:, None] >> np.arange(32)[None, :]) & 1
                nib = nib | (bits.astype(np.int32) << 4)
            sub = {2: 8, 3: 0, 6: 16, 7: 0}[q]
            qv = (nib - sub).astype(np.float32)
        x = R(_mul(d, qv), mid)
        if q in (3, 7):
            x = R(_add(x, R(_f16(b, 2), mid)[:, None]), mid)
        y[:] = R(x, out)
        return to_out_bits(y.ravel(), out)
    if q in (12, 13):
        d = R(_f16(b, 0), mid)
        dmin = R(_f16(b, 2), mid)
        s = b[:, 4:16]
        qs = bi[:, 16:144] if q == 12 else bi[:, 48:176]
        qh = bi[:, 16:48] if q == 13 else None
        for j in range(4):                      # pairs of sub-blocks: 64 values, 32 bytes of qs
            sc1, m1 = _scale_min_k4(s, 2 * j)
            sc2, m2 = _scale_min_k4(s, 2 * j + 1)
            d1 = R(_mul(d, sc1.astype(np.float32)), mid)[:, None]
            dm1 = R(_mul(dmin, m1.astype(np.float32)), mid)[:, None]
            d2 = R(_mul(d, sc2.astype(np.float32)), mid)[:, None]
            dm2 = R(_mul(dmin, m2.astype(np.float32)), mid)[:, None]
            ql = qs[:, 32 * j:32 * j + 32]
            lo, hi = ql & 0xF, ql >> 4
            if qh is not None:
                lo = lo + (((qh >> (2 * j)) & 1) << 4)
                hi = hi + (((qh >> (2 * j + 1)) & 1) << 4)
            y[:, 64 * j:64 * j + 32] = R(_sub(R(_mul(d1, lo.astype(np.float32)), mid), dm1), mid)
            y[:, 64 * j + 32:64 * j + 64] = R(_sub(R(_mul(d2, hi.astype(np.float32)), mid), dm2), mid)
    elif q == 14:
        ql = bi[:, 0:128]
        qh = bi[:, 128:192]
        sc = b[:, 192:208].view(np.int8).astype(np.float32)
        d = R(_f16(b, 208), mid)
        for n in range(2):                      # 128-value halves: 64 bytes of ql, 32 of qh, 8 scales
            L = ql[:, 64 * n:64 * n + 64]
            H = qh[:, 32 * n:32 * n + 32]
            q1 = ((L[:, 0:32] & 0xF) | (((H >> 0) & 3) << 4)) - 32
            q2 = ((L[:, 32:64] & 0xF) | (((H >> 2) & 3) << 4)) - 32
            q3 = ((L[:, 0:32] >> 4) | (((H >> 4) & 3) << 4)) - 32
            q4 = ((L[:, 32:64] >> 4) | (((H >> 6) & 3) << 4)) - 32
            for part, qq in enumerate((q1, q2, q3, q4)):
                for half in range(2):           # scale index: 8n + 2 * part + l // 16
                    dsc = R(_mul(d, sc[:, 8 * n + 2 * part + half]), mid)[:, None]
                    seg = qq[:, 16 * half:16 * half + 16].astype(np.float32)
                    o = 128 * n + 32 * part + 16 * half
                    y[:, o:o + 16] = R(_mul(dsc, seg), mid)
    elif q == 11:
        hm = bi[:, 0:32]
        qs = bi[:, 32:96]
        a = bi[:, 96:108]
        d_all = R(_f16(b, 108), mid)
        # 16 six-bit scales: low nibble from a[0..7] (two per byte), high 2 bits from a[8..11]
        scl = np.empty((nb, 16), dtype=np.int32)
        for i in range(16):
            low = (a[:, i % 8] >> (4 * (i // 8))) & 0xF
            high = (a[:, 8 + i % 4] >> (2 * (i // 4))) & 3
            scl[:, i] = (low | (high << 4)) - 32
        m = 1
        isx = 0
        for n in range(2):
            Q = qs[:, 32 * n:32 * n + 32]
            for shift in (0, 2, 4, 6):
                for half in range(2):
                    dl = R(_mul(d_all, scl[:, isx].astype(np.float32)), mid)[:, None]
                    isx += 1
                    l = slice(16 * half, 16 * half + 16)
                    qv = ((Q[:, l] >> shift) & 3) - np.where(hm[:, l] & m, 0, 4)
                    o = 128 * n + 32 * (shift // 2) + 16 * half
                    y[:, o:o + 16] = R(_mul(dl, qv.astype(np.float32)), mid)
                m <<= 1
    elif q == 10:
        sc = bi[:, 0:16]
        qs = bi[:, 16:80]
        d = R(_f16(b, 80), mid)
        mn = R(_f16(b, 82), mid)
        isx = 0
        for n in range(2):
            Q = qs[:, 32 * n:32 * n + 32]
            for shift in (0, 2, 4, 6):
                for half in range(2):
                    s = sc[:, isx]
                    isx += 1
                    dl = R(_mul(d, (s & 0xF).astype(np.float32)), mid)[:, None]
                    ml = R(_mul(mn, (s >> 4).astype(np.float32)), mid)[:, None]
                    l = slice(16 * half, 16 * half + 16)
                    qv = ((Q[:, l] >> shift) & 3).astype(np.float32)
                    o = 128 * n + 32 * (shift // 2) + 16 * half
                    y[:, o:o + 16] = R(_sub(R(_mul(dl, qv), mid), ml), mid)
    else:
        raise KeyError(qtype)
    return to_out_bits(R(y.ravel(), out), out)


def bits_to_f32(bits, D):
    """Stored representation -> float32 values (exact)."""
    if D == F16:
        return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)
    if D == BF16:
        return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
    return np.asarray(bits, dtype=np.float32)


def gemm_ref_f64(x, w, bias=None):
    """y = x @ w.T (+ bias) in float64: the reference for bf16-MFMA GEMMs (tolerance, not bits)."""
    y = np.asarray(x, dtype=np.float64) @ np.asarray(w, dtype=np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)[None, :]
    return y


# ----------------------------------------------------------------------------------- ConvRot row quantisation
# Sum orders of one radix-4 stage (a, b, c, d) -> 4 outputs. "ltr" is the reference's: every output summed left
# to right (enhancers/fused_block.py:40-43, enhancers/fused_kernels.py:65-81). The others are plausible slips
# (pairwise sums, right-to-left) kept so tests can show which inputs tell the orders apart.
_STAGE_ORDERS = {
    "ltr": lambda a, b, c, d: (((a + b) + c) - d, ((a + b) - c) + d, ((a - b) + c) + d, ((-a + b) + c) + d),
    "pair": lambda a, b, c, d: ((a + b) + (c - d), (a + b) + (d - c), (a - b) + (c + d), (b - a) + (c + d)),
    "rtl": lambda a, b, c, d: (a + (b + (c - d)), a + (b + (d - c)), a + ((c + d) - b), ((b + c) + d) - a),
}


def quant_rows_convrot(x_bf16_bits, order="ltr"):
    """The ConvRot-256 row quantisation of _quant_row with PRE_NONE (enhancers/fused_kernels.py:137-174) in numpy
    float32, every operation rounded on its own: radix-4 stages of stride 1, 4, 16, 64 in the given sum order,
    * 0.0625, amax clamped to 3.38953139e38, scale = max(amax / 127, 1e-30), q = clamp(rint(bf16(bf16(y) /
    bf16(scale))), -128, 127) (IEEE division, ties to even). x: bf16 bits [M, K], K % 256 == 0.
    Returns (int8 [M, K], float32 scales [M])."""
    x = np.asarray(x_bf16_bits, dtype=np.uint16)
    M, K = x.shape
    y = (x.astype(np.uint32) << 16).view(np.float32).reshape(M, K // 256, 256)
    fn = _STAGE_ORDERS[order]
    with np.errstate(over="ignore", invalid="ignore"):
        for S in (1, 4, 16, 64):
            v = y.reshape(M, K // 256, 256 // (4 * S), 4, S)
            outs = fn(v[:, :, :, 0], v[:, :, :, 1], v[:, :, :, 2], v[:, :, :, 3])
            y = np.stack(outs, axis=3).astype(np.float32).reshape(M, K // 256, 256)
        y = (y.reshape(M, K) * np.float32(0.0625)).astype(np.float32)
        amax = np.minimum(np.abs(y).max(axis=1), np.float32(3.38953139e38)).astype(np.float32)
        scale = np.maximum((amax / np.float32(127.0)).astype(np.float32), np.float32(1e-30)).astype(np.float32)
        sb = bf16_bits_rule(scale)
        q = np.rint(bf16_bits_rule((bf16_bits_rule(y) / sb[:, None]).astype(np.float32)))
    return np.clip(q, -128, 127).astype(np.int8), scale
