"""Synthetic GGUF inputs: block encoders and random-block generators for the benchmarks, the smoke check and the
tests (no part of the hot path: ComfyUI-GGUF hands the kernels blocks from .gguf files).

The encoders turn float32 weights into valid blocks of the GGML layouts the reference decodes
(enhancers/gguf_dequant.py:52-56,195-249): Q8_0 (d = f16(absmax / 127), q = rint(x / d)), and simple deterministic
K-quant encoders (per sub-block min / max -> 6-bit scales and mins against the super-block's f16 d / dmin). They are
input generators, not a reproduction of llama.cpp's search-based quantisers; decoding is what is checked.

``random_blocks`` fills every byte at random and then sets the f16 fields (d, dmin) from a chosen family, so parity
tests see every quant / scale bit pattern.
"""
import numpy as np

TYPE_SIZE = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34, 10: 84, 11: 110, 12: 144, 13: 176, 14: 210}
PER_BLOCK = {2: 32, 3: 32, 6: 32, 7: 32, 8: 32, 10: 256, 11: 256, 12: 256, 13: 256, 14: 256}
# byte offsets of the f16 fields of each format
F16_FIELDS = {2: (0,), 3: (0, 2), 6: (0,), 7: (0, 2), 8: (0,), 10: (80, 82), 11: (108,), 12: (0, 2), 13: (0, 2),
              14: (208,)}


def weights(shape, seed=1234, std=0.02):
    """float32 N(0, std) weights from numpy's PCG64 generator with the given seed."""
    return (np.random.default_rng(seed).standard_normal(size=shape, dtype=np.float32) * np.float32(std))


def _f16(x):
    with np.errstate(over="ignore"):
        return np.asarray(x, dtype=np.float32).astype(np.float16)


def _safe_div(a, b):
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(b != 0, a / np.where(b != 0, b, 1), 0)
    return r.astype(np.float32)


def encode_q8_0(w):
    x = np.asarray(w, dtype=np.float32).reshape(-1, 32)
    d16 = _f16(np.abs(x).max(axis=1) / 127.0)
    d = d16.astype(np.float32)
    q = np.clip(np.rint(_safe_div(x, d[:, None])), -127, 127).astype(np.int8)
    out = np.empty((x.shape[0], 34), dtype=np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:34] = q.view(np.uint8)
    return out.ravel()


def _kscales(x, qmax):
    """Per 32-value sub-block (scale, min) -> 6-bit codes against f16 d / dmin. x: [nb, 8, 32]."""
    mn = np.maximum(0.0, -x.min(axis=2))
    mx = x.max(axis=2)
    sc = np.maximum(mx + mn, 0.0) / qmax
    d16 = _f16(sc.max(axis=1) / 63.0)
    dmin16 = _f16(mn.max(axis=1) / 63.0)
    d, dmin = d16.astype(np.float32), dmin16.astype(np.float32)
    sc6 = np.clip(np.rint(_safe_div(sc, d[:, None])), 0, 63).astype(np.int32)
    m6 = np.clip(np.rint(_safe_div(mn, dmin[:, None])), 0, 63).astype(np.int32)
    step = d[:, None] * sc6
    off = dmin[:, None] * m6
    q = np.clip(np.rint(_safe_div(x + off[:, :, None], step[:, :, None])), 0, qmax).astype(np.int32)
    return d16, dmin16, sc6, m6, q


def _pack_scales(sc6, m6):
    nb = sc6.shape[0]
    s = np.zeros((nb, 12), dtype=np.int32)
    s[:, 0:4] = sc6[:, 0:4] | ((sc6[:, 4:8] >> 4) << 6)
    s[:, 4:8] = m6[:, 0:4] | ((m6[:, 4:8] >> 4) << 6)
    s[:, 8:12] = (sc6[:, 4:8] & 0xF) | ((m6[:, 4:8] & 0xF) << 4)
    return s.astype(np.uint8)


def encode_q4_k(w):
    x = np.asarray(w, dtype=np.float32).reshape(-1, 8, 32)
    nb = x.shape[0]
    d16, dmin16, sc6, m6, q = _kscales(x, 15)
    out = np.empty((nb, 144), dtype=np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = dmin16.view(np.uint8).reshape(-1, 2)
    out[:, 4:16] = _pack_scales(sc6, m6)
    qs = q[:, 0::2, :] | (q[:, 1::2, :] << 4)           # pair p: low nibble sub 2p, high nibble sub 2p + 1
    out[:, 16:144] = qs.reshape(nb, 128).astype(np.uint8)
    return out.ravel()


def encode_q5_k(w):
    x = np.asarray(w, dtype=np.float32).reshape(-1, 8, 32)
    nb = x.shape[0]
    d16, dmin16, sc6, m6, q = _kscales(x, 31)
    out = np.empty((nb, 176), dtype=np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = dmin16.view(np.uint8).reshape(-1, 2)
    out[:, 4:16] = _pack_scales(sc6, m6)
    qh = np.zeros((nb, 32), dtype=np.int32)
    for sub in range(8):
        qh |= ((q[:, sub, :] >> 4) & 1) << sub
    out[:, 16:48] = qh.astype(np.uint8)
    ql = q & 0xF
    out[:, 48:176] = (ql[:, 0::2, :] | (ql[:, 1::2, :] << 4)).reshape(nb, 128).astype(np.uint8)
    return out.ravel()


def encode_q6_k(w):
    x = np.asarray(w, dtype=np.float32).reshape(-1, 16, 16)
    nb = x.shape[0]
    sc = np.abs(x).max(axis=2) / 31.0
    d16 = _f16(sc.max(axis=1) / 127.0)
    d = d16.astype(np.float32)
    sc8 = np.clip(np.rint(_safe_div(sc, d[:, None])), -128, 127).astype(np.int32)
    step = d[:, None] * sc8
    q = (np.clip(np.rint(_safe_div(x, step[:, :, None])), -32, 31) + 32).astype(np.int32).reshape(nb, 256)
    out = np.zeros((nb, 210), dtype=np.uint8)
    v = np.arange(256)
    h, r = v // 128, v % 128
    ql = np.zeros((nb, 128), dtype=np.int32)
    qh = np.zeros((nb, 64), dtype=np.int32)
    for i in range(256):
        ql[:, h[i] * 64 + r[i] % 64] |= (q[:, i] & 0xF) << (4 * (r[i] // 64))
        qh[:, h[i] * 32 + r[i] % 32] |= (q[:, i] >> 4) << (2 * (r[i] // 32))
    out[:, 0:128] = ql.astype(np.uint8)
    out[:, 128:192] = qh.astype(np.uint8)
    out[:, 192:208] = sc8.astype(np.int8).view(np.uint8)
    out[:, 208:210] = d16.view(np.uint8).reshape(-1, 2)
    return out.ravel()


def _legacy(w, qtype):
    """Q4_0 / Q5_0 (symmetric: d = f16(v / -2^(bits-1)) where v is the block's value of largest magnitude, q in
    [0, 2^bits) with x ~ d * (q - 2^(bits-1))) and Q4_1 / Q5_1 (d = f16((max - min) / (2^bits - 1)), m = f16(min),
    x ~ d * q + m), the blocks laid out as the decoder reads them (enhancers/gguf_dequant.py:145-160): nibble v / 16 of
    qs[v % 16], bit v of qh."""
    x = np.asarray(w, dtype=np.float32).reshape(-1, 32)
    nb = x.shape[0]
    bits = 5 if qtype in (6, 7) else 4
    top = (1 << bits) - 1
    if qtype in (2, 6):
        idx = np.abs(x).argmax(axis=1)
        v = x[np.arange(nb), idx]
        d16 = _f16(v / -float(1 << (bits - 1)))
        d = d16.astype(np.float32)
        q = np.clip(np.rint(_safe_div(x, d[:, None])) + (1 << (bits - 1)), 0, top).astype(np.int32)
        m16 = None
    else:
        lo, hi = x.min(axis=1), x.max(axis=1)
        d16 = _f16((hi - lo) / float(top))
        m16 = _f16(lo)
        d, m = d16.astype(np.float32), m16.astype(np.float32)
        q = np.clip(np.rint(_safe_div(x - m[:, None], d[:, None])), 0, top).astype(np.int32)
    ts = TYPE_SIZE[qtype]
    out = np.zeros((nb, ts), dtype=np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    o = 2
    if m16 is not None:
        out[:, 2:4] = m16.view(np.uint8).reshape(-1, 2)
        o = 4
    if bits == 5:
        qh = np.zeros(nb, dtype=np.uint64)
        for v in range(32):
            qh |= ((q[:, v] >> 4) & 1).astype(np.uint64) << np.uint64(v)
        out[:, o:o + 4] = qh.astype(np.uint32).view(np.uint8).reshape(-1, 4)
        o += 4
    qn = q & 0xF
    out[:, o:o + 16] = (qn[:, 0:16] | (qn[:, 16:32] << 4)).astype(np.uint8)
    return out.ravel()


def encode_q4_0(w):
    return _legacy(w, 2)


def encode_q4_1(w):
    return _legacy(w, 3)


def encode_q5_0(w):
    return _legacy(w, 6)


def encode_q5_1(w):
    return _legacy(w, 7)


ENCODERS = {2: encode_q4_0, 3: encode_q4_1, 6: encode_q5_0, 7: encode_q5_1, 8: encode_q8_0, 12: encode_q4_k,
            13: encode_q5_k, 14: encode_q6_k}


def encode(w, qtype):
    return ENCODERS[int(qtype)](w)


def f16_family(n, rng, family):
    """n float16 bit patterns: 'normal' (|d| in 2^-14 .. 2^-4, either sign: typical scales), 'finite' (any finite
    f16, subnormals and +-0 included), 'edge' (a fixed set: +-0, subnormal extremes, 1, 65504)."""
    if family == "normal":
        mag = rng.uniform(-14, -4, size=n)
        v = (2.0 ** mag) * rng.choice([-1.0, 1.0], size=n)
        return _f16(v).view(np.uint16)
    if family == "finite":
        bits = rng.integers(0, 1 << 16, size=n, dtype=np.uint32).astype(np.uint16)
        bad = (bits & 0x7C00) == 0x7C00
        bits[bad] &= 0x83FF                      # inf / nan -> a subnormal of the same sign
        return bits
    if family == "edge":
        edge = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x03FF, 0x0400, 0x3C00, 0xBC00, 0x7BFF, 0xFBFF, 0x3555,
                         0x2E66], dtype=np.uint16)
        return edge[rng.integers(0, edge.size, size=n)]
    raise ValueError(family)


def random_blocks(qtype, nblocks, seed=0, family="normal"):
    """nblocks blocks of random bytes with their f16 fields drawn from ``family``."""
    q = int(qtype)
    rng = np.random.default_rng(seed)
    ts = TYPE_SIZE[q]
    b = rng.integers(0, 256, size=(nblocks, ts), dtype=np.uint16).astype(np.uint8)
    for off in F16_FIELDS[q]:
        b[:, off:off + 2] = f16_family(nblocks, rng, family).view(np.uint8).reshape(-1, 2)
    return b.ravel()
