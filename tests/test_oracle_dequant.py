"""Pins the oracle's dequantisation (enhancers/gguf_dequant.py:136-256 of the reference).

* Three formulations agree bit for bit on random blocks of every format, every MID x OUT dtype pair and three
  families of scales (typical, any finite float16 incl. subnormals and +-0, edge values): the C restatement of the
  reference's flat-index formulas, the numpy restatement in GGML's block-loop form, and (hot formats) the
  torch-CPU op chain of ComfyUI-GGUF.
* Q8_0 against its closed form on all 65536 float16 scales x 256 quants, rounded by numpy / torch.
* Hand-computed known answers for Q8_0, Q4_K, Q5_K, Q6_K and the legacy Q4_0 / Q4_1 / Q5_0 / Q5_1 blocks (index
  layout of each format).
* The 6-bit scale / min packing round trip for all 64 x 64 pairs of every sub-block.
* encode -> decode stays within the quantisation step of the source weights (a dropped or sign-flipped term fails).
"""
import numpy as np
import pytest
import torch

from conftest import sub
from oracle import lib, np_oracle, torch_chain

encode = sub("gguf_encode")

F16, BF16, F32 = 0, 1, 2
TD = {F16: torch.float16, BF16: torch.bfloat16, F32: torch.float32}
ALL_TYPES = [2, 3, 6, 7, 8, 10, 11, 12, 13, 14]
PAIRS = [(m, o) for m in range(3) for o in range(3)]


def _same(a, b, D):
    """Bitwise equality, NaNs compared as NaN (their payloads are not part of the contract)."""
    fa, fb = np_oracle.bits_to_f32(a, D), np_oracle.bits_to_f32(b, D)
    both_nan = np.isnan(fa) & np.isnan(fb)
    return bool(np.all((np.asarray(a).view(np.uint8).reshape(len(fa), -1)
                        == np.asarray(b).view(np.uint8).reshape(len(fb), -1)).all(axis=1) | both_nan))


def _torch_bits(t, D):
    if D == F32:
        return t.numpy().astype(np.float32)
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("qtype", ALL_TYPES)
@pytest.mark.parametrize("family", ["normal", "finite", "edge"])
def test_formulations_agree(qtype, family):
    raw = encode.random_blocks(qtype, 160, seed=qtype * 7 + len(family), family=family)
    n = raw.size // encode.TYPE_SIZE[qtype] * encode.PER_BLOCK[qtype]
    for mid, out in PAIRS:
        c = lib.dequant(raw, qtype, mid, out, n)
        npv = np_oracle.dequant(raw, qtype, mid, out)
        assert _same(c, npv, out), (qtype, family, mid, out)
        if qtype in torch_chain.TYPE_SIZE:
            t = torch_chain.dequantize(torch.from_numpy(raw.copy()), qtype, (n,), TD[mid], TD[out])
            assert _same(c, _torch_bits(t, out), out), (qtype, family, mid, out, "torch chain")


def _q8_all_cases():
    """Blocks covering every float16 d (finite) with every int8 quant: 8 blocks of 32 quants per d."""
    d = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    d = d[(d & 0x7C00) != 0x7C00]                       # finite scales
    q = np.arange(256, dtype=np.int32).astype(np.int8).view(np.uint8).reshape(8, 32)
    blocks = np.empty((d.size, 8, 34), dtype=np.uint8)
    blocks[:, :, 0:2] = d.view(np.uint8).reshape(-1, 1, 2)
    blocks[:, :, 2:] = q[None, :, :]
    return blocks.reshape(-1, 34), np.repeat(d, 8 * 32), np.tile(q.view(np.int8).ravel(), d.size)


def _round_f64(x, D):
    """Single rounding of float64 values to dtype D (numpy for f16, torch RNE for bf16 / f32)."""
    if D == F16:
        with np.errstate(all="ignore"):
            return x.astype(np.float16).astype(np.float64)
    t = torch.from_numpy(x)
    return t.to(torch.bfloat16 if D == BF16 else torch.float32).to(torch.float64).numpy()


@pytest.mark.parametrize("mid", [F16, BF16, F32])
def test_q8_0_closed_form_all_scales(mid):
    blocks, dbits, q = _q8_all_cases()
    d = dbits.view(np.float16).astype(np.float64)
    # R_MID(d) * q is exact in float64; the reference's float32 product of these is exact too (<= 19 bits)
    x = _round_f64(_round_f64(d, mid) * q.astype(np.float64), mid)
    for out in (F16, BF16, F32):
        ref = _round_f64(x, out)
        got = np_oracle.bits_to_f32(lib.dequant(blocks.ravel(), 8, mid, out, q.size), out).astype(np.float64)
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan], ref[~nan]), (mid, out)
        # signed zeros: -0.0 where the exact product is a negative zero
        z = (ref == 0) & ~nan
        assert np.array_equal(np.signbit(got[z]), np.signbit(ref[z]))


def _f16b(v):
    return np.array([v], dtype=np.float16).view(np.uint8)


def test_kat_q8_0():
    b = np.zeros(34, dtype=np.uint8)
    b[0:2] = _f16b(0.25)
    b[2:] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    got = np_oracle.bits_to_f32(lib.dequant(b, 8, F16, F32, 32), F32)
    assert np.array_equal(got, 0.25 * np.arange(-16, 16, dtype=np.float32))


def _kat_k_block(qtype):
    """A Q4_K / Q5_K super-block built by hand: d = 1, dmin = 0.5, sub-block s has scale s + 1 and min s; quant
    byte k = (k % 16) | ((15 - k % 16) << 4); Q5_K: qh[l] = 0b10100101 rotated by l."""
    sc = np.arange(1, 9)
    mn = np.arange(0, 8)
    s = np.zeros(12, dtype=np.int64)
    for j in range(4):  # GGML packing: low sub-blocks in the 6 low bits, high ones split into a nibble + 2 bits
        s[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    qs = np.array([(k % 16) | ((15 - k % 16) << 4) for k in range(128)], dtype=np.uint8)
    head = np.concatenate([_f16b(1.0), _f16b(0.5), s.astype(np.uint8)])
    qh = np.array([((0xA5 << (l % 8)) | (0xA5 >> (8 - l % 8))) & 0xFF for l in range(32)], dtype=np.uint8)
    blk = np.concatenate([head, qs]) if qtype == 12 else np.concatenate([head, qh, qs])
    expect = np.empty(256, dtype=np.float32)
    for v in range(256):
        sub, l = v // 32, v % 32
        byte = int(qs[32 * (sub // 2) + l])
        nib = byte & 0xF if sub % 2 == 0 else byte >> 4
        if qtype == 13:
            nib += 16 * ((int(qh[l]) >> sub) & 1)
        expect[v] = (1.0 * sc[sub]) * nib - 0.5 * mn[sub]   # exact in float16 and float32
    return blk, expect


@pytest.mark.parametrize("qtype", [12, 13])
def test_kat_q4_k_q5_k(qtype):
    blk, expect = _kat_k_block(qtype)
    for mid in (F16, BF16, F32):
        got = np_oracle.bits_to_f32(lib.dequant(blk, qtype, mid, F32, 256), F32)
        # every product is an exact small number in each dtype; only the final subtraction can round, and only in
        # bfloat16 (8 significant bits): round the exact value once there
        ref = expect if mid != BF16 else torch.from_numpy(expect).to(torch.bfloat16).float().numpy()
        assert np.array_equal(got, ref), mid


def test_kat_q6_k():
    ql = np.array([(k * 7) & 0xFF for k in range(128)], dtype=np.uint8)
    qh = np.array([(k * 13 + 5) & 0xFF for k in range(64)], dtype=np.uint8)
    sc = np.arange(-8, 8, dtype=np.int8)
    blk = np.concatenate([ql, qh, sc.view(np.uint8), _f16b(0.125)])
    expect = np.empty(256, dtype=np.float32)
    for v in range(256):
        half, r = v // 128, v % 128
        byte = int(ql[64 * half + r % 64])
        lo = byte & 0xF if r < 64 else byte >> 4
        hi = (int(qh[32 * half + r % 32]) >> (2 * (r // 32))) & 3
        expect[v] = (0.125 * sc[v // 16]) * ((lo | (hi << 4)) - 32)
    for mid in (F16, BF16, F32):
        got = np_oracle.bits_to_f32(lib.dequant(blk, 14, mid, F32, 256), F32)
        assert np.array_equal(got, expect), mid


def test_scale_min_roundtrip_all_pairs():
    """GGML's 12-byte packing of eight (6-bit scale, 6-bit min) pairs, decoded by the oracle: every pair of every
    sub-block comes back."""
    L = lib.load()
    import ctypes
    sc_out, m_out = ctypes.c_int(), ctypes.c_int()
    rng = np.random.default_rng(5)
    for sc_val in range(64):
        for m_val in range(64):
            sc6 = rng.integers(0, 64, size=(1, 8))
            m6 = rng.integers(0, 64, size=(1, 8))
            sub = (sc_val + m_val) % 8
            sc6[0, sub], m6[0, sub] = sc_val, m_val
            packed = encode._pack_scales(sc6, m6).ravel()
            L.wfo_scale_min(packed.ctypes.data, sub, ctypes.byref(sc_out), ctypes.byref(m_out))
            assert (sc_out.value, m_out.value) == (sc_val, m_val)


@pytest.mark.parametrize("qtype", [2, 3, 6, 7, 8, 12, 13, 14])
def test_encode_decode_within_step(qtype):
    w = encode.weights((64, 512), seed=3)
    raw = encode.encode(w, qtype)
    got = np_oracle.bits_to_f32(lib.dequant(raw, qtype, F32, F32, w.size), F32).reshape(w.shape)
    err = np.abs(got - w)
    amax = np.abs(w).max()
    bound = {2: amax / 8, 3: amax * 2 / 15, 6: amax / 16, 7: amax * 2 / 31, 8: amax / 127, 12: amax * 2 / 15,
             13: amax * 2 / 31, 14: amax / 31}[qtype]
    assert err.max() <= bound, (qtype, err.max(), bound)
    assert np.abs(got - w).mean() < 0.3 * bound


def test_rejects_mismatched_sizes():
    raw = encode.random_blocks(12, 4)
    with pytest.raises(ValueError):
        lib.dequant(raw, 12, F16, BF16, 4 * 256 + 1)
    with pytest.raises(ValueError):
        lib.dequant(raw[:-1], 12, F16, BF16, 4 * 256)


@pytest.mark.parametrize("qtype", [2, 3, 6, 7])
def test_kat_legacy(qtype):
    """Q4_0 / Q4_1 / Q5_0 / Q5_1 blocks built by hand: d = 0.5, m = -3 (Q4_1 / Q5_1), quant byte k = k | ((15 - k) <<
    4), qh = 0xA5C3F00F (Q5_x). Value v: nibble v // 16 of qs[v % 16] (the low nibbles are values 0..15), bit v of qh
    as bit 4; q - 8 (Q4_0) or q - 16 (Q5_0)."""
    qs = np.array([k | ((15 - k) << 4) for k in range(16)], dtype=np.uint8)
    qh = np.array([0xA5C3F00F], dtype="<u4").view(np.uint8)
    head = [_f16b(0.5)]
    if qtype in (3, 7):
        head.append(_f16b(-3.0))
    if qtype in (6, 7):
        head.append(qh)
    blk = np.concatenate(head + [qs])
    assert blk.size == encode.TYPE_SIZE[qtype]
    expect = np.empty(32, dtype=np.float32)
    for v in range(32):
        nib = int(qs[v % 16]) & 0xF if v < 16 else int(qs[v % 16]) >> 4
        if qtype in (6, 7):
            nib |= ((0xA5C3F00F >> v) & 1) << 4
        sub = {2: 8, 6: 16}.get(qtype, 0)
        expect[v] = 0.5 * (nib - sub) + (-3.0 if qtype in (3, 7) else 0.0)   # exact in every dtype
    for mid in (F16, BF16, F32):
        got = np_oracle.bits_to_f32(lib.dequant(blk, qtype, mid, F32, 32), F32)
        assert np.array_equal(got, expect), (qtype, mid)


def test_kat_q2_k():
    """A Q2_K super-block packed the way GGML writes it: value v = 128n + 32s + l sits at bits 2s of qs[32n + l],
    sub-block v // 16 has (scale, min) in the low / high nibble of scale byte v // 16; d = 0.5, dmin = 0.25. The
    expected values 0.5 * scale * q - 0.25 * min are exact in every dtype."""
    rng = np.random.default_rng(21)
    q = rng.integers(0, 4, size=256)
    sc, mn = rng.integers(0, 16, size=16), rng.integers(0, 16, size=16)
    qs = np.zeros(64, dtype=np.int64)
    for v in range(256):
        n, s, l = v // 128, (v % 128) // 32, v % 32
        qs[32 * n + l] |= q[v] << (2 * s)
    blk = np.concatenate([(sc | (mn << 4)).astype(np.uint8), qs.astype(np.uint8), _f16b(0.5), _f16b(0.25)])
    assert blk.size == 84
    expect = np.array([0.5 * sc[v // 16] * q[v] - 0.25 * mn[v // 16] for v in range(256)], dtype=np.float32)
    for mid in (F16, BF16, F32):
        got = np_oracle.bits_to_f32(lib.dequant(blk, 10, mid, F32, 256), F32)
        assert np.array_equal(got, expect), mid


def test_kat_q3_k():
    """A Q3_K super-block packed the way GGML writes it: value v = 128n + 32s + l has its 2 low bits at bits 2s of
    qs[32n + l] and its high bit (set for q >= 0) at bit 4n + s of hmask[l]; sub-block i = v // 16 has a 6-bit
    scale whose low nibble is nibble i // 8 of byte i % 8 and whose 2 high bits sit at bits 2(i // 4) of byte
    8 + i % 4 of the 12 scale bytes, minus 32; d = 0.5. The expected values 0.5 * (scale - 32) * q are exact."""
    rng = np.random.default_rng(22)
    q = rng.integers(-4, 4, size=256)
    sc = rng.integers(0, 64, size=16)
    qs = np.zeros(64, dtype=np.int64)
    hm = np.zeros(32, dtype=np.int64)
    for v in range(256):
        n, s, l = v // 128, (v % 128) // 32, v % 32
        qs[32 * n + l] |= (q[v] & 3) << (2 * s)
        hm[l] |= int(q[v] >= 0) << (4 * n + s)
    scb = np.zeros(12, dtype=np.int64)
    for i in range(16):
        scb[i % 8] |= (sc[i] & 0xF) << (4 * (i // 8))
        scb[8 + i % 4] |= (sc[i] >> 4) << (2 * (i // 4))
    blk = np.concatenate([hm.astype(np.uint8), qs.astype(np.uint8), scb.astype(np.uint8), _f16b(0.5)])
    assert blk.size == 110
    expect = np.array([0.5 * (sc[v // 16] - 32) * q[v] for v in range(256)], dtype=np.float32)
    for mid in (F16, BF16, F32):
        got = np_oracle.bits_to_f32(lib.dequant(blk, 11, mid, F32, 256), F32)
        assert np.array_equal(got, expect), mid
