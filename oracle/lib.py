"""ORACLE (test infrastructure only): ctypes binding of the scalar C restatement ``oracle/wf_oracle.c``.

The shared library is built by ``oracle/Makefile`` into ``oracle/_build/libwf_oracle.so`` (``build()`` of the
entry module does it; ``load()`` builds it on first use when it is missing -- gcc only, no GPU).
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "libwf_oracle.so")
_lib = None

F16, BF16, F32 = 0, 1, 2
NP_OUT = {F16: np.uint16, BF16: np.uint16, F32: np.float32}


def build(force=False):
    if force or not os.path.exists(_SO):
        subprocess.run(["make", "-s", "-C", _HERE] + (["-B"] if force else []), check=True)
    return _SO


def load():
    global _lib
    if _lib is None:
        build()
        lib = ctypes.CDLL(_SO)
        p, i64, c_int = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        lib.wfo_f32_to_f16_bits.argtypes = [ctypes.c_float]
        lib.wfo_f32_to_f16_bits.restype = ctypes.c_uint16
        lib.wfo_f16_bits_to_f32.argtypes = [ctypes.c_uint16]
        lib.wfo_f16_bits_to_f32.restype = ctypes.c_float
        lib.wfo_round.argtypes = [ctypes.c_float, c_int]
        lib.wfo_round.restype = ctypes.c_float
        lib.wfo_kquant_bytes.argtypes = [c_int]
        lib.wfo_kquant_bytes.restype = c_int
        lib.wfo_scale_min.argtypes = [p, c_int, p, p]
        lib.wfo_scale_min.restype = None
        lib.wfo_dequant.argtypes = [p, i64, c_int, c_int, c_int, p, i64]
        lib.wfo_dequant.restype = c_int
        lib.wfo_dequant_add.argtypes = [p, i64, c_int, c_int, c_int, p, ctypes.c_float, p, i64]
        lib.wfo_dequant_add.restype = c_int
        lib.wfo_quant_rows.argtypes = [p, i64, i64, c_int, p, p, p]
        lib.wfo_ln_stats.argtypes = [p, i64, p, p]
        lib.wfo_quant_rows_pre.argtypes = [p, i64, i64, c_int, p, p, i64, ctypes.c_float, p, p, p, p]
        lib.wfo_quant_rows_pre.restype = c_int
        lib.wfo_quant_rows.restype = c_int
        lib.wfo_linear_i8.argtypes = [p, p, p, p, p, p, c_int, i64, i64, i64, p]
        lib.wfo_linear_i8.restype = c_int
        lib.wfo_linear_i8_residual.argtypes = [p, p, p, p, p, p, p, i64, i64, i64, i64]
        lib.wfo_linear_i8_residual.restype = c_int
        _lib = lib
    return _lib


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def f32_to_f16_bits(x):
    """Vector form of the C textbook f32 -> f16 RNE conversion (one ctypes call per element: small inputs)."""
    lib = load()
    x = np.asarray(x, dtype=np.float32).ravel()
    return np.array([lib.wfo_f32_to_f16_bits(float(v)) for v in x], dtype=np.uint16)


def dequant(raw, qtype, mid, out, n):
    """wfo_dequant: raw uint8 blocks -> n values of dtype ``out`` (uint16 bits for f16/bf16, float32 for f32)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    dst = np.empty(n, dtype=NP_OUT[out])
    rc = load().wfo_dequant(_ptr(raw), raw.size, qtype, mid, out, _ptr(dst), n)
    if rc != 0:
        raise ValueError(f"oracle dequant rejected the input (rc={rc})")
    return dst


def dequant_add(raw, qtype, mid, out, diff, sa, base=None):
    """wfo_dequant_add: the LoRA add of one difference ``diff`` (float32, n values) scaled by ``sa``, onto the
    dequantisation of ``raw`` when it is given (the first LoRA), else onto ``base`` (values of dtype ``out``: uint16
    bits for f16/bf16, float32 for f32)."""
    diff = np.ascontiguousarray(diff, dtype=np.float32).ravel()
    n = diff.size
    if raw is None:
        dst = np.array(base, dtype=NP_OUT[out]).ravel().copy()
        assert dst.size == n
        rc = load().wfo_dequant_add(None, 0, 0, 0, out, _ptr(diff), float(sa), _ptr(dst), n)
    else:
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        dst = np.empty(n, dtype=NP_OUT[out])
        rc = load().wfo_dequant_add(_ptr(raw), raw.size, qtype, mid, out, _ptr(diff), float(sa), _ptr(dst), n)
    if rc != 0:
        raise ValueError(f"oracle dequant_add rejected the input (rc={rc})")
    return dst


def quant_rows(x_bf16_bits, mode):
    """wfo_quant_rows: bf16 bits [M, K] -> (int8 [M, K], float32 scales [M])."""
    x = np.ascontiguousarray(x_bf16_bits, dtype=np.uint16)
    M, K = x.shape
    xq = np.empty((M, K), dtype=np.int8)
    xs = np.empty(M, dtype=np.float32)
    work = np.empty(K, dtype=np.float32)
    rc = load().wfo_quant_rows(_ptr(x), M, K, mode, _ptr(xq), _ptr(xs), _ptr(work))
    if rc != 0:
        raise ValueError(f"oracle quant_rows rejected the input (rc={rc})")
    return xq, xs


def ln_stats(row_bf16_bits):
    """(mean, sigma2 / K) of one bf16 row by the reference's Welford order (wfo_ln_stats)."""
    r = np.ascontiguousarray(row_bf16_bits, dtype=np.uint16)
    mu, var = np.zeros(1, np.float32), np.zeros(1, np.float32)
    load().wfo_ln_stats(_ptr(r), r.size, _ptr(mu), _ptr(var))
    return mu[0], var[0]


def quant_rows_pre(x_bf16_bits, pre, s=None, h=None, rows_per_group=1, eps=0.0):
    """ConvRot row quantisation with the operation ``pre`` first (wfo_quant_rows_pre): GELU with ``s`` the bf16 bits
    of the 65536-entry table; MOD / LNMOD with ``s`` = bf16 bits of 1 + scale and ``h`` of the shift, [groups, K]."""
    x = np.ascontiguousarray(x_bf16_bits, dtype=np.uint16)
    M, K = x.shape
    xq = np.empty((M, K), dtype=np.int8)
    xs = np.empty(M, dtype=np.float32)
    work = np.empty(K, dtype=np.float32)
    rowbuf = np.empty(K, dtype=np.uint16)
    s_ = np.ascontiguousarray(s, dtype=np.uint16) if s is not None else None
    h_ = np.ascontiguousarray(h, dtype=np.uint16) if h is not None else None
    rc = load().wfo_quant_rows_pre(_ptr(x), M, K, pre, _ptr(s_), _ptr(h_), rows_per_group, float(eps), _ptr(xq),
                                   _ptr(xs), _ptr(work), _ptr(rowbuf))
    if rc != 0:
        raise ValueError(f"oracle quant_rows_pre rejected the input (rc={rc})")
    return xq, xs


def linear_i8(xq, wq, xs, ws, out_dt=BF16, bias=None, want_acc=False):
    """wfo_linear_i8: exact int32 GEMM + epilogue. Returns out (bits / float32) and optionally the int32 acc."""
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    wq = np.ascontiguousarray(wq, dtype=np.int8)
    xs = np.ascontiguousarray(xs, dtype=np.float32).ravel()
    ws = np.ascontiguousarray(ws, dtype=np.float32).ravel()
    M, K = xq.shape
    N = wq.shape[0]
    out = np.empty((M, N), dtype=NP_OUT[out_dt])
    acc = np.empty((M, N), dtype=np.int32) if want_acc else None
    if bias is not None:
        bias = np.ascontiguousarray(bias)
    rc = load().wfo_linear_i8(_ptr(xq), _ptr(wq), _ptr(xs), _ptr(ws), _ptr(bias), _ptr(out), out_dt, M, N, K,
                              _ptr(acc))
    if rc != 0:
        raise ValueError(f"oracle linear_i8 failed (rc={rc})")
    return (out, acc) if want_acc else out


def linear_i8_residual(xq, wq, xs, ws, gate_bits, resid_bits, rows_per_group):
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    wq = np.ascontiguousarray(wq, dtype=np.int8)
    xs = np.ascontiguousarray(xs, dtype=np.float32).ravel()
    ws = np.ascontiguousarray(ws, dtype=np.float32).ravel()
    gate = np.ascontiguousarray(gate_bits, dtype=np.uint16)
    resid = np.ascontiguousarray(resid_bits, dtype=np.uint16)
    M, K = xq.shape
    N = wq.shape[0]
    out = np.empty((M, N), dtype=np.uint16)
    load().wfo_linear_i8_residual(_ptr(xq), _ptr(wq), _ptr(xs), _ptr(ws), _ptr(gate), _ptr(resid), _ptr(out),
                                  M, N, K, rows_per_group)
    return out
