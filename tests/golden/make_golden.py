"""Writes the golden fixtures of tests/golden/ from the oracle (run from the repository root:
``python tests/golden/make_golden.py``). The reference holds no golden vectors of its own for this path, so these
are the oracle's answers, committed so that any later change to the oracle or to the kernels that moves a bit is
seen against a fixed record; the oracle itself is pinned by the known-answer and cross-formulation tests.

Contents (numpy .npz, no pickles):
* dequant.npz: per GGML type t, ``raw_t`` (6 blocks, typical and edge float16 scales) and, per MID/OUT pair
  (m, o), ``out_t_m_o`` -- the output bits (uint16 for f16/bf16, float32 for f32);
* quant_rows.npz: ``x`` (5 rows of 512 bf16 bits, incl. a zero row and ties), ``q_<mode>`` int8 and ``s_<mode>``
  float32 for mode 0 (plain per token) and 1 (ConvRot-256);
* linear_i8.npz: ``xq`` [4, 64], ``wq`` [6, 64] int8, ``xs`` [4], ``ws`` [6] float32, ``y`` the bf16 bits and
  ``acc`` the int32 accumulators;
* convrot_order.npz: ``x`` (6 rows of 256 bf16 bits spanning 24 binades, drawn so that summing a radix-4 stage in
  any other order than left to right changes at least one int8 value of every row), ``q`` int8 and ``s`` float32
  of the ConvRot quantisation."""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import lib, np_oracle  # noqa: E402

TYPES = [2, 3, 6, 7, 8, 10, 11, 12, 13, 14]
TYPE_SIZE = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34, 10: 84, 11: 110, 12: 144, 13: 176, 14: 210}
PER_BLOCK = {2: 32, 3: 32, 6: 32, 7: 32, 8: 32, 10: 256, 11: 256, 12: 256, 13: 256, 14: 256}
F16_FIELDS = {2: (0,), 3: (0, 2), 6: (0,), 7: (0, 2), 8: (0,), 10: (80, 82), 11: (108,), 12: (0, 2), 13: (0, 2),
              14: (208,)}
# float16 scales: typical magnitudes, +-0, subnormal, 1, the largest finite
SCALES = np.array([0x1A3D, 0x9E12, 0x0000, 0x8000, 0x0005, 0x3C00, 0x7BFF, 0x2E66, 0xA401, 0x03FF, 0x1001, 0x8C00],
                  dtype=np.uint16)


def blocks(qtype, seed):
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, size=(6, TYPE_SIZE[qtype]), dtype=np.uint16).astype(np.uint8)
    k = 0
    for i in range(6):
        for off in F16_FIELDS[qtype]:
            b[i, off:off + 2] = SCALES[k % SCALES.size:k % SCALES.size + 1].view(np.uint8)
            k += 1
    return b.ravel()


def main():
    lib.build()
    d = {}
    for t in TYPES:
        raw = blocks(t, 100 + t)
        d[f"raw_{t}"] = raw
        n = 6 * PER_BLOCK[t]
        for m in range(3):
            for o in range(3):
                d[f"out_{t}_{m}_{o}"] = lib.dequant(raw, t, m, o, n)
    np.savez_compressed(os.path.join(HERE, "dequant.npz"), **d)

    rng = np.random.default_rng(7)
    x = (rng.standard_normal((5, 512)).astype(np.float32) * np.float32(3.0)).view(np.uint32)
    x = ((x + 0x7FFF + ((x >> 16) & 1)) >> 16).astype(np.uint16)        # float32 -> bf16 bits (RNE)
    x[1] = 0                                                             # a zero row: scale floor 1e-30
    x[2, :4] = [0x3F80, 0x3FC0, 0x4020, 0xC0A0]                          # 1.0, 1.5, 2.5, -5.0
    q = {"x": x}
    for mode in (0, 1):
        qq, ss = lib.quant_rows(x, mode)
        q[f"q_{mode}"], q[f"s_{mode}"] = qq, ss
    np.savez_compressed(os.path.join(HERE, "quant_rows.npz"), **q)

    xq = rng.integers(-128, 128, size=(4, 64)).astype(np.int8)
    wq = rng.integers(-127, 128, size=(6, 64)).astype(np.int8)
    xs = (rng.random(4) * 0.05).astype(np.float32)
    ws = (rng.random(6) * 0.01).astype(np.float32)
    y, acc = lib.linear_i8(xq, wq, xs, ws, out_dt=lib.BF16, want_acc=True)
    np.savez_compressed(os.path.join(HERE, "linear_i8.npz"), xq=xq, wq=wq, xs=xs, ws=ws, y=y, acc=acc)
    np.savez_compressed(os.path.join(HERE, "convrot_order.npz"), **convrot_order_rows())


def convrot_order_rows(n=6, seed=11, candidates=20000):
    """Rows whose ConvRot int8 result depends on the stage sum order: bf16 values of random sign and magnitude
    2^U(-12, 12), kept when both other orders of np_oracle give a different int8 row than the left-to-right one."""
    rng = np.random.default_rng(seed)
    f = rng.choice([-1.0, 1.0], (candidates, 256)) * 2.0 ** rng.uniform(-12, 12, (candidates, 256))
    u = f.astype(np.float32).view(np.uint32)
    x = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    ltr, _ = np_oracle.quant_rows_convrot(x, "ltr")
    keep = np.ones(candidates, dtype=bool)
    for order in ("pair", "rtl"):
        other, _ = np_oracle.quant_rows_convrot(x, order)
        keep &= (other != ltr).any(axis=1)
    rows = x[np.nonzero(keep)[0][:n]]
    q, s = lib.quant_rows(rows, 1)
    return {"x": rows, "q": q, "s": s}


if __name__ == "__main__":
    main()
