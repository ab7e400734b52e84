"""Generate tests/golden/quant_vectors.npz with the scalar model (scalar_model.py).

Rows (D = 256, bf16 inputs stored as uint16 bits) cover: N(0, 3); N(0, 1) with 8 outlier channels x8 (the
configurations' K); exact .5 ties at s = 1 for both quantizers (absmax 7 / 127 rows); a zero row; a zero group;
the -7..7 row; fp16-max clamp rows (1e6, bf16 max); small values whose scales are fp16 subnormals (groups
whose scale underflows to 0 are excluded: the torch reference gives inf/NaN codes there).  Stored per row: INT8-G64 codes/scales, INT8-G256
codes/scales, INT4-G32 packed bytes/scales, bf16 dequant bits of each, and the INT8-G64 -> INT4 requant.

    python tests/golden/gen_vectors.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import scalar_model as sm  # noqa: E402

D = 256
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "quant_vectors.npz")


def bf16_bits_of(x: float) -> int:
    return sm.bf16_round_bits(np.float32(x))


def rows():
    rs = np.random.RandomState(1234)
    out = []
    for _ in range(8):
        out.append(rs.randn(D) * 3)
    for _ in range(8):
        r = rs.randn(D)
        ch = rs.permutation(D)[:8]
        r[ch] *= 8
        out.append(r)
    tie7 = np.tile([7.0, 2.5, -2.5, 0.5, -0.5, 1.5, 3.5, -6.5], D // 8)          # s4 = 1: .5 ties at every step
    out.append(tie7)
    tie127 = np.tile([127.0, 4.5, -4.5, 0.5, 100.5, -126.5, 63.5, 1.5], D // 8)  # s8 = 1 in every group
    out.append(tie127)
    out.append(np.zeros(D))
    zg = rs.randn(D) * 3
    zg[64:96] = 0
    out.append(zg)
    out.append(np.array([-7, 7, -6, 6, -5, 5, -4, 4, -3, 3, -2, 2, -1, 1, 0, 7] * 16, dtype=np.float64))
    big = np.zeros(D)
    big[:32] = [1e6, -1e6, 5e5, -5e5, 4.6e5, -4.6e5, 1e5, -1e5] * 4
    big[64:96] = 3.3895313892515355e38                                            # bf16 max
    out.append(big)
    out.append(rs.randn(D) * 1e-4)                                                # fp16-subnormal scales
    out.append(rs.randn(D) * 300)
    return out


def main():
    xs = rows()
    bits = np.array([[bf16_bits_of(v) for v in r] for r in xs], dtype=np.uint16)
    vals = [[sm.bf16_value(int(b)) for b in r] for r in bits]
    res = {"x_bf16_bits": bits}
    q8, s8, d8, q8b, s8b, p4, s4, d4, rq, rs4 = ([] for _ in range(10))
    for r in vals:
        c, s = sm.quant_row(r, 64, 127.0)
        q8.append(c); s8.append(s); d8.append(sm.dequant_row_bits(c, s, 64))
        cb, sb = sm.quant_row(r, 256, 127.0)
        q8b.append(cb); s8b.append(sb)
        c4, sc4 = sm.quant_row(r, 32, 7.0)
        p4.append(sm.pack_row(c4)); s4.append(sc4); d4.append(sm.dequant_row_bits(c4, sc4, 32))
        cr, sr = sm.requant_row(c, s, 64)
        rq.append(sm.pack_row(cr)); rs4.append(sr)
    res.update(
        q8_g64=np.array(q8, dtype=np.int8), s8_g64=np.array(s8, dtype=np.float16), d8_g64_bits=np.array(d8, dtype=np.uint16),
        q8_g256=np.array(q8b, dtype=np.int8), s8_g256=np.array(s8b, dtype=np.float16),
        p4=np.array(p4, dtype=np.uint8), s4=np.array(s4, dtype=np.float16), d4_bits=np.array(d4, dtype=np.uint16),
        requant_p4=np.array(rq, dtype=np.uint8), requant_s4=np.array(rs4, dtype=np.float16),
    )
    np.savez_compressed(OUT, **res)
    print(f"wrote {OUT}: {len(xs)} rows")


if __name__ == "__main__":
    main()
