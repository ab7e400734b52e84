"""Scalar restatement of the quantizers, one element at a time with numpy fp32 scalars, Python's round-half-even
``round`` and hand-written bf16 rounding: an implementation independent of the torch oracle (no reshapes, no
broadcasting, no torch rounding), used to pin oracle/ref.py and to generate the golden vectors.

Formulas (reference: patches/kv_tiers.py:332-387, patches/kv_int4.py:324-341, gemv/test_kv_tiers.py:65-87):
  a = max_i |x_i| over the group;  s = fp16(min(a > 0 ? a / qmax : 1, 65504));  q_i = clamp(rne(x_i / s), +-qmax)
  dequant = bf16(q * s) (computed in fp32);  INT4 byte = (q_even + 8) | (q_odd + 8) << 4.
"""
from __future__ import annotations

import struct
from typing import List, Tuple

import numpy as np

F32 = np.float32


def f32(x) -> np.float32:
    return F32(x)


def fp16_round(x: np.float32) -> np.float32:
    return F32(np.float16(x))


def bf16_round_bits(x: np.float32) -> int:
    """fp32 -> bf16 bits, round to nearest even (non-NaN inputs)."""
    b = struct.unpack("<I", struct.pack("<f", float(x)))[0]
    lsb = (b >> 16) & 1
    b = (b + 0x7FFF + lsb) & 0xFFFFFFFF
    return b >> 16


def bf16_value(bits: int) -> float:
    return struct.unpack("<f", struct.pack("<I", (bits & 0xFFFF) << 16))[0]


def quant_group(xs: List[np.float32], qmax: float) -> Tuple[List[int], np.float32]:
    a = F32(0.0)
    for x in xs:
        if abs(x) > a:
            a = F32(abs(x))
    s = (F32(a) / F32(qmax)) if a > 0 else F32(1.0)
    if s > F32(65504.0):
        s = F32(65504.0)
    s = fp16_round(s)
    qs = []
    for x in xs:
        qf = float(F32(x) / s)  # the fp32 quotient
        r = round(max(-qmax, min(qmax, qf)))  # clamp then round-half-even (same result as round then clamp)
        qs.append(int(r))
    return qs, s


def quant_row(xs: List[float], group: int, qmax: float, sm_inv: List[float] = None):
    """One row -> (codes list, scales list as float)."""
    vals = [F32(v) for v in xs]
    if sm_inv is not None:
        vals = [F32(v * F32(m)) for v, m in zip(vals, sm_inv)]
    codes, scales = [], []
    for g in range(len(vals) // group):
        q, s = quant_group(vals[g * group:(g + 1) * group], qmax)
        codes += q
        scales.append(float(s))
    return codes, scales


def pack_row(codes: List[int]) -> List[int]:
    return [((codes[2 * j] + 8) | ((codes[2 * j + 1] + 8) << 4)) & 0xFF for j in range(len(codes) // 2)]


def dequant_row_bits(codes: List[int], scales: List[float], group: int, sm: List[float] = None) -> List[int]:
    """bf16 bits of f32(c) * f32(s) (* f32(sm) per channel when given), products in fp32 left to right."""
    out = []
    for i, c in enumerate(codes):
        x = F32(F32(c) * F32(scales[i // group]))
        if sm is not None:
            x = F32(x * F32(sm[i]))
        out.append(bf16_round_bits(x))
    return out


def unpack_row(packed: List[int]) -> List[int]:
    """INT4 bytes -> codes: low nibble the even channel, high nibble the odd one, each minus 8."""
    codes = []
    for b in packed:
        codes += [(b & 15) - 8, (b >> 4) - 8]
    return codes


def requant_row(codes8: List[int], scales8: List[float], group8: int):
    """Evicted ring row -> INT4-G32: x = f32(q8) * f32(s8) (exact), then the INT4 quantizer."""
    xs = [F32(F32(c) * F32(scales8[i // group8])) for i, c in enumerate(codes8)]
    return quant_row([float(x) for x in xs], 32, 7.0)
