"""Bit-level number-format conversions used by the oracle (numpy only).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Pins (tests/test_oracle_fp8.py):
* ``f32_to_e4m3fn`` is checked against torch's own ``Tensor.to(torch.float8_e4m3fn)``
  (a library routine, RNE, no saturation: values >= 464 become NaN) on every
  bf16 bit pattern, on every fp8 value, on every midpoint between adjacent fp8
  values (ties-to-even) and on random fp32 values.
* ``e4m3fn_to_f32`` is checked against torch's fp8 -> fp32 cast for all 256 codes.
* ``f32_to_bf16`` is checked against torch's fp32 -> bf16 cast (RNE).
"""
from __future__ import annotations

import numpy as np

FP8_MAX = 448.0  # torch.finfo(torch.float8_e4m3fn).max (fp8_linear.py:19-20)


def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32 (exact)."""
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def fp16_to_f32(u16: np.ndarray) -> np.ndarray:
    """fp16 bit patterns (uint16) -> float32 (exact)."""
    return np.asarray(u16, dtype=np.uint16).view(np.float16).astype(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round-to-nearest-even; NaN -> quiet NaN."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = x.view(np.uint32)
    lsb = (b >> 16) & 1
    r = ((b + np.uint32(0x7FFF) + lsb) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r = r.copy()
        r[nan] = ((b[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 value, returned as float32."""
    return bf16_to_f32(f32_to_bf16(x))


def e4m3fn_to_f32(q: np.ndarray) -> np.ndarray:
    """OCP e4m3fn codes (uint8) -> float32 (exact). 0x7F/0xFF are NaN."""
    q = np.asarray(q, dtype=np.uint8).astype(np.int32)
    sign = np.where(q & 0x80, -1.0, 1.0)
    e = (q >> 3) & 0xF
    m = q & 0x7
    normal = np.ldexp(1.0 + m / 8.0, e - 7)
    sub = np.ldexp(m / 8.0, -6)
    v = np.where(e == 0, sub, normal) * sign
    v = np.where((q & 0x7F) == 0x7F, np.nan, v)
    return v.astype(np.float32)


def f32_to_e4m3fn(x: np.ndarray) -> np.ndarray:
    """float32 -> OCP e4m3fn codes, round-to-nearest-even, no saturation.

    Same contract as torch's CPU cast: |x| >= 464 (the tie above 448 rounds
    away from the even code) and NaN/inf give NaN (0x7F, sign kept for
    finite overflow the way torch does: torch returns 0x7F/0xFF by sign).
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = x.view(np.uint32)
    sign = ((bits >> 24) & 0x80).astype(np.uint8)
    a = np.abs(x).astype(np.float32)
    out = np.zeros(x.shape, dtype=np.uint8)

    # subnormal range of e4m3fn: |x| < 2^-6, step 2^-9. x * 2^9 is exact.
    sub = a < np.float32(2.0 ** -6)
    k = np.rint(a[sub].astype(np.float64) * 512.0).astype(np.int64)  # rint = half-even
    out[sub] = k.astype(np.uint8)  # k == 8 is the code of 2^-6 (e=1, m=0)

    # normal range: round the fp32 mantissa to 3 bits, half-even.
    nrm = ~sub
    ab = a[nrm].view(np.uint32).astype(np.int64)
    lsb = (ab >> 20) & 1
    rounded = (ab + 0x7FFFF + lsb) >> 20  # exponent(8) | mantissa(3)
    e32 = rounded >> 3
    m3 = rounded & 7
    e8 = e32 - 127 + 7
    code = (e8 << 3) | m3
    overflow = (e8 > 15) | ((e8 == 15) & (m3 == 7))
    code = np.where(overflow, 0x7F, code)
    out[nrm] = code.astype(np.uint8)

    out = out | sign
    nan = ~np.isfinite(x)
    out[nan] = 0x7F | sign[nan]
    return out
