"""FP8 x FP8 -> bf16/fp16 row/column-scaled GEMM (numpy).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Contract restated from ``joyomni_ops/csrc/fp8_gemm.cu:1450-1487`` (argument
rules) and its epilogue tree ``fp8_gemm.cu:99-136``::

    acc[m, n] = sum_k A[m, k] * B[k, n]          (fp8 values, exact products)
    t         = fp32(acc * scales_b[n])
    out[m, n] = round_out(fp32(t * scales_a[m] + bias[n]))

``B`` is given as ``Wq[N, K]`` row-major, i.e. the (K, N) column-major matrix
the reference passes (``fp8_linear.py:83-84``).

``reference_fp32`` is the benchmark's tolerance reference: fp32
dequantise-then-matmul ``(qa * sa) @ (qb * sb)^T + bias``.

Pins (tests/test_oracle_gemm.py): brute-force triple loop on tiny inputs; a
small-integer construction in which every partial sum is exact in fp32, so
the result is fixed exactly (independent of summation order) and the
epilogue's single final rounding is checked bit for bit; linearity in
``scales_a``/``scales_b``; bias-only output when A = 0; agreement with
torch's CPU ``torch._scaled_mm`` (tensor-wise scales, the only variant the
CPU backend supports) on the unscaled product.
"""
from __future__ import annotations

import numpy as np

from .fp8 import bf16_to_f32, e4m3fn_to_f32, f32_to_bf16, fp16_to_f32


def dequant(q_u8: np.ndarray) -> np.ndarray:
    return e4m3fn_to_f32(q_u8)


def exact_acc(qa_u8: np.ndarray, qb_nk_u8: np.ndarray) -> np.ndarray:
    """Unscaled accumulator in float64 (exact for K up to ~2^20 of fp8 products:
    every fp8 x fp8 product has <= 8 significant bits and |p| <= 448^2)."""
    a = dequant(qa_u8).astype(np.float64)
    b = dequant(qb_nk_u8).astype(np.float64)
    return a @ b.T


def abs_acc(qa_u8: np.ndarray, qb_nk_u8: np.ndarray) -> np.ndarray:
    """sum_k |A[m,k] * B[k,n]| (float64): the scale of fp32 accumulation error."""
    a = np.abs(dequant(qa_u8).astype(np.float64))
    b = np.abs(dequant(qb_nk_u8).astype(np.float64))
    return a @ b.T


def epilogue(acc: np.ndarray, sa: np.ndarray, sb: np.ndarray, bias_f32=None) -> np.ndarray:
    """fp8_gemm.cu:99-136: t = fp32(acc*sb[n]); o = fp32(t*sa[m] + bias[n]) (one fma)."""
    t = (acc.astype(np.float32) * sb.astype(np.float32)[None, :]).astype(np.float32)
    o = t.astype(np.float64) * sa.astype(np.float32)[:, None].astype(np.float64)
    if bias_f32 is not None:
        o = o + bias_f32.astype(np.float64)[None, :]
    return o.astype(np.float32)  # fma: exact product + add, rounded once


def scaled_mm(qa_u8, qb_nk_u8, sa, sb, bias_u16=None, out_dtype: str = "bf16"):
    """Full reference: returns (out bit patterns uint16 [M, N], fp32 pre-rounding)."""
    acc = exact_acc(qa_u8, qb_nk_u8)
    bias = None
    if bias_u16 is not None:
        bias = bf16_to_f32(bias_u16) if out_dtype == "bf16" else fp16_to_f32(bias_u16)
    o = epilogue(acc, sa, sb, bias)
    if out_dtype == "bf16":
        return f32_to_bf16(o), o
    return o.astype(np.float16).view(np.uint16), o


def reference_fp32(qa_u8, qb_nk_u8, sa, sb, bias_u16=None) -> np.ndarray:
    """The benchmark's tolerance reference: fp32 dequantise-then-matmul + bias."""
    a = dequant(qa_u8) * sa.astype(np.float32)[:, None]
    b = dequant(qb_nk_u8) * sb.astype(np.float32)[:, None]
    o = (a.astype(np.float64) @ b.astype(np.float64).T).astype(np.float32)
    if bias_u16 is not None:
        o = o + bf16_to_f32(bias_u16)[None, :]
    return o


def gelu_tanh(x: np.ndarray) -> np.ndarray:
    """GELU, tanh approximation (``dit.py:87-89``; torch ``approximate='tanh'``)."""
    x64 = x.astype(np.float64)
    c = np.sqrt(2.0 / np.pi)
    return (0.5 * x64 * (1.0 + np.tanh(c * (x64 + 0.044715 * x64 ** 3)))).astype(np.float32)
