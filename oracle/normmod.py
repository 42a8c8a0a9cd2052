"""(Layer|RMS)Norm + adaLN scale/shift, and its FP8-emitting variant (numpy).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Restated from ``normScaleShiftPerRow`` (``joyomni_ops/csrc/fused_norm_scale_shift.cu:97-182``),
the kernel behind ``fused_layernorm_modulate`` (``deploy/xvideo/models/dit/sgl_fused_ops.py:46-91``),
per row of x [M, N]::

    mean = sum(x) / N                                   (LayerNorm)
    r    = rsqrt(sum((x - mean)^2) / N + eps)           (LayerNorm, two passes)
         = rsqrt(sum(x^2) / N + eps)                    (RMSNorm)
    y    = T(((x - mean) * r * g + b) * (1 + scale) + shift)     LayerNorm
         = T((x * r * g) * (1 + scale) + shift)                  RMSNorm

in fp32 with one final rounding to the activation type T; g = 1 and b = 0 when
absent, and b only with g (``:125,158-162``); scale/shift one row broadcast or
one row per token. The FP8 variant is ``quant.quant_per_token`` of y.

Pins (tests/test_oracle_normmod.py): torch's own CPU ``F.layer_norm`` (with and
without affine weights) and the RMS formula of ``sgl_fused_ops.py:202-209`` in
fp32, times ``(1 + scale) + shift``, bit-equal on all but a handful of
rounding ties while a variant with the unbiased variance or without the
``1 +`` fails; a constant row (x - mean = 0 exactly, so y = b * (1 + scale) +
shift); the FP8 variant equals the quantiser oracle on y.
"""
from __future__ import annotations

import numpy as np

from . import quant
from .fp8 import bf16_to_f32, f32_to_bf16, fp16_to_f32


def to_f32(bits: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_to_f32(bits)
    if dtype == "fp16":
        return fp16_to_f32(bits)
    return np.asarray(bits, np.float32)


def from_f32(v: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return f32_to_bf16(v)
    if dtype == "fp16":
        return np.asarray(v, np.float32).astype(np.float16).view(np.uint16)
    return np.asarray(v, np.float32)


def norm_scale_shift_f32(x, gamma, beta, scale, shift, norm_type: int, eps: float) -> np.ndarray:
    """fp32 values in, fp32 y (before the final rounding) out. scale/shift: [1 or M, N]."""
    x = np.asarray(x, np.float32)
    M, N = x.shape
    one = np.float32(1.0)
    g = np.ones(N, np.float32) if gamma is None else np.asarray(gamma, np.float32)
    b = np.zeros(N, np.float32) if (beta is None or gamma is None or norm_type == 1) else np.asarray(beta, np.float32)
    sc = np.asarray(scale, np.float32)
    sh = np.asarray(shift, np.float32)
    if norm_type == 0:
        mean = (np.sum(x.astype(np.float64), axis=1, keepdims=True) / N).astype(np.float32)
        d = (x - mean).astype(np.float32)
        var = (np.sum(d.astype(np.float64) ** 2, axis=1, keepdims=True) / N).astype(np.float32)
        r = (1.0 / np.sqrt(var.astype(np.float64) + np.float32(eps))).astype(np.float32)
        y = ((d * r) * g + b) * (one + sc) + sh
    else:
        ms = (np.sum(x.astype(np.float64) ** 2, axis=1, keepdims=True) / N).astype(np.float32)
        r = (1.0 / np.sqrt(ms.astype(np.float64) + np.float32(eps))).astype(np.float32)
        y = ((x * r) * g) * (one + sc) + sh
    return y.astype(np.float32)


def term_magnitude(x, gamma, beta, scale, shift, norm_type: int, eps: float) -> np.ndarray:
    """Magnitude of the terms of every output before rounding (fp32 values in): the scale of
    the fp32 rounding error of y, used to bound results that cancel to near zero. The norm term
    counts |x| + |mean| (the error of x - mean follows its operands), then |beta| and |shift|."""
    x = np.asarray(x, np.float64)
    N = x.shape[1]
    g = np.ones(N) if gamma is None else np.asarray(gamma, np.float64)
    b = np.zeros(N) if (beta is None or gamma is None or norm_type == 1) else np.asarray(beta, np.float64)
    sc = 1.0 + np.asarray(scale, np.float64)
    mean = x.mean(1, keepdims=True) if norm_type == 0 else np.zeros((x.shape[0], 1))
    r = 1.0 / np.sqrt(((x - mean) ** 2).mean(1, keepdims=True) + eps)
    return ((np.abs(x) + np.abs(mean)) * r * np.abs(g * sc) + np.abs(b * sc)
            + np.abs(np.asarray(shift, np.float64)))


def norm_scale_shift(x_bits, gamma_bits, beta_bits, scale_bits, shift_bits, norm_type: int, eps: float,
                     dtype: str = "bf16") -> np.ndarray:
    """Oracle of ``fused_norm_scale_shift``: bit patterns (or fp32 arrays) in, same dtype out."""
    cv = lambda t: None if t is None else to_f32(t, dtype)  # noqa: E731
    y = norm_scale_shift_f32(cv(x_bits), cv(gamma_bits), cv(beta_bits), cv(scale_bits), cv(shift_bits),
                             norm_type, eps)
    return from_f32(y, dtype)


def norm_scale_shift_fp8(x_bits, gamma_bits, beta_bits, scale_bits, shift_bits, norm_type: int, eps: float,
                         dtype: str = "bf16", variant: str = "div"):
    """Oracle of ``fused_norm_scale_shift_fp8``: (q e4m3fn codes, s fp32, y bits)."""
    y = norm_scale_shift(x_bits, gamma_bits, beta_bits, scale_bits, shift_bits, norm_type, eps, dtype)
    q, s = quant.quant_per_token(y, dtype, variant)
    return q, s, y
