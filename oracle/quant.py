"""Per-token activation and per-channel weight FP8 quantisation (numpy).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Reference semantics restated:

* ``quant_per_token(..., variant="div")`` follows ``_quantize_per_token_impl``
  (``deploy/xvideo/models/dit/fp8_linear.py:38-43``)::

      s = clamp_min(absmax_row(x).float(), 1e-8) / 448
      q = e4m3fn(clamp(x.float() / s, -448, 448))          # RNE cast

* ``variant="rcp"`` follows the reference's gfx950 HIP kernel
  (``joyomni_ops/csrc/per_token_quant_fp8_rocm.hip:60-78``): the same scale,
  then ``q = e4m3fn(clamp(x * (1/s)))``.
* ``quant_weight_per_channel`` follows ``_quantize_weight_per_channel``
  (``fp8_linear.py:77-85``): one scale per output channel n of W[N, K].

Pins (tests/test_oracle_quant.py): the division variant against torch's own
CPU ops evaluated on the same inputs (library routines: bf16->fp32, amax,
division, clamp, e4m3fn cast); both variants against the independent C
restatement ``oracle/quant_ref.c``; special cases zero row (s = 1e-8/448,
q = 0, ``test_parity_light.py:119``), a row holding one value (|q| = 448 at the
absmax element), and the known division-vs-reciprocal byte disagreements.
"""
from __future__ import annotations

import numpy as np

from .fp8 import FP8_MAX, bf16_to_f32, f32_to_e4m3fn, fp16_to_f32


def _to_f32(x_u16: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_to_f32(x_u16)
    if dtype == "fp16":
        return fp16_to_f32(x_u16)
    raise ValueError(dtype)


def row_scales(xf: np.ndarray) -> np.ndarray:
    """Per-row scale ``max(absmax, 1e-8) / 448`` in fp32 (correctly rounded)."""
    absmax = np.abs(xf).max(axis=1) if xf.shape[1] else np.zeros(xf.shape[0], np.float32)
    absmax = np.maximum(absmax.astype(np.float32), np.float32(1e-8))
    return (absmax / np.float32(FP8_MAX)).astype(np.float32)


def _clamp_keep_nan(v: np.ndarray) -> np.ndarray:
    # torch.clamp keeps NaN; np.clip does too.
    return np.clip(v, np.float32(-FP8_MAX), np.float32(FP8_MAX))


def quant_per_token(x_u16: np.ndarray, dtype: str = "bf16", variant: str = "div"):
    """x: uint16 bit patterns [M, K] -> (q uint8 [M, K], s float32 [M])."""
    xf = _to_f32(np.asarray(x_u16), dtype)
    s = row_scales(xf)
    if variant == "div":
        v = (xf / s[:, None]).astype(np.float32)
    elif variant == "rcp":
        inv = (np.float32(1.0) / s).astype(np.float32)
        v = (xf * inv[:, None]).astype(np.float32)
    else:
        raise ValueError(variant)
    return f32_to_e4m3fn(_clamp_keep_nan(v)), s


def quant_weight_per_channel(w_u16: np.ndarray):
    """W bf16 bits [N, K] -> (Wq uint8 [N, K] (== (K,N) col-major), s_w float32 [N]).

    Same arithmetic as ``quant_per_token(variant="div")`` applied per output
    channel (``fp8_linear.py:80-82``).
    """
    return quant_per_token(w_u16, "bf16", "div")
