"""3-D (t, h, w) RoPE tables (numpy).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Restated from ``get_1d_rotary_pos_embed`` (``deploy/xvideo/models/dit/rope.py:31-52``),
the per-axis concatenation of ``get_rotary_pos_embed_from_ids``
(``deploy/xvideo/models/dit/dit.py:896-934``; tokens t-major, then h, then w,
``dit.py:911-915``) and the half-width bf16 packing of ``prepare_fused_rope``
(``deploy/xvideo/models/dit/sgl_fused_ops.py:94-119``)::

    freqs_a[j] = 1 / theta^(2j / dim_a)               j < dim_a/2   (fp32)
    angle      = pos_a * freqs_a                       (fp32)
    full table = [t-dims | h-dims | w-dims], each pair-interleaved (repeat_interleave(2))
    half table = full[..., ::2] -> bf16

Pins (tests/test_oracle_rope.py): closed form with float64 math (the fp32
angles differ from exact angles by < 1 ulp, so the bf16 tables agree except
where a value lies within 1 fp32 ulp of a bf16 rounding boundary); axis
structure (t-dims depend only on t, etc.); cos^2 + sin^2 = 1; position 0 gives
cos = 1, sin = 0.
"""
from __future__ import annotations

import numpy as np

from .fp8 import f32_to_bf16


def axis_freqs(dim: int, theta: float) -> np.ndarray:
    j = np.arange(0, dim, 2, dtype=np.float32)[: dim // 2]
    return (np.float32(1.0) / (np.float32(theta) ** (j / np.float32(dim)))).astype(np.float32)


def grid_positions(frame_ids, height: int, width: int):
    """Token order of ``dit.py:906-915``: t-major, then h, then w (row-major)."""
    frame_ids = np.asarray(frame_ids, dtype=np.float32)
    hh, ww = np.meshgrid(np.arange(height, dtype=np.float32), np.arange(width, dtype=np.float32), indexing="ij")
    t = np.repeat(frame_ids, height * width)
    h = np.tile(hh.reshape(-1), len(frame_ids))
    w = np.tile(ww.reshape(-1), len(frame_ids))
    return t, h, w


def rope_half_tables(frame_ids, height: int, width: int, dims=(44, 42, 42), theta: float = 10000.0):
    """Returns (cos, sin) as float32 [L, D/2] before bf16 rounding, and their bf16 bits."""
    pos = grid_positions(frame_ids, height, width)
    cos_parts, sin_parts = [], []
    for dim, p in zip(dims, pos):
        f = axis_freqs(dim, theta)
        ang = (p[:, None].astype(np.float32) * f[None, :]).astype(np.float32)
        cos_parts.append(np.cos(ang.astype(np.float64)).astype(np.float32))
        sin_parts.append(np.sin(ang.astype(np.float64)).astype(np.float32))
    cos = np.concatenate(cos_parts, axis=1)
    sin = np.concatenate(sin_parts, axis=1)
    return cos, sin, f32_to_bf16(cos), f32_to_bf16(sin)
