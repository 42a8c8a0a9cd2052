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

The role rotation of ``generate_source_id_rope`` (``dit.py:936-960``) and its
composition by angle addition (``dit.py:1146-1155``)::

    f_j      = 1 / theta_r^(2j / role_dim)             j < role_dim/2 (fp32), rest unrotated
    role     = source_id * f_j                          (fp32)
    new_cos  = cos3 * cos_r - sin3 * sin_r              (fp32, each op rounded once)
    new_sin  = sin3 * cos_r + cos3 * sin_r

Pins (tests/test_oracle_rope.py): closed form with float64 math (the fp32
angles differ from exact angles by < 1 ulp, so the bf16 tables agree except
where a value lies within 1 fp32 ulp of a bf16 rounding boundary); axis
structure (t-dims depend only on t, etc.); cos^2 + sin^2 = 1; position 0 gives
cos = 1, sin = 0. Composition: source id 0 leaves the 3-D tables bit-identical;
composed entries equal float64 cos/sin of the summed fp32 angles within 4e-7
(a swapped sign, a role rotation on the wrong dims or a wrong role theta miss
by > 1e-2); the dims past role_dim keep the 3-D values exactly.
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


def source_id_half(source_ids, head_dim: int, role_dim: int = 128, theta: float = 256.0):
    """Half-width float32 (cos, sin) [L, head_dim/2] of the role rotation (``dit.py:936-960``)."""
    role_dim = max(0, min(int(role_dim), int(head_dim)))
    sid = np.asarray(source_ids, dtype=np.float32)
    cos = np.ones((sid.shape[0], head_dim // 2), dtype=np.float32)
    sin = np.zeros_like(cos)
    f = axis_freqs(role_dim, theta) if role_dim else np.zeros(0, np.float32)
    ang = (sid[:, None] * f[None, :]).astype(np.float32)
    cos[:, : role_dim // 2] = np.cos(ang.astype(np.float64)).astype(np.float32)
    sin[:, : role_dim // 2] = np.sin(ang.astype(np.float64)).astype(np.float32)
    return cos, sin


def compose(cos_a, sin_a, cos_b, sin_b):
    """Angle addition in float32 with each product and sum rounded once (``dit.py:1153-1154``)."""
    f = np.float32
    c = (cos_a.astype(f) * cos_b.astype(f)).astype(f) - (sin_a.astype(f) * sin_b.astype(f)).astype(f)
    s = (sin_a.astype(f) * cos_b.astype(f)).astype(f) + (cos_a.astype(f) * sin_b.astype(f)).astype(f)
    return c.astype(f), s.astype(f)


def visual_half_tables(current_shape, ref_video_frames=None, temporal_ids=None, dims=(16, 56, 56),
                       theta: float = 256.0, role_dim: int = 128, role_theta: float = 256.0,
                       ref_image_cache: bool = False):
    """[current chunk | ref-video] tables as ``dit.py:1093-1155`` assembles them; returns the
    float32 half tables and their bf16 bits."""
    frames, h, w = current_shape
    ids_cur = np.arange(frames) if temporal_ids is None else np.asarray(temporal_ids)
    cos, sin, _, _ = rope_half_tables(ids_cur, h, w, dims, theta)
    n = cos.shape[0]
    role = [np.full(n, 2.0 if ref_image_cache else 0.0, np.float32)]
    if ref_video_frames is not None:
        ids_ref = np.arange(ref_video_frames) if temporal_ids is None else np.asarray(temporal_ids)
        c2, s2, _, _ = rope_half_tables(ids_ref, h, w, dims, theta)
        cos, sin = np.concatenate([cos, c2]), np.concatenate([sin, s2])
        role.append(np.full(c2.shape[0], 1.0, np.float32))
    cr, sr = source_id_half(np.concatenate(role), sum(dims), role_dim, role_theta)
    c, s = compose(cos, sin, cr, sr)
    return c, s, f32_to_bf16(c), f32_to_bf16(s)
