"""Per-head q/k RMSNorm + interleaved RoPE, fused QKV split and KV-ring write (numpy).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Restated from the reference's gfx950 kernel
``joyomni_ops/csrc/fused_qknorm_rope_3d_kernel.cu:68-105``, per (token, head)::

    r      = rsqrt(sum_d x_d^2 / D + eps)                (fp32)
    xh_d   = x_d * r * w_d                              (fp32, one rounding at the end)
    pair i = (2i, 2i+1), c, s = bf16 cos/sin[token, i]
    o_2i   = xh_2i * c - xh_2i+1 * s
    o_2i+1 = xh_2i * s + xh_2i+1 * c
    k_pre  = bf16(xh)      (normalised K before rotation, ``:97-100``)

The QKV split is ``rearrange(qkv, "B L (K H D) -> K B L H D", K=3)``
(``deploy/xvideo/models/dit/dit.py:409-411``); the cache write stores the
pre-RoPE K and a compact copy of V for the current chunk
(``dit.py:446-451,867-882``, ``_compact_kv_tensor`` ``dit.py:131-137``) -- here
into slot ``slot`` of a ``[n_slots, L_cap, H, D]`` ring.

Pins (tests/test_oracle_qknorm.py): the reference test's closed form
``ref_one`` (``joyomni_ops/tests/test_parity_light.py:93-103``) evaluated with
torch CPU ops; special cases c = 1, s = 0 (pure RMSNorm, equal to k_pre);
x = const per head with w = 1 (|o| = 1/sqrt(1 + eps/x^2) on every element);
a rotation-only check against complex multiplication (numpy complex128);
norm preservation of the rotation; V copied bit-exactly.
"""
from __future__ import annotations

import numpy as np

from .fp8 import bf16_to_f32, f32_to_bf16


def norm_rope_heads(x: np.ndarray, w: np.ndarray, cos: np.ndarray, sin: np.ndarray, eps: float):
    """x: fp32 [L, H, D] (bf16 values); w: fp32 [D]; cos/sin fp32 [L, D/2] (bf16 values).

    Returns (rotated fp32 [L,H,D], normalised fp32 [L,H,D]) before bf16 rounding.
    """
    x = x.astype(np.float32)
    D = x.shape[-1]
    ss = np.sum(x.astype(np.float64) ** 2, axis=-1, keepdims=True)
    r = (1.0 / np.sqrt(ss / D + eps)).astype(np.float32)
    xh = (x * r * w.astype(np.float32)[None, None, :]).astype(np.float32)
    c = cos.astype(np.float32)[:, None, :]
    s = sin.astype(np.float32)[:, None, :]
    x0 = xh[..., 0::2]
    x1 = xh[..., 1::2]
    o = np.empty_like(xh)
    o[..., 0::2] = x0 * c - x1 * s
    o[..., 1::2] = x0 * s + x1 * c
    return o, xh


def qk_norm_rope_paired(q_u16, k_u16, seq_len, num_heads, eps, qw_u16, kw_u16, cos_u16, sin_u16):
    """Oracle of ``fused_qk_norm_rope_3d_paired`` (in-place op, pybind.cpp:53-55).

    q, k: bf16 bits [B, seq_len*num_heads, D]. Returns bf16 bits (q_out, k_out, k_pre).
    """
    B, LH, D = q_u16.shape
    L, H = seq_len, num_heads
    assert LH == L * H
    cos = bf16_to_f32(cos_u16)
    sin = bf16_to_f32(sin_u16)
    outs = []
    for x_u16, w_u16 in ((q_u16, qw_u16), (k_u16, kw_u16)):
        xf = bf16_to_f32(x_u16).reshape(B * L, H, D)
        cs = np.tile(cos, (B, 1))
        sn = np.tile(sin, (B, 1))
        o, xh = norm_rope_heads(xf, bf16_to_f32(w_u16), cs, sn, eps)
        outs.append((f32_to_bf16(o).reshape(B, LH, D), f32_to_bf16(xh).reshape(B, LH, D)))
    return outs[0][0], outs[1][0], outs[1][1]


def qkv_norm_rope_cache(qkv_u16, num_heads, eps, qw_u16, kw_u16, cos_u16, sin_u16):
    """Oracle of the fused QKV split + q/k RMSNorm + RoPE + KV-ring write.

    qkv: bf16 bits [L, 3*H*D] (token row = [q | k | v]).
    Returns bf16 bits: q_rope [L,H,D], k_rope [L,H,D], k_pre [L,H,D], v [L,H,D].
    The ring write is ``cache_k[slot, :L] = k_pre`` and ``cache_v[slot, :L] = v``.
    """
    L, E3 = qkv_u16.shape
    H = num_heads
    D = E3 // (3 * H)
    t = qkv_u16.reshape(L, 3, H, D)
    q, k, v = t[:, 0], t[:, 1], t[:, 2]
    cos = bf16_to_f32(cos_u16)
    sin = bf16_to_f32(sin_u16)
    oq, _ = norm_rope_heads(bf16_to_f32(q), bf16_to_f32(qw_u16), cos, sin, eps)
    ok, kh = norm_rope_heads(bf16_to_f32(k), bf16_to_f32(kw_u16), cos, sin, eps)
    return f32_to_bf16(oq), f32_to_bf16(ok), f32_to_bf16(kh), np.ascontiguousarray(v)
