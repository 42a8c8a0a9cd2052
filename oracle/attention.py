"""Joint-attention core: softmax(q k^T * scale) v per head (numpy, float64).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Restated from the reference model's ``_sdpa_attention``
(``deploy/xvideo/models/dit/dit.py:154-167``)::

    out = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2),
                                         v.transpose(1, 2), is_causal=False).transpose(1, 2)

on bf16 ``[1, S, H, D]`` tensors: no mask, no dropout, default scale ``1/sqrt(D)``
(the definition of ``F.scaled_dot_product_attention``), i.e. per head h and query i::

    s_ij  = scale * sum_d q[i, h, d] k[j, h, d]
    p_ij  = exp(s_ij - max_j s_ij) / sum_j exp(s_ij - max_j s_ij)
    o_ihd = sum_j p_ij v[j, h, d]

computed here in float64 from the exact bf16 input values (the result the
bf16 kernels approximate). Inputs are bf16 bit patterns (uint16) ``[L, H, D]``.

Pins (tests/test_oracle_attention.py): torch's own CPU
``F.scaled_dot_product_attention`` in float64 on the same values (a library
routine, agreement to 1e-12); closed forms -- a single key gives out = v[0];
identical keys give the mean of the values; a key whose score exceeds the others
by 60 (in scale units) gives its value row; constant value rows give that
constant; the output is invariant to a permutation of the keys (with their
values) and is a convex combination of the value rows (per head and d, between
their min and max). A dropped scale, a transposed operand or a softmax over the
wrong axis fails these.
"""
from __future__ import annotations

import math

import numpy as np

from .fp8 import bf16_to_f32


def sdpa(q_u16: np.ndarray, k_u16: np.ndarray, v_u16: np.ndarray, scale: float | None = None) -> np.ndarray:
    """float64 [Lq, H, D] attention output from bf16 [L, H, D] patterns."""
    q = bf16_to_f32(q_u16).astype(np.float64)
    k = bf16_to_f32(k_u16).astype(np.float64)
    v = bf16_to_f32(v_u16).astype(np.float64)
    return sdpa_f64(q, k, v, scale)


def sdpa_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float | None = None) -> np.ndarray:
    D = q.shape[-1]
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    qh = np.transpose(q, (1, 0, 2))  # [H, Lq, D]
    kh = np.transpose(k, (1, 0, 2))
    vh = np.transpose(v, (1, 0, 2))
    s = np.matmul(qh, np.transpose(kh, (0, 2, 1))) * sc  # [H, Lq, Lk]
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    o = np.matmul(p, vh)  # [H, Lq, D]
    return np.transpose(o, (1, 0, 2))
