"""Joint-attention Q/K/V pack and cached-K rotation (numpy).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Restated from the reference's kernels in ``joyomni_ops/csrc/fused_joint_qkv_pack.cu``:

* ``joint_qkv_pack`` (``fusedJointQKVPack`` ``:81-164``)::

      Q = [img_q | rms(txt_q)]
      K = [cached_k | img_k | rms(txt_k)]
      V = [cached_v | img_v | txt_v]
      rms(x) = bf16(bf16(x * r) * w),  r = 1 / sqrt(sum(x^2) / D + eps)   (``:58-79``)

  two roundings, as the model's own RMSNorm (``deploy/xvideo/models/dit/dit.py:292-296``).
* ``cached_kv_pack`` (``fusedCachedKVPack`` ``:166-220``): for each token t of the
  concatenated cached segments and each pair (2i, 2i+1), with
  c = cos[t, 2i], s = sin[t, 2i] (fp32 full-width tables, ``:207-218``)::

      o_2i   = k_2i * c - k_2i+1 * s
      o_2i+1 = k_2i * s + k_2i+1 * c        -> bf16 (RNE)

  V segments are concatenated unchanged.

Arrays are bf16 bit patterns (uint16) shaped [L, H, D].

Pins (tests/test_oracle_kvpack.py): the reference test's closed forms
(``joyomni_ops/tests/test_parity_light.py:136-199``) evaluated with torch CPU
ops -- ``torch.cat`` plus the two-rounding norm, and ``k*cos + rotate(k)*sin``
with ``repeat_interleave`` tables; the cached rotation bit-exactly, the norm on
all but a few near-tie elements while a one-rounding norm misses many more;
identity and quarter-turn tables (exact copy / exact (-k1, k0)); a constant
row with unit weight; segment order and V copied bit-exactly.
"""
from __future__ import annotations

import numpy as np

from .fp8 import bf16_round, bf16_to_f32, f32_to_bf16


def rms_two_round(x_u16: np.ndarray, w_u16: np.ndarray, eps: float) -> np.ndarray:
    """bf16(bf16(x * r) * w) per row of the last axis; r in fp32 from a float64 sum."""
    x = bf16_to_f32(x_u16)
    D = x.shape[-1]
    ss = np.sum(x.astype(np.float64) ** 2, axis=-1, keepdims=True)
    r = (1.0 / np.sqrt(ss / D + eps)).astype(np.float32)
    n = bf16_round((x * r).astype(np.float32))
    return f32_to_bf16((n * bf16_to_f32(w_u16)).astype(np.float32))


def joint_qkv_pack(img_q, img_k, img_v, txt_q, txt_k, txt_v, cached_k, cached_v, qw, kw, eps):
    """Oracle of ``fused_joint_qkv_pack`` for bf16 [L, H, D] inputs (cached_* may be None)."""
    q = np.concatenate((img_q, rms_two_round(txt_q, qw, eps)), axis=0)
    k_parts = [img_k, rms_two_round(txt_k, kw, eps)]
    v_parts = [img_v, txt_v]
    if cached_k is not None:
        k_parts.insert(0, cached_k)
        v_parts.insert(0, cached_v)
    return q, np.concatenate(k_parts, axis=0), np.concatenate(v_parts, axis=0)


def rotate_pairs(k_u16: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """k: bf16 [L, H, D]; cos/sin: fp32 [L, D] (entry 2i used for pair i). Returns bf16 bits."""
    k = bf16_to_f32(k_u16)
    c = np.asarray(cos, np.float32)[:, None, 0::2]
    s = np.asarray(sin, np.float32)[:, None, 0::2]
    x0 = k[..., 0::2]
    x1 = k[..., 1::2]
    o = np.empty_like(k)
    o[..., 0::2] = x0 * c - x1 * s
    o[..., 1::2] = x0 * s + x1 * c
    return f32_to_bf16(o)


def cached_kv_pack(key0, value0, key1, value1, cos, sin):
    """Oracle of ``fused_cached_kv_pack``: bf16 [L, H, D] segments, fp32 [L0+L1, D] tables."""
    keys = [key0] + ([key1] if key1 is not None else [])
    vals = [value0] + ([value1] if value1 is not None else [])
    k = np.concatenate(keys, axis=0)
    L, H, D = k.shape
    return (rotate_pairs(k, np.asarray(cos).reshape(L, D), np.asarray(sin).reshape(L, D)),
            np.concatenate(vals, axis=0))
