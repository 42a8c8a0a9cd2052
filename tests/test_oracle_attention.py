"""CPU pins of oracle/attention.py (restatement of dit.py:154-167's SDPA call)."""
import math

import numpy as np
import torch

from oracle import attention as oa
from oracle.fp8 import bf16_to_f32, f32_to_bf16


def _bf16(shape, rng, scale=1.0):
    return f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def _torch_sdpa(q, k, v, scale=None):
    """torch's own CPU SDPA in float64 on [L, H, D] arrays."""
    t = lambda a: torch.from_numpy(np.ascontiguousarray(np.transpose(a, (1, 0, 2))))[None]  # noqa: E731
    o = torch.nn.functional.scaled_dot_product_attention(t(q), t(k), t(v), is_causal=False, scale=scale)
    return np.transpose(o[0].numpy(), (1, 0, 2))


def test_matches_torch_sdpa_float64():
    rng = np.random.default_rng(0)
    for Lq, Lk, H in ((7, 13, 3), (1, 1, 1), (33, 200, 2)):
        q, k, v = _bf16((Lq, H, 128), rng), _bf16((Lk, H, 128), rng), _bf16((Lk, H, 128), rng)
        ref = _torch_sdpa(*(bf16_to_f32(a).astype(np.float64) for a in (q, k, v)))
        assert np.allclose(oa.sdpa(q, k, v), ref, rtol=1e-12, atol=1e-12)
        # explicit scale, as the reference's default 1/sqrt(D)
        ref_s = _torch_sdpa(*(bf16_to_f32(a).astype(np.float64) for a in (q, k, v)), scale=0.3)
        assert np.allclose(oa.sdpa(q, k, v, 0.3), ref_s, rtol=1e-12, atol=1e-12)


def test_planted_mistakes_are_caught():
    """A dropped scale or a softmax over the query axis disagrees with torch's SDPA."""
    rng = np.random.default_rng(1)
    q, k, v = (bf16_to_f32(_bf16((9, 2, 128), rng)).astype(np.float64) for _ in range(3))
    ref = _torch_sdpa(q, k, v)
    assert np.abs(oa.sdpa_f64(q, k, v, scale=1.0) - ref).max() > 1e-3
    qh, kh, vh = (np.transpose(a, (1, 0, 2)) for a in (q, k, v))
    s = qh @ np.transpose(kh, (0, 2, 1)) / math.sqrt(128)
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)  # wrong axis
    assert np.abs(np.transpose(p @ vh, (1, 0, 2)) - ref).max() > 1e-3


def test_closed_forms():
    rng = np.random.default_rng(2)
    H, D = 2, 128
    q = _bf16((5, H, D), rng)
    # single key: the value row itself
    k1, v1 = _bf16((1, H, D), rng), _bf16((1, H, D), rng)
    assert np.array_equal(oa.sdpa(q, k1, v1), np.broadcast_to(bf16_to_f32(v1), (5, H, D)))
    # identical keys: the mean of the value rows
    k = np.broadcast_to(_bf16((1, H, D), rng), (16, H, D)).copy()
    v = _bf16((16, H, D), rng)
    assert np.allclose(oa.sdpa(q, k, v), bf16_to_f32(v).astype(np.float64).mean(axis=0)[None], atol=1e-12)
    # one key dominating by 60 in scale units: its value row
    qd = np.zeros((3, H, D), np.float64)
    qd[..., 0] = 1.0
    kd = np.zeros((8, H, D), np.float64)
    kd[5, :, 0] = 60.0 * math.sqrt(D)
    vd = bf16_to_f32(_bf16((8, H, D), rng)).astype(np.float64)
    assert np.allclose(oa.sdpa_f64(qd, kd, vd), vd[5][None], rtol=1e-20, atol=1e-20)
    # constant value rows: the constant
    vc = np.full((16, H, D), 0.75)
    assert np.allclose(oa.sdpa_f64(bf16_to_f32(q).astype(np.float64), bf16_to_f32(_bf16((16, H, D), rng)), vc),
                       0.75, atol=1e-15)


def test_permutation_invariance_and_convexity():
    rng = np.random.default_rng(3)
    q, k, v = _bf16((11, 3, 128), rng), _bf16((40, 3, 128), rng), _bf16((40, 3, 128), rng)
    o = oa.sdpa(q, k, v)
    perm = rng.permutation(40)
    assert np.allclose(oa.sdpa(q, k[perm], v[perm]), o, atol=1e-12)
    vf = bf16_to_f32(v)
    assert (o <= vf.max(axis=0)[None] + 1e-12).all() and (o >= vf.min(axis=0)[None] - 1e-12).all()
