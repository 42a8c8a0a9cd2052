"""Pins the norm/RoPE oracle: the reference test's closed form (golden fixture,
torch), special cases, complex rotation, norm preservation, V copy."""
import os

import numpy as np

from oracle import qknorm as oqk
from oracle.fp8 import bf16_to_f32, f32_to_bf16

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_matches_reference_closed_form_fixture():
    d = np.load(os.path.join(GOLD, "qk_norm_rope.npz"))
    B, LH, D = d["q"].shape
    L, H = 16, 4
    qo, ko, kpre = oqk.qk_norm_rope_paired(d["q"], d["k"], L, H, 1e-6, d["qw"], d["kw"], d["cos"], d["sin"])
    for got, ref in ((qo, d["q_ref"]), (ko, d["k_ref"]), (kpre, d["k_pre_ref"])):
        a = bf16_to_f32(got)
        # one bf16 rounding away from the fp32 closed form
        assert np.all(np.abs(a - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-6)


def test_identity_rotation_is_pure_rmsnorm():
    rng = np.random.default_rng(0)
    L, H, D = 8, 3, 64
    x = bf16_to_f32(f32_to_bf16(rng.standard_normal((L, H, D)).astype(np.float32)))
    w = np.ones(D, np.float32)
    o, xh = oqk.norm_rope_heads(x, w, np.ones((L, D // 2), np.float32), np.zeros((L, D // 2), np.float32), 1e-6)
    assert np.array_equal(o, xh)
    rms = np.sqrt(np.mean(xh.astype(np.float64) ** 2, axis=-1))
    assert np.allclose(rms, 1.0, atol=1e-5)


def test_constant_head():
    L, H, D = 2, 2, 128
    x = np.full((L, H, D), 0.5, np.float32)
    eps = 1e-6
    o, xh = oqk.norm_rope_heads(x, np.ones(D, np.float32), np.ones((L, D // 2), np.float32),
                                np.zeros((L, D // 2), np.float32), eps)
    assert np.allclose(xh, 0.5 / np.sqrt(0.25 + eps), rtol=1e-6)


def test_rotation_is_complex_multiplication_and_preserves_norm():
    rng = np.random.default_rng(1)
    L, H, D = 6, 2, 128
    x = rng.standard_normal((L, H, D)).astype(np.float32)
    ang = rng.random((L, D // 2)) * 2 * np.pi
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    o, xh = oqk.norm_rope_heads(x, np.ones(D, np.float32), c, s, 1e-6)
    z = (xh[..., 0::2] + 1j * xh[..., 1::2]).astype(np.complex128) * np.exp(1j * ang)[:, None, :]
    assert np.allclose(o[..., 0::2], z.real, atol=2e-6)
    assert np.allclose(o[..., 1::2], z.imag, atol=2e-6)
    assert np.allclose(np.linalg.norm(o, axis=-1), np.linalg.norm(xh, axis=-1), rtol=1e-5)


def test_qkv_split_and_cache_semantics():
    rng = np.random.default_rng(2)
    L, H, D = 5, 3, 64
    qkv = f32_to_bf16(rng.standard_normal((L, 3 * H * D)).astype(np.float32))
    qw = kw = f32_to_bf16(np.ones(D, np.float32))
    cos = f32_to_bf16(np.ones((L, D // 2), np.float32))
    sin = f32_to_bf16(np.zeros((L, D // 2), np.float32))
    q, k, kpre, v = oqk.qkv_norm_rope_cache(qkv, H, 1e-6, qw, kw, cos, sin)
    t = qkv.reshape(L, 3, H, D)
    assert np.array_equal(v, t[:, 2])  # compact V copy
    assert np.array_equal(k, kpre)     # identity rotation: roped K == pre-RoPE K
    q2, k2, kp2 = oqk.qk_norm_rope_paired(t[None, :, 0].reshape(1, L * H, D), t[None, :, 1].reshape(1, L * H, D),
                                          L, H, 1e-6, qw, kw, cos, sin)
    assert np.array_equal(q2.reshape(L, H, D), q)
    assert np.array_equal(kp2.reshape(L, H, D), kpre)
