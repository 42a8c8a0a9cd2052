"""Pins the RoPE-table oracle with closed forms and invariants."""
import numpy as np

from oracle import rope as orope
from oracle.fp8 import bf16_to_f32


def test_frequencies_closed_form():
    f = orope.axis_freqs(44, 10000.0)
    exact = 1.0 / 10000.0 ** (np.arange(0, 44, 2) / 44.0)
    assert f[0] == 1.0
    assert np.allclose(f, exact, rtol=2e-7)


def test_tables_structure_and_invariants():
    frames, h, w = [0, 1, 2], 3, 5
    cos, sin, cb, sb = orope.rope_half_tables(frames, h, w, (44, 42, 42), 10000.0)
    L = 3 * 3 * 5
    assert cos.shape == (L, 64)
    assert np.allclose(cos ** 2 + sin ** 2, 1.0, atol=1e-6)
    # token 0 is (0,0,0): identity rotation
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    t, hh, ww = orope.grid_positions(frames, h, w)
    # t-dims depend only on t, h-dims only on h, w-dims only on w
    for lo, hi, pos in ((0, 22, t), (22, 43, hh), (43, 64, ww)):
        for p in np.unique(pos):
            rows = cos[pos == p, lo:hi]
            assert np.all(rows == rows[0])
    # the first frequency of every axis is 1: angle == position
    assert np.allclose(cos[:, 0], np.cos(t), atol=1e-6)
    assert np.allclose(cos[:, 22], np.cos(hh), atol=1e-6)
    assert np.allclose(cos[:, 43], np.cos(ww), atol=1e-6)
    # token order: t-major, then h, then w
    assert list(t[:16]) == [0] * 15 + [1]
    assert list(ww[:6]) == [0, 1, 2, 3, 4, 0]
    assert np.all(np.abs(bf16_to_f32(cb) - cos) <= np.abs(cos) * 2.0 ** -8 + 1e-30)


def _angles64(frames, h, w, dims, theta):
    """float64 angles from the fp32 per-axis angles of the oracle's 3-D tables."""
    pos = orope.grid_positions(frames, h, w)
    parts = []
    for dim, p in zip(dims, pos):
        f = orope.axis_freqs(dim, theta)
        parts.append((p[:, None].astype(np.float32) * f[None, :]).astype(np.float32).astype(np.float64))
    return np.concatenate(parts, axis=1)


def test_source_id_zero_is_identity():
    """Target tokens (source id 0) keep the plain 3-D tables bit for bit (dit.py:1104,1153-1154)."""
    c3, s3, cb3, sb3 = orope.rope_half_tables([0, 1], 3, 4, (16, 56, 56), 256.0)
    c, s, cb, sb = orope.visual_half_tables((2, 3, 4))
    assert np.array_equal(c, c3) and np.array_equal(s, s3)
    assert np.array_equal(cb, cb3) and np.array_equal(sb, sb3)


def test_source_id_composition_matches_exact_angle_sum():
    """[current | ref video] and ref-image tables equal cos/sin of (3-D angle + role angle)."""
    frames, h, w, dims = [0, 1], 3, 4, (16, 56, 56)
    a3 = _angles64(frames, h, w, dims, 256.0)
    n = a3.shape[0]
    fr = orope.axis_freqs(128, 256.0)
    for ref_image, sid_cur in ((False, 0.0), (True, 2.0)):
        c, s, _, _ = orope.visual_half_tables((2, h, w), ref_video_frames=2, ref_image_cache=ref_image)
        sid = np.concatenate([np.full(n, sid_cur), np.full(n, 1.0)]).astype(np.float32)
        ar = (sid[:, None] * fr[None, :]).astype(np.float32).astype(np.float64)
        ang = np.concatenate([a3, a3]) + ar
        assert np.abs(c - np.cos(ang)).max() < 4e-7 and np.abs(s - np.sin(ang)).max() < 4e-7
        # planted mistakes miss by far more: opposite sign of the role angle, role theta 10000
        assert np.abs(c - np.cos(np.concatenate([a3, a3]) - ar)).max() > 1e-2
        ar_wrong = (sid[:, None] * orope.axis_freqs(128, 10000.0)[None, :]).astype(np.float64)
        assert np.abs(c - np.cos(np.concatenate([a3, a3]) + ar_wrong)).max() > 1e-2
        # the ref-video role rotates every pair: its first pair turns by exactly 1 rad more
        assert np.abs(c[n:, 0] - np.cos(a3[:, 0] + 1.0)).max() < 4e-7


def test_source_id_role_dim_limits_rotated_pairs():
    """Pairs past role_dim keep the 3-D values exactly; a role_dim above head_dim is clamped."""
    c3, s3, _, _ = orope.rope_half_tables([0], 2, 3, (16, 56, 56), 256.0)
    cr, sr = orope.source_id_half(np.full(6, 1.0), 128, role_dim=64)
    assert np.all(cr[:, 32:] == 1.0) and np.all(sr[:, 32:] == 0.0)
    c, s = orope.compose(c3, s3, cr, sr)
    assert np.array_equal(c[:, 32:], c3[:, 32:]) and np.array_equal(s[:, 32:], s3[:, 32:])
    assert not np.array_equal(c[:, :32], c3[:, :32])
    cr2, _ = orope.source_id_half(np.full(6, 1.0), 128, role_dim=512)
    cr3, _ = orope.source_id_half(np.full(6, 1.0), 128, role_dim=128)
    assert np.array_equal(cr2, cr3)
