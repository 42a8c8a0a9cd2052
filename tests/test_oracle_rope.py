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
