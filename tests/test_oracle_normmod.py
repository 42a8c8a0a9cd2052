"""Pins the norm + adaLN oracle against torch's own CPU layer_norm / RMS formula,
closed-form special cases, and planted mistakes that the pins must reject."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import normmod as onm
from oracle import quant as oq
from oracle.fp8 import bf16_to_f32


def u16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def torch_ref(x, g, b, sc, sh, norm_type, eps):
    """fp32 library LayerNorm / the RMS formula of sgl_fused_ops.py:202-209, then adaLN, one rounding."""
    xf = x.float()
    if norm_type == 0:
        y = F.layer_norm(xf, (x.shape[1],), None if g is None else g.float(),
                         None if (g is None or b is None) else b.float(), eps)
    else:
        y = xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps)
        if g is not None:
            y = y * g.float()
    return (y * (1 + sc.float()) + sh.float()).to(x.dtype)


def inputs(M, N, rows, seed, affine):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(M, N, generator=g) * 3 + 0.5).to(torch.bfloat16)
    sc = (torch.randn(rows, N, generator=g) * 0.2).to(torch.bfloat16)
    sh = (torch.randn(rows, N, generator=g) * 0.2).to(torch.bfloat16)
    ga = (1 + 0.1 * torch.randn(N, generator=g)).to(torch.bfloat16) if affine else None
    be = (0.1 * torch.randn(N, generator=g)).to(torch.bfloat16) if affine else None
    return x, ga, be, sc, sh


@pytest.mark.parametrize("norm_type", [0, 1])
@pytest.mark.parametrize("affine,rows", [(False, 1), (True, 1), (False, 64)])
def test_matches_torch_library_norm(norm_type, affine, rows):
    x, ga, be, sc, sh = inputs(64, 512, rows, norm_type * 10 + rows, affine)
    cv = lambda t: None if t is None else u16(t)  # noqa: E731
    got = onm.norm_scale_shift(u16(x), cv(ga), cv(be), u16(sc), u16(sh), norm_type, 1e-6)
    ref = u16(torch_ref(x, ga, be, sc, sh, norm_type, 1e-6))
    diff = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    assert diff.max() <= 1 and np.count_nonzero(diff) <= 2e-3 * got.size, np.count_nonzero(diff)


def test_planted_mistakes_are_rejected():
    """The torch pin above would catch an unbiased variance or a dropped '1 +'."""
    x, _, _, sc, sh = inputs(64, 512, 1, 3, False)
    xf = bf16_to_f32(u16(x))
    ref = u16(torch_ref(x, None, None, sc, sh, 0, 1e-6))
    # unbiased variance
    d = xf - xf.mean(1, keepdims=True)
    r = 1.0 / np.sqrt((d.astype(np.float64) ** 2).sum(1, keepdims=True) / (xf.shape[1] - 1) + 1e-6)
    bad = onm.from_f32((d * r) * (1 + bf16_to_f32(u16(sc))) + bf16_to_f32(u16(sh)), "bf16")
    assert np.count_nonzero(bad != ref) > 0.05 * ref.size
    # scale applied without the "1 +"
    r32 = r.astype(np.float32)
    bad2 = onm.from_f32((d * r32) * bf16_to_f32(u16(sc)) + bf16_to_f32(u16(sh)), "bf16")
    assert np.count_nonzero(bad2 != ref) > 0.5 * ref.size


def test_constant_row_is_exact():
    N = 256
    x = np.full((3, N), 0x4040, np.uint16)  # bf16 3.0 in every element
    sc = np.full((1, N), 0x3F00, np.uint16)  # 0.5
    sh = np.full((1, N), 0x3E80, np.uint16)  # 0.25
    gb = np.full(N, 0x3F80, np.uint16)       # gamma 1.0
    bb = np.full(N, 0x4000, np.uint16)       # beta 2.0
    y = bf16_to_f32(onm.norm_scale_shift(x, gb, bb, sc, sh, 0, 1e-6))
    assert np.all(y == 2.0 * 1.5 + 0.25)
    y = bf16_to_f32(onm.norm_scale_shift(x, None, bb, sc, sh, 0, 1e-6))  # beta without gamma is ignored
    assert np.all(y == 0.25)


def test_fp8_variant_is_quantiser_of_output():
    x, ga, be, sc, sh = inputs(32, 1024, 1, 7, True)
    q, s, y = onm.norm_scale_shift_fp8(u16(x), u16(ga), u16(be), u16(sc), u16(sh), 0, 1e-6)
    q2, s2 = oq.quant_per_token(y, "bf16", "div")
    assert np.array_equal(q, q2) and np.array_equal(s, s2)
    assert np.array_equal(y, onm.norm_scale_shift(u16(x), u16(ga), u16(be), u16(sc), u16(sh), 0, 1e-6))
