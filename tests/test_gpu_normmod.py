"""GPU parity: fused_norm_scale_shift (HIP) and its FP8-emitting variant vs the oracle.
Norm output within one rounding step of the oracle plus the fp32 error of its
terms, differing at all on at most 0.1 % of bf16/fp16 elements; the FP8 bytes and
scales are bit-exact against the quantiser oracle applied to the kernel's own
rounded output."""
import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, gen, u16, u8
from oracle import normmod as onm
from oracle import quant as oq

pytestmark = pytest.mark.gpu

DT = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}


def bits(t):
    if t is None:
        return None
    if t.dtype == torch.float32:
        return t.detach().cpu().numpy()
    return u16(t)


def make(M, N, rows, dtype, affine, seed):
    g = gen(seed)
    x = (torch.randn(M, N, generator=g) * 2 + 0.3).to(dtype)
    sc = (torch.randn(rows, N, generator=g) * 0.2).to(dtype)
    sh = (torch.randn(rows, N, generator=g) * 0.2).to(dtype)
    ga = (1 + 0.1 * torch.randn(N, generator=g)).to(dtype) if affine else None
    be = (0.1 * torch.randn(N, generator=g)).to(dtype) if affine else None
    return x, ga, be, sc, sh


def dev(t):
    return None if t is None else t.to(DEV)


def assert_close(got, exp, inputs, dtype, norm_type, what):
    """|got - exp| <= 1 ulp(exp) + 2^-16 * (|norm term| + |shift terms|): one rounding step, plus
    the fp32 error of the terms (the 5120-term sums of mean and variance carry ~2^-17 relative
    error in any summation order), which matters where they cancel to near zero or for fp32
    output; at most 0.1 % of bf16/fp16 outputs differ at all."""
    nt = 0 if norm_type == "layer" else 1
    mag = onm.term_magnitude(*[None if t is None else onm.to_f32(bits(t), DT[dtype]) for t in inputs],
                             nt, 1e-6)
    a = onm.to_f32(got, DT[dtype]).astype(np.float64)
    b = onm.to_f32(exp, DT[dtype]).astype(np.float64)
    ulp_scale = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10 if dtype == torch.float16 else 2.0 ** -23
    bound = ulp_scale * np.abs(b) + 2.0 ** -16 * mag + 1e-30
    bad = np.abs(a - b) > bound
    assert not bad.any(), f"{what}: {np.count_nonzero(bad)} values outside the bound"
    if dtype != torch.float32:
        assert np.count_nonzero(a != b) <= 1e-3 * a.size + 2, f"{what}: {np.count_nonzero(a != b)} values differ"


@pytest.mark.parametrize("norm_type", ["layer", "rms"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M,N,rows,affine", [(300, 5120, 1, False), (64, 4096, 64, True),
                                             (100, 2048, 100, True), (9, 256, 1, False),
                                             (7, 8192, 1, False), (12, 4104, 1, False),
                                             (17, 4100, 1, True), (5, 12288, 5, False)])
def test_norm_scale_shift(norm_type, dtype, M, N, rows, affine):
    """Vector path: the persistent row walk (broadcast modulation, no affine; N = 5120, 8192,
    4104 with a partly idle last wave), one workgroup per row (N = 4096 per-row modulation),
    one wave per row (N = 2048, 256); the scalar path (N = 4100, 12288, fp32)."""
    import joyomni_ops as jo
    announce("norm_scale_shift", norm_type, dtype, M, N, rows, affine)
    x, ga, be, sc, sh = make(M, N, rows, dtype, affine, M + N + rows)
    y = jo.fused_norm_scale_shift(dev(x), dev(ga), dev(be), dev(sc), dev(sh), norm_type, 1e-6)
    torch.cuda.synchronize()
    nt = 0 if norm_type == "layer" else 1
    exp = onm.norm_scale_shift(bits(x), bits(ga), bits(be), bits(sc), bits(sh), nt, 1e-6, DT[dtype])
    assert_close(bits(y), exp, (x, ga, be, sc, sh), dtype, norm_type, f"{norm_type} {dtype} {M}x{N}")


def test_norm_strided_rows():
    import joyomni_ops as jo
    announce("norm_scale_shift strided")
    x, _, _, sc, sh = make(40, 1024, 1, torch.bfloat16, False, 3)
    wide = torch.zeros(40, 1024 + 64, dtype=torch.bfloat16)
    wide[:, :1024] = x
    y = jo.fused_norm_scale_shift(wide.to(DEV)[:, :1024], None, None, dev(sc), dev(sh), "layer", 1e-6)
    torch.cuda.synchronize()
    exp = onm.norm_scale_shift(u16(x), None, None, u16(sc), u16(sh), 0, 1e-6)
    assert_close(u16(y), exp, (x, None, None, sc, sh), torch.bfloat16, "layer", "strided")


@pytest.mark.parametrize("exact_division", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,rows", [(10800, 5120, 1), (512, 5120, 512), (40, 1024, 1), (33, 4100, 1)])
def test_norm_fp8(exact_division, dtype, M, N, rows):
    import joyomni_ops as jo
    announce("norm fp8", exact_division, dtype, M, N, rows)
    x, _, _, sc, sh = make(M, N, rows, dtype, False, 11 + M)
    xd = x.to(DEV)
    q = torch.empty(M, N, dtype=torch.float8_e4m3fn, device=DEV)
    s = torch.empty(M, 1, device=DEV)
    y = torch.empty(M, N, dtype=dtype, device=DEV)
    jo.fused_norm_scale_shift_fp8(xd, None, None, dev(sc), dev(sh), "layer", 1e-6, q, s, y, exact_division)
    # the same call without the optional y output gives the same bytes
    q2 = torch.empty_like(q)
    s2 = torch.empty_like(s)
    jo.fused_norm_scale_shift_fp8(xd, None, None, dev(sc), dev(sh), "layer", 1e-6, q2, s2, None, exact_division)
    # and y equals the plain op
    y_plain = jo.fused_norm_scale_shift(xd, None, None, dev(sc), dev(sh), "layer", 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(q.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(s, s2)
    assert torch.equal(y, y_plain)
    rows_chk = np.arange(M) if M <= 1024 else np.sort(np.random.default_rng(0).choice(M, 512, replace=False))
    ri = torch.from_numpy(rows_chk).to(DEV)
    y_bits = u16(y[ri])
    qe, se = oq.quant_per_token(y_bits, DT[dtype], "div" if exact_division else "rcp")
    assert np.array_equal(u8(q[ri]), qe), "fp8 bytes differ from the quantiser of y"
    assert np.array_equal(s[ri].cpu().numpy().reshape(-1), se), "scales differ"
    rc = torch.from_numpy(rows_chk)
    xs, scs, shs = x[rc], (sc if rows == 1 else sc[rc]), (sh if rows == 1 else sh[rc])
    exp = onm.norm_scale_shift(u16(xs), None, None, u16(scs), u16(shs), 0, 1e-6, DT[dtype])
    assert_close(y_bits, exp, (xs, None, None, scs, shs), dtype, "layer", "y")


@pytest.mark.parametrize("affine", [False, True])
def test_norm_fp8_matches_separate_quantiser_full_rows(affine):
    """FP8 variant == per_token_quant_fp8(fused_norm_scale_shift(x)) on the device, whole tensor
    (without affine weights: the persistent row walk; with them: one workgroup per row)."""
    import joyomni_ops as jo
    announce("norm fp8 vs separate quant", affine)
    x, ga, be, sc, sh = make(2048, 5120, 1, torch.bfloat16, affine, 5)
    xd, gd, bd, scd, shd = dev(x), dev(ga), dev(be), dev(sc), dev(sh)
    q = torch.empty(2048, 5120, dtype=torch.float8_e4m3fn, device=DEV)
    s = torch.empty(2048, 1, device=DEV)
    jo.fused_norm_scale_shift_fp8(xd, gd, bd, scd, shd, "layer", 1e-6, q, s)
    y = jo.fused_norm_scale_shift(xd, gd, bd, scd, shd, "layer", 1e-6)
    q_ref = torch.empty_like(q)
    s_ref = torch.empty_like(s)
    jo.per_token_quant_fp8(y, q_ref, s_ref, True)
    torch.cuda.synchronize()
    assert torch.equal(q.view(torch.uint8), q_ref.view(torch.uint8)) and torch.equal(s, s_ref)


@pytest.mark.parametrize("norm_type", ["layer", "rms"])
@pytest.mark.parametrize("M,N,rows", [(40, 5120, 1), (16, 4096, 16), (8, 2048, 8), (5, 4100, 5)])
def test_fp16_zero_rows_output_denormal_shift(norm_type, M, N, rows):
    """A zero input row normalises to 0, so its output is the shift itself: with fp16-denormal
    shift values a conversion that flushed them would show (every kernel shape)."""
    import joyomni_ops as jo
    announce("norm fp16 denormal shift", norm_type, M, N, rows)
    x, _, _, sc, sh = make(M, N, rows, torch.float16, False, 21 + N)
    x[::3] = 0
    sh_bits = u16(sh).copy()
    sh_bits[:, ::4] = np.random.default_rng(N).integers(1, 1024, sh_bits[:, ::4].shape).astype(np.uint16)
    sh = torch.from_numpy(sh_bits.view(np.int16)).view(torch.float16)
    y = jo.fused_norm_scale_shift(dev(x), None, None, dev(sc), dev(sh), norm_type, 1e-6)
    torch.cuda.synchronize()
    yb = u16(y)
    exp_rows = np.broadcast_to(sh_bits, (M, N))[::3]
    assert np.array_equal(yb[::3], exp_rows)
    nt = 0 if norm_type == "layer" else 1
    exp = onm.norm_scale_shift(bits(x), None, None, bits(sc), sh_bits, nt, 1e-6, "fp16")
    assert_close(yb, exp, (x, None, None, sc, sh), torch.float16, norm_type, "denormal shift")


def test_norm_argument_errors():
    import joyomni_ops as jo
    announce("norm argument errors")
    x = torch.zeros(4, 64, dtype=torch.bfloat16, device=DEV)
    sc = torch.zeros(2, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="broadcast"):
        jo.fused_norm_scale_shift(x, None, None, sc, sc, "layer", 1e-6)
    with pytest.raises(RuntimeError, match="divisible by 4"):
        jo.fused_norm_scale_shift(x[:, :62], None, None, sc[:1, :62], sc[:1, :62], "layer", 1e-6)
    with pytest.raises(RuntimeError, match="dtype must match"):
        jo.fused_norm_scale_shift(x, None, None, sc[:1].half(), sc[:1].half(), "layer", 1e-6)
