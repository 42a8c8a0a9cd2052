"""GPU parity: per-token FP8 quantisation, bit-exact bytes and scales vs the oracle."""
import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, gen, outlier_acts, u16, u8
from oracle import quant as oq
from oracle.fp8 import bf16_to_f32

pytestmark = pytest.mark.gpu


def run_quant(x: torch.Tensor, exact_division: bool):
    import joyomni_ops as jo
    xd = x.to(DEV)
    q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=DEV)
    s = torch.empty(x.shape[0], 1, dtype=torch.float32, device=DEV)
    if exact_division:
        jo.per_token_quant_fp8(xd, q, s, True)
    else:
        jo.sgl_per_token_quant_fp8(xd, q, s)
    torch.cuda.synchronize()
    return u8(q), s.cpu().numpy().reshape(-1)


def check(x: torch.Tensor, variant: str, rows=None):
    name = "bf16" if x.dtype == torch.bfloat16 else "fp16"
    q, s = run_quant(x, variant == "div")
    xs = u16(x) if rows is None else u16(x[rows])
    qr, sr = oq.quant_per_token(xs, name, variant)
    if rows is not None:
        q, s = q[rows], s[rows]
    assert np.array_equal(s, sr), "scales differ"
    bad = np.count_nonzero(q != qr)
    assert bad == 0, f"{bad} of {q.size} fp8 bytes differ"


@pytest.mark.parametrize("variant", ["div", "rcp"])
def test_reference_test_geometry_zero_row(variant):
    announce("quant m67 k4096 zero-row", variant)
    x = torch.randn(67, 4096, generator=gen(0)).to(torch.bfloat16)
    x[0].zero_()
    check(x, variant)


@pytest.mark.parametrize("variant", ["div", "rcp"])
@pytest.mark.parametrize("M,K", [(256, 4096), (64, 5120), (512, 5120), (1, 13824), (1560, 4096)])
def test_outlier_activations(variant, M, K):
    announce("quant outliers", M, K, variant)
    check(outlier_acts(M, K, gen(M + K)), variant)


@pytest.mark.parametrize("K", [5120, 13824])
def test_full_size_rows(K):
    announce("quant full M=10800", K)
    x = outlier_acts(10800, K, gen(K))
    rows = np.sort(np.random.default_rng(K).choice(10800, 384, replace=False))
    check(x, "div", rows)


@pytest.mark.parametrize("variant", ["div", "rcp"])
def test_fp16_and_ragged_k(variant):
    announce("quant fp16 / ragged K", variant)
    check((torch.randn(33, 2048, generator=gen(5)) * 7).to(torch.float16), variant)
    for K in (1, 7, 100, 1000, 20000):  # K % 8 != 0 or K > 64*32*8 -> scalar path
        check(torch.randn(9, K, generator=gen(K)).to(torch.bfloat16), variant)


@pytest.mark.parametrize("variant", ["div", "rcp"])
@pytest.mark.parametrize("K", [2048, 12288, 16384])
def test_fp16_denormal_inputs(variant, K):
    """fp16 rows with a small absmax, where fp16 denormal inputs (|x| < 2^-14) quantise to
    nonzero fp8 bytes: a conversion that flushed them would write 0. K = 16384 is the
    widest row kept in registers."""
    announce("quant fp16 denormals", variant, K)
    g = gen(K + 3)
    x = torch.randn(16, K, generator=g) * 1e-3
    x[:, ::7] = (torch.rand(16, x[:, ::7].shape[1], generator=g) - 0.5) * 2.0 ** -13
    x = x.to(torch.float16)
    bits = u16(x)
    den = ((bits & 0x7C00) == 0) & ((bits & 0x3FF) != 0)
    qr, _ = oq.quant_per_token(bits, "fp16", variant)
    assert den.mean() > 0.1 and np.count_nonzero(qr[den] & 0x7F) > 0.9 * den.sum()
    check(x, variant)


def test_every_bf16_value_against_many_scales():
    """Every finite bf16 pattern is quantised under scales spanning the whole
    range: rows hold all |x| <= a plus a itself (fixing the row absmax)."""
    announce("quant exhaustive bf16 cast")
    allv = bf16_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    finite = np.arange(65536)[np.isfinite(allv)].astype(np.uint16)
    rng = np.random.default_rng(7)
    amax_vals = [1e-30, 1e-8, 3e-6, 1e-3, 0.07, 1.0, 3.14159, 100.0, 448.0, 1e4, 3e38]
    amax_vals += list(np.exp(rng.uniform(-20, 20, 24)))
    rows = []
    K = 8192
    for a in amax_vals:
        ab = u16(torch.tensor([a]).to(torch.bfloat16))[0]
        af = bf16_to_f32(np.array([ab], np.uint16))[0]
        xs = finite[np.abs(bf16_to_f32(finite)) <= af]
        xs = np.concatenate([xs, np.full((-len(xs)) % (K - 1), ab, np.uint16)])
        for chunk in xs.reshape(-1, K - 1):
            rows.append(np.concatenate([[ab], chunk]).astype(np.uint16))
    x = torch.from_numpy(np.stack(rows).view(np.int16)).view(torch.bfloat16)
    for variant in ("div", "rcp"):
        check(x, variant)


def test_nonfinite_rows_follow_torch():
    announce("quant inf rows")
    x = torch.randn(4, 256, generator=gen(9)).to(torch.bfloat16)
    x[1, 5] = float("inf")
    x[2, 7] = float("-inf")
    q, s = run_quant(x, True)
    qr, sr = oq.quant_per_token(u16(x), "bf16", "div")
    assert np.array_equal(s, sr)
    # finite rows exact; rows with inf: scale inf, finite elements -> 0, inf -> NaN code
    assert np.array_equal(q[[0, 3]], qr[[0, 3]])
    assert np.array_equal(q[1] & 0x7F, qr[1] & 0x7F) and np.array_equal(q[2] & 0x7F, qr[2] & 0x7F)


# Row counts above what one round of resident waves holds (every row checked), for
# 1, 2, 2 ragged, 4, 8, 12 and 16 vectors per lane.
@pytest.mark.parametrize("M,K", [(9000, 512), (9000, 1024), (9001, 1000), (8000, 2048), (5000, 4096),
                                 (3500, 5120), (2500, 8192)])
def test_many_rows_every_row(M, K):
    announce("quant many rows", M, K)
    x = outlier_acts(M, K, gen(M ^ K))
    check(x, "div")
    check(x.to(torch.float16), "rcp")


def test_many_rows_nonfinite_rows():
    announce("quant many rows, inf rows")
    M, K = 9000, 1024
    x = outlier_acts(M, K, gen(11))
    bad = [17, 4500, 8999]
    x[17, 3] = float("inf")
    x[4500, 1000] = float("-inf")
    x[8999, 0] = float("nan")
    q, s = run_quant(x, True)
    qr, sr = oq.quant_per_token(u16(x), "bf16", "div")
    good = np.setdiff1d(np.arange(M), bad)
    assert np.array_equal(s[good], sr[good]) and np.array_equal(q[good], qr[good])
    assert np.isinf(s[17]) and np.isinf(s[4500]) and np.isnan(s[8999])
    assert np.array_equal(q[bad] & 0x7F, qr[bad] & 0x7F)
