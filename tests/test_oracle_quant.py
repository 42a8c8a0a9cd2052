"""Pins the quantiser oracle: torch library routines on the reference formula,
the independent C restatement, golden fixtures, special cases, and the
exhaustive proof that the device's division formula equals IEEE division."""
import ctypes
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from oracle import quant as oq
from oracle.fp8 import FP8_MAX

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = os.path.join(ROOT, "tests", "golden")
LIBORACLE = os.path.join(ROOT, "oracle", "liboracle.so")


def u16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def torch_quant(x, variant):
    absmax = x.abs().amax(dim=1, keepdim=True).float().clamp_min(1e-8)
    s = absmax / FP8_MAX
    v = x.float() / s if variant == "div" else x.float() * (1.0 / s)
    return v.clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn).view(torch.uint8).numpy(), s.reshape(-1).numpy()


def oracle_lib():
    if not os.path.exists(LIBORACLE):
        pytest.skip("oracle/liboracle.so not built (make -C oracle)")
    lib = ctypes.CDLL(LIBORACLE)
    lib.oracle_quant_rows.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                      ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.oracle_check_device_division.restype = ctypes.c_int64
    lib.oracle_check_device_division.argtypes = [
        ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32, ctypes.POINTER(ctypes.c_int64),
        ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint32)]
    return lib


def c_quant(lib, x_u16, is_fp16, variant):
    M, K = x_u16.shape
    q = np.empty((M, K), np.uint8)
    s = np.empty(M, np.float32)
    x = np.ascontiguousarray(x_u16)
    lib.oracle_quant_rows(x.ctypes.data, int(is_fp16), M, K, 0 if variant == "div" else 1,
                          q.ctypes.data, s.ctypes.data)
    return q, s


@pytest.mark.parametrize("variant", ["div", "rcp"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_numpy_oracle_matches_torch_formula(variant, dtype):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(257, 1536, generator=g)
    x[:, ::97] *= 20
    x[5].zero_()
    x[7] = 3.0  # constant row: every element is the absmax
    x = x.to(dtype)
    q, s = oq.quant_per_token(u16(x), "bf16" if dtype == torch.bfloat16 else "fp16", variant)
    qt, st = torch_quant(x, variant)
    assert np.array_equal(s, st)
    assert np.array_equal(q, qt)


@pytest.mark.parametrize("variant", ["div", "rcp"])
def test_c_oracle_matches_numpy_oracle(variant):
    lib = oracle_lib()
    rng = np.random.default_rng(4)
    x = torch.from_numpy(rng.standard_normal((129, 2048)).astype(np.float32) * 3).to(torch.bfloat16)
    for dt, name in ((torch.bfloat16, "bf16"), (torch.float16, "fp16")):
        xb = u16(x.to(dt))
        qn, sn = oq.quant_per_token(xb, name, variant)
        qc, sc = c_quant(lib, xb, name == "fp16", variant)
        assert np.array_equal(sn, sc)
        assert np.array_equal(qn, qc)


@pytest.mark.parametrize("fixture", ["quant_m67_zero_row.npz", "quant_outliers.npz"])
def test_oracle_matches_golden(fixture):
    d = np.load(os.path.join(GOLD, fixture))
    q, s = oq.quant_per_token(d["x"], "bf16", "div")
    assert np.array_equal(s, d["s"])
    assert np.array_equal(q, d["q_div"])
    q, _ = oq.quant_per_token(d["x"], "bf16", "rcp")
    assert np.array_equal(q, d["q_rcp"])


def test_special_cases():
    x = np.zeros((2, 64), np.uint16)
    x[1, 3] = 0x3F80  # 1.0 in bf16, the only non-zero
    q, s = oq.quant_per_token(x, "bf16", "div")
    assert s[0] == np.float32(np.float32(1e-8) / np.float32(448))  # zero row: clamp_min(1e-8)
    assert not q[0].any()
    assert q[1, 3] == 0x7E  # absmax element -> 448
    assert np.count_nonzero(q[1]) == 1


def test_division_and_reciprocal_variants_differ():
    # The two reference roundings disagree on a small fraction of N(0,1) bytes.
    g = torch.Generator().manual_seed(0)
    x = torch.randn(512, 4096, generator=g).to(torch.bfloat16)
    qd, _ = oq.quant_per_token(u16(x), "bf16", "div")
    qr, _ = oq.quant_per_token(u16(x), "bf16", "rcp")
    diff = np.count_nonzero(qd != qr)
    assert 0 < diff < qd.size * 1e-3
    # every disagreement is one code step
    assert np.all(np.abs(qd[qd != qr].astype(np.int16) - qr[qd != qr].astype(np.int16)) == 1)


@pytest.mark.parametrize("is_fp16", [0, 1])
def test_device_division_formula_exhaustive(is_fp16):
    """r = RN(1/s); q0 = x*r; e = fma(-q0, s, x); copysign(fma(e, r, q0), x) gives
    the same e4m3fn byte as IEEE x/s for every 16-bit x and every quantiser scale."""
    lib = oracle_lib()

    def run(a0):
        n = ctypes.c_int64()
        fx, fa = ctypes.c_uint32(), ctypes.c_uint32()
        bad = lib.oracle_check_device_division(is_fp16, a0, a0 + 1024, ctypes.byref(n),
                                               ctypes.byref(fx), ctypes.byref(fa))
        return bad, n.value, fx.value, fa.value

    with ThreadPoolExecutor(max(1, min(16, os.cpu_count() or 1))) as ex:
        res = list(ex.map(run, range(0, 0x8000, 1024)))
    bad = sum(r[0] for r in res)
    pairs = sum(r[1] for r in res)
    assert pairs > 9e8
    assert bad == 0, [r for r in res if r[0]][:1]


def test_scaled_absmax_stays_below_the_rounding_midpoint():
    """The device quantiser converts x / s (or x * (1 / s)) without clamping on rows
    with a finite scale. That equals clamp-then-cast only if the scaled absmax never
    reaches 464, the midpoint between 448 and the next e4m3 step: checked over every
    positive finite bf16 and fp16 absmax, both roundings (division emulated as the
    kernel does it: reciprocal, two FMAs)."""
    bf = (np.arange(1, 0x7F80, dtype=np.uint32) << 16).view(np.float32)
    fp = np.arange(1, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    for amax in (bf, fp):
        s = (np.maximum(amax, np.float32(1e-8)) / np.float32(448)).astype(np.float32)
        r = (np.float32(1) / s).astype(np.float32)
        q0 = (amax * r).astype(np.float32)
        e = (-q0.astype(np.float64) * s + amax).astype(np.float32)
        q1 = (e.astype(np.float64) * r + q0).astype(np.float32)
        for v in (q0, q1):
            assert v.max() < 464.0 and v.max() <= np.float32(448) * (1 + 2.0 ** -22)
        assert (q0 > 448).any()  # the bound is reached: the conversion's rounding does the clamp
