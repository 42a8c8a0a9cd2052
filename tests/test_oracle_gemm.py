"""Pins the GEMM oracle: brute force, exact small-integer construction (epilogue
bit for bit), linearity, bias-only, torch's CPU _scaled_mm, golden fixture."""
import os

import numpy as np
import torch

from oracle import gemm as og
from oracle.fp8 import bf16_to_f32, f32_to_bf16, f32_to_e4m3fn

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def rand_fp8(rng, shape, scale=1.0):
    return f32_to_e4m3fn((rng.standard_normal(shape) * scale).astype(np.float32).clip(-448, 448))


def test_brute_force_triple_loop():
    rng = np.random.default_rng(0)
    M, N, K = 5, 7, 33
    qa, qb = rand_fp8(rng, (M, K), 4), rand_fp8(rng, (N, K), 4)
    sa = rng.random(M).astype(np.float32) + 0.5
    sb = rng.random(N).astype(np.float32) + 0.5
    bias = f32_to_bf16(rng.standard_normal(N).astype(np.float32))
    a, b = og.dequant(qa), og.dequant(qb)
    acc = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            for k in range(K):
                acc[m, n] += float(a[m, k]) * float(b[n, k])
    assert np.array_equal(og.exact_acc(qa, qb), acc)
    bits, o = og.scaled_mm(qa, qb, sa, sb, bias)
    for m in range(M):
        for n in range(N):
            t = np.float32(np.float32(acc[m, n]) * sb[n])
            v = np.float32(float(t) * float(sa[m]) + float(bf16_to_f32(bias[n:n + 1])[0]))
            assert o[m, n] == v


def test_small_integer_exact_epilogue():
    # fp8 integers in [-8, 8], K=64: |acc| <= 4096, exact in fp32 in any order;
    # power-of-two scales keep every product exact, so the output is fixed bit for bit.
    rng = np.random.default_rng(1)
    M, N, K = 32, 24, 64
    a = rng.integers(-8, 9, (M, K)).astype(np.float32)
    b = rng.integers(-8, 9, (N, K)).astype(np.float32)
    qa, qb = f32_to_e4m3fn(a), f32_to_e4m3fn(b)
    sa = (2.0 ** rng.integers(-6, 3, M)).astype(np.float32)
    sb = (2.0 ** rng.integers(-6, 3, N)).astype(np.float32)
    bias = f32_to_bf16((rng.integers(-64, 64, N) / 8).astype(np.float32))
    bits, o = og.scaled_mm(qa, qb, sa, sb, bias)
    exact = (a.astype(np.int64) @ b.astype(np.int64).T).astype(np.float64) * sa[:, None] * sb[None, :] \
        + bf16_to_f32(bias)[None, :]
    assert np.array_equal(o, exact.astype(np.float32))
    assert np.array_equal(bits, f32_to_bf16(exact.astype(np.float32)))


def test_linearity_in_scales_and_bias_only():
    rng = np.random.default_rng(2)
    M, N, K = 16, 16, 128
    qa, qb = rand_fp8(rng, (M, K)), rand_fp8(rng, (N, K))
    sa = rng.random(M).astype(np.float32)
    sb = rng.random(N).astype(np.float32)
    _, o1 = og.scaled_mm(qa, qb, sa, sb)
    _, o2 = og.scaled_mm(qa, qb, sa * np.float32(2), sb * np.float32(4))
    assert np.array_equal(o2, o1 * np.float32(8))
    bias = f32_to_bf16(rng.standard_normal(N).astype(np.float32))
    _, o3 = og.scaled_mm(np.zeros_like(qa), qb, sa, sb, bias)
    assert np.array_equal(o3, np.broadcast_to(bf16_to_f32(bias), (M, N)))


def test_unscaled_product_matches_torch_cpu_scaled_mm():
    # CPU _scaled_mm supports tensor-wise scales only; with unit scales it gives the raw product.
    rng = np.random.default_rng(3)
    M, N, K = 32, 48, 256
    qa, qb = rand_fp8(rng, (M, K)), rand_fp8(rng, (N, K))
    ta = torch.from_numpy(qa).view(torch.float8_e4m3fn)
    tb = torch.from_numpy(qb).view(torch.float8_e4m3fn)
    one = torch.tensor(1.0)
    out = torch._scaled_mm(ta, tb.t(), one, one, out_dtype=torch.float32)
    ref = og.exact_acc(qa, qb)
    assert np.allclose(out.numpy(), ref, rtol=1e-6, atol=1e-4)


def test_reference_fp32_matches_golden():
    d = np.load(os.path.join(GOLD, "gemm_small.npz"))
    ref = og.reference_fp32(d["qa"], d["qw"], d["sa"], d["sw"], d["bias"])
    assert np.allclose(ref, d["ref"], rtol=1e-6, atol=1e-6)
    bits, o = og.scaled_mm(d["qa"], d["qw"], d["sa"], d["sw"], d["bias"])
    rms = np.sqrt(np.mean(d["ref"].astype(np.float64) ** 2))
    assert np.abs(bf16_to_f32(bits) - d["ref"]).max() <= 2e-2 * rms


def test_gelu_tanh_matches_torch():
    x = np.linspace(-8, 8, 4001).astype(np.float32)
    ref = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    assert np.allclose(og.gelu_tanh(x), ref, rtol=1e-6, atol=1e-6)
