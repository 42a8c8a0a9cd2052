"""Writes the committed golden fixtures of this directory.

The reference repository holds no golden vectors for this path (its tests draw
inputs on the GPU, joyomni_ops/tests/test_parity_light.py:15-16). These
fixtures are produced on the CPU by torch library routines evaluating the
reference's own formulas, independently of the numpy/C oracle they pin:

* quant_*.npz  -- _quantize_per_token_impl (deploy/xvideo/models/dit/fp8_linear.py:38-43):
  torch amax / division / clamp / e4m3fn cast; plus the reciprocal-multiply
  variant of joyomni_ops/csrc/per_token_quant_fp8_rocm.hip:72-77.
  Geometries: the reference test's M=67 with a zero row (test_parity_light.py:113-120,
  K reduced to 512) and benchmark cfg 0's outlier distribution (K reduced to 1024).
* gemm_small.npz -- torch fp8 -> fp32 dequantisation and float64 matmul, the
  fp32 dequantise-then-matmul reference of benchmark cfg 0 at 48x256x40.
* qk_norm_rope.npz -- the reference test's fp32 closed form ``ref_one``
  (test_parity_light.py:93-103) at B=1, L=16, H=4, D=128 with random bf16 tables.

Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
FP8 = torch.float8_e4m3fn
FP8_MAX = torch.finfo(FP8).max


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def u8(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint8).numpy()


def torch_quant(x: torch.Tensor, variant: str):
    absmax = x.abs().amax(dim=1, keepdim=True).float().clamp_min(1e-8)
    scale = absmax / FP8_MAX
    if variant == "div":
        v = x.float() / scale
    else:
        v = x.float() * (1.0 / scale)
    return v.clamp(-FP8_MAX, FP8_MAX).to(FP8), scale


def make_quant(name: str, x: torch.Tensor) -> None:
    qd, s = torch_quant(x, "div")
    qr, _ = torch_quant(x, "rcp")
    np.savez_compressed(os.path.join(HERE, name), x=u16(x), q_div=u8(qd), q_rcp=u8(qr),
                        s=s.reshape(-1).numpy())


def main() -> None:
    g = torch.Generator().manual_seed(0)
    # reference test geometry: M=67, row 0 zero
    x = torch.randn(67, 512, generator=g).to(torch.bfloat16)
    x[0].zero_()
    make_quant("quant_m67_zero_row.npz", x)
    # benchmark cfg 0 distribution: N(0,1), 0.5% of channels x20
    K = 1024
    x = torch.randn(32, K, generator=g)
    cols = torch.randperm(K, generator=g)[: max(1, K // 200)]
    x[:, cols] *= 20
    make_quant("quant_outliers.npz", x.to(torch.bfloat16))

    # small GEMM, cfg-0 distributions
    M, Kg, N = 48, 256, 40
    xa = torch.randn(M, Kg, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, Kg, generator=g) * 0.02).to(torch.bfloat16)
    bias = (torch.randn(N, generator=g) * 0.01).to(torch.bfloat16)
    qa, sa = torch_quant(xa, "div")
    qw, sw = torch_quant(w, "div")
    a = qa.float().double() * sa.double()
    b = qw.float().double() * sw.double()
    ref = (a @ b.t()).float() + bias.float()
    np.savez_compressed(os.path.join(HERE, "gemm_small.npz"), qa=u8(qa), sa=sa.reshape(-1).numpy(),
                        qw=u8(qw), sw=sw.reshape(-1).numpy(), bias=u16(bias), ref=ref.numpy())

    # qk norm + rope, reference test closed form
    B, L, H, D = 1, 16, 4, 128
    q = torch.randn(B, L * H, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, L * H, D, generator=g).to(torch.bfloat16)
    qw_ = torch.randn(D, generator=g).to(torch.bfloat16)
    kw_ = torch.randn(D, generator=g).to(torch.bfloat16)
    cos = torch.randn(L, D // 2, generator=g).to(torch.bfloat16)
    sin = torch.randn(L, D // 2, generator=g).to(torch.bfloat16)

    def ref_one(x, wt):
        xf = x.float().view(B, L, H, D)
        xn = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) * wt.float()
        c = cos.float().view(L, 1, D // 2)
        s = sin.float().view(L, 1, D // 2)
        x1, x2 = xn[..., 0::2], xn[..., 1::2]
        o = torch.empty_like(xn)
        o[..., 0::2] = x1 * c - x2 * s
        o[..., 1::2] = x1 * s + x2 * c
        return o.view(B, L * H, D)

    kf = k.float()
    k_pre = kf * torch.rsqrt(kf.pow(2).mean(-1, keepdim=True) + 1e-6) * kw_.float()
    np.savez_compressed(os.path.join(HERE, "qk_norm_rope.npz"), q=u16(q), k=u16(k), qw=u16(qw_),
                        kw=u16(kw_), cos=u16(cos), sin=u16(sin),
                        q_ref=ref_one(q, qw_).numpy(), k_ref=ref_one(k, kw_).numpy(),
                        k_pre_ref=k_pre.numpy())


if __name__ == "__main__":
    main()
