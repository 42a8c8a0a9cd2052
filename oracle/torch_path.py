"""The reference's CPU-runnable torch code path for the hot path, restated (torch, CPU).

TEST / BASELINE INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``. ``bench.py``
times these functions on the host cores as the reported CPU baseline.

* ``qkv_norm_rope_cache`` -- the reference's per-block sequence for one stream:
  ``rearrange(qkv, "B L (K H D) -> K B L H D")`` (``dit.py:409-411``), then the
  torch fallback of ``fused_qk_norm_rope_3d`` (``sgl_fused_ops.py:170-199``:
  fp32 RMSNorm, ``repeat_interleave`` tables, rotate-half, cast), with the
  pre-RoPE K kept (``return_k_pre_rope``) and V compacted for the cache
  (``dit.py:131-137,446-451``), written into a ring slot.
* ``fp8_linear`` -- ``_quantize_per_token_impl`` (``fp8_linear.py:38-43``) followed
  by fp32 dequantise-then-matmul + bias -> bf16, the BASELINE GEMM reference
  (row-wise ``torch._scaled_mm`` is not available on the CPU backend).
"""
from __future__ import annotations

import torch

FP8 = torch.float8_e4m3fn
FP8_MAX = torch.finfo(FP8).max


def _rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    out = xf * torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)
    return (out * w.float()).to(dtype=x.dtype)


def qkv_norm_rope_cache(qkv: torch.Tensor, num_heads: int, eps: float, q_weight, k_weight,
                        cos_half, sin_half, cache_k: torch.Tensor, cache_v: torch.Tensor, slot: int):
    """qkv [L, 3*H*D] bf16; cos/sin half tables [L, D/2]; cache [S, L, H, D]. Returns (q, k)."""
    L = qkv.shape[0]
    D = qkv.shape[1] // (3 * num_heads)
    q, k, v = qkv.view(L, 3, num_heads, D).unbind(1)
    qn = _rmsnorm(q, q_weight, eps)
    kn = _rmsnorm(k, k_weight, eps)
    cos = cos_half.repeat_interleave(2, dim=-1).reshape(L, 1, D).float()
    sin = sin_half.repeat_interleave(2, dim=-1).reshape(L, 1, D).float()

    def apply(x):
        xf = x.float()
        pairs = xf.reshape(*x.shape[:-1], -1, 2)
        rotated = torch.stack((-pairs[..., 1], pairs[..., 0]), dim=-1).flatten(-2)
        return (xf * cos + rotated * sin).to(dtype=x.dtype)

    q_out, k_out = apply(qn), apply(kn)
    cache_k[slot, :L].copy_(kn)
    cache_v[slot, :L].copy_(v.clone())
    return q_out, k_out


def quantize_per_token(x: torch.Tensor):
    absmax = x.abs().amax(dim=1, keepdim=True).float().clamp_min(1e-8)
    scale = absmax / FP8_MAX
    q = (x.float() / scale).clamp(-FP8_MAX, FP8_MAX).to(FP8)
    return q, scale


def fp8_linear(x: torch.Tensor, w_q: torch.Tensor, w_s: torch.Tensor, bias: torch.Tensor):
    """x [M, K] bf16; w_q [N, K] e4m3fn; w_s [N] fp32; bias [N] bf16 -> bf16 [M, N]."""
    q, s = quantize_per_token(x)
    a = q.float() * s
    b = w_q.float() * w_s.reshape(-1, 1)
    return (a @ b.t() + bias.float()).to(torch.bfloat16)
