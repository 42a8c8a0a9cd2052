"""FP8 linear layer on the gfx950 kernels -- counterpart of the reference's
``deploy/xvideo/models/dit/fp8_linear.py``.

Same API (``available``, ``backend``, ``Fp8Linear.from_linear``, ``forward``,
``_quantize_weight_per_channel``) and the same numerics contract:

* weights: per-output-channel e4m3fn with ``s_w = max(absmax, 1e-8) / 448`` and
  division (``fp8_linear.py:77-85``), stored as the (K, N) column-major view;
* activations: per-token e4m3fn rounded the way the reference's ROCm path
  rounds them (``_quantize_per_token_rocm``, ``fp8_linear.py:57-74``):
  reciprocal-multiply for K < 8192 (its native kernel,
  ``per_token_quant_fp8_rocm.hip:72-77``) and division for K >= 8192 (the
  compiled ``_quantize_per_token_impl``, ``fp8_linear.py:38-43``); one gfx950
  kernel serves both, bit-identical to either formula
  (``quant_rounding="division"`` forces division for every K);
* GEMM: ``y = bf16(fma(acc * s_w[n], s_x[m], bias[n]))`` (``fp8_gemm.cu:99-136``)
  in place of ``torch._scaled_mm`` (``fp8_linear.py:124-132``). An optional
  fused GELU-tanh epilogue serves the MLP up-projection (``dit.py:87-89,508-513``).

The reference picks torch._scaled_mm whenever ROCm is detected
(``fp8_linear.py:21,119``); this module always routes to joyomni_ops, which
reports ``has_fp8() == True``.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from . import (fp8_scaled_mm, fp8_scaled_mm_gated_residual, fp8_scaled_mm_gelu_tanh, has_fp8, has_quant,
               per_token_quant_fp8)

FP8_DTYPE = torch.float8_e4m3fn
FP8_MAX = torch.finfo(FP8_DTYPE).max


def available() -> bool:
    return bool(has_fp8() and has_quant())


def backend() -> str:
    return "joyomni_ops/gfx950-hip" if available() else "unavailable"


# The reference's ROCm quantiser switches from its reciprocal-multiply kernel to
# the compiled division formula at this K (fp8_linear.py:62).
ROCM_DIVISION_MIN_K = 8192


def exact_division_for(K: int, quant_rounding: str = "reference_rocm") -> bool:
    """Rounding of the activation quantiser for an input width K."""
    if quant_rounding == "division":
        return True
    if quant_rounding == "reciprocal":
        return False
    if quant_rounding == "reference_rocm":
        return K >= ROCM_DIVISION_MIN_K
    raise ValueError(f"unknown quant_rounding {quant_rounding!r}")


def quantize_per_token(x_2d: torch.Tensor, exact_division: bool = True):
    """x [M, K] bf16/fp16 (contiguous, on the GPU) -> (q e4m3fn [M, K], s fp32 [M, 1])."""
    q = torch.empty_like(x_2d, dtype=FP8_DTYPE)
    s = torch.empty((x_2d.shape[0], 1), device=x_2d.device, dtype=torch.float32)
    per_token_quant_fp8(x_2d, q, s, exact_division)
    return q, s


def _quantize_weight_per_channel(w_bf16: torch.Tensor):
    """W [N, K] bf16 -> (Wq as (K, N) with stride (1, K), s_w (1, N) fp32)."""
    w = w_bf16.to(torch.bfloat16).contiguous()
    N, K = w.shape
    wq, s = quantize_per_token(w, True)  # weights: division (fp8_linear.py:77-85)
    w_q_cm = wq.t()
    assert w_q_cm.shape == (K, N) and w_q_cm.stride() == (1, K)
    return w_q_cm, s.reshape(1, N).contiguous()


class Fp8Linear(nn.Module):
    def __init__(self, weight_fp8: torch.Tensor, weight_scale: torch.Tensor,
                 bias: Optional[torch.Tensor], out_dtype: torch.dtype = torch.bfloat16,
                 gelu_tanh: bool = False, quant_rounding: str = "reference_rocm"):
        super().__init__()
        self.register_buffer("weight_fp8", weight_fp8, persistent=False)
        self.register_buffer("weight_scale", weight_scale, persistent=False)
        if bias is not None:
            self.register_buffer("bias", bias.contiguous(), persistent=False)
        else:
            self.bias = None
        self.out_dtype = out_dtype
        self.gelu_tanh = gelu_tanh
        K, N = weight_fp8.shape
        self.in_features = K
        self.out_features = N
        self.exact_division = exact_division_for(K, quant_rounding)

    @classmethod
    def from_linear(cls, lin: nn.Linear, out_dtype: torch.dtype = torch.bfloat16,
                    gelu_tanh: bool = False, quant_rounding: str = "reference_rocm") -> "Fp8Linear":
        assert available(), "joyomni_ops fp8 ops not available; cannot build Fp8Linear"
        w_q, w_s = _quantize_weight_per_channel(lin.weight.data.to(torch.bfloat16))
        b = lin.bias.data.to(dtype=out_dtype) if lin.bias is not None else None
        return cls(w_q, w_s, b, out_dtype=out_dtype, gelu_tanh=gelu_tanh, quant_rounding=quant_rounding)

    def gemm(self, x_q: torch.Tensor, x_scale: torch.Tensor) -> torch.Tensor:
        """The GEMM (+ fused epilogue) on already quantised activations [M, K]."""
        mm = fp8_scaled_mm_gelu_tanh if self.gelu_tanh else fp8_scaled_mm
        return mm(x_q, self.weight_fp8, x_scale, self.weight_scale, self.out_dtype, self.bias)

    def gemm_gated_residual(self, x_q: torch.Tensor, x_scale: torch.Tensor, residual: torch.Tensor,
                            gate: torch.Tensor, inplace: bool = False) -> torch.Tensor:
        """residual + gemm(x_q, x_scale) * gate with the gated residual in the GEMM epilogue
        (the block's fused_add_gate, sgl_fused_ops.py:302-305); residual [M, N]."""
        assert not self.gelu_tanh, "the gated-residual epilogue has no GELU"
        assert residual.dtype == self.out_dtype, "residual dtype must be the output dtype"
        return fp8_scaled_mm_gated_residual(x_q, self.weight_fp8, x_scale, self.weight_scale, residual,
                                            gate, self.bias, inplace)

    def gated_residual(self, x: torch.Tensor, residual: torch.Tensor, gate: torch.Tensor,
                       inplace: bool = False) -> torch.Tensor:
        """residual + self(x) * gate: x [M, K] quantised per token, then one GEMM launch."""
        x_2d = x.reshape(-1, x.shape[-1]).contiguous()
        assert x_2d.shape[1] == self.in_features, f"in features mismatch {x_2d.shape[1]} vs {self.in_features}"
        x_q, x_scale = quantize_per_token(x_2d, self.exact_division)
        return self.gemm_gated_residual(x_q, x_scale, residual, gate, inplace)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        orig_shape = x.shape
        x_2d = x.reshape(-1, orig_shape[-1]).contiguous()
        M, K = x_2d.shape
        assert K == self.in_features, f"in features mismatch {K} vs {self.in_features}"
        x_q, x_scale = quantize_per_token(x_2d, self.exact_division)
        return self.gemm(x_q, x_scale).reshape(*orig_shape[:-1], self.out_features)
