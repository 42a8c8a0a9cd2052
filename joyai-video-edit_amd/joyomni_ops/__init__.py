"""joyomni_ops -- MI355X (gfx950) drop-in for the reference's operator package.

Same namespace, op schemas, FakeTensor registrations and Python wrappers as the
reference's ``joyomni_ops/joyomni_ops/__init__.py`` (schemas from
``joyomni_ops/csrc/pybind.cpp:52-75``), so ``torch.ops.joyomni_ops.*`` and
``from joyomni_ops import ...`` keep working for ``deploy/xvideo``.

The quantised hot path -- ``sgl_per_token_quant_fp8``, ``fp8_scaled_mm``,
``fused_qk_norm_rope_3d_paired``, the new ``fused_qkv_norm_rope_cache``, the
cache read side ``fused_joint_qkv_pack`` / ``fused_cached_kv_pack`` and the
adaLN ``fused_norm_scale_shift`` (plus its FP8-emitting variant) -- runs in
hand-written gfx950 kernels of ``libjoyomni_hip.so`` reached through its C ABI
(``include/joyomni_hip.h``). Importing fails when that library is missing,
exactly like the reference (``__init__.py:15-19``); nothing falls back.

``rmsnorm``, which the model never calls, keeps its reference schema as a
torch device composition, so the reference's imports
(``sgl_fused_ops.py:27-33``) still resolve.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional

import torch

from . import _lib

_LIB = _lib.load()  # raises ImportError when the HIP library is not built

__all__ = [
    "fused_qk_norm_rope_3d_paired",
    "fused_joint_qkv_pack",
    "fused_cached_kv_pack",
    "fused_norm_scale_shift",
    "rmsnorm",
    "sgl_per_token_quant_fp8",
    "fp8_scaled_mm",
    "has_quant",
    "has_fp8",
    # additions of this build
    "per_token_quant_fp8",
    "fp8_scaled_mm_gelu_tanh",
    "fused_qkv_norm_rope_cache",
    "fp8_qkv_norm_rope_cache",
    "fused_norm_scale_shift_fp8",
    "fp8_scaled_mm_gated_residual",
    "fused_cached_kv_pack_out",
    "fused_text_qkv_pack",
    "sdpa_attention",
    "sdpa_attention_out",
]

_NS = "joyomni_ops"
_lib_def = torch.library.Library(_NS, "DEF")

# --- reference schemas (pybind.cpp:52-75); one annotation added: the kernel writes k_pre_rope
# (fused_qknorm_rope_3d_kernel.cu:97-100), which the reference schema leaves undeclared, so under
# torch.compile functionalisation would not see that write. Declaring it mutable keeps every call
# site valid and makes the write visible. ---
_lib_def.define(
    "fused_qk_norm_rope_3d_paired(Tensor! q, Tensor! k, int seq_len, int num_heads, float eps, "
    "Tensor q_weight, Tensor k_weight, Tensor cos, Tensor sin, Tensor(a!)? k_pre_rope) -> ()")
_lib_def.define(
    "fused_joint_qkv_pack(Tensor img_q, Tensor img_k, Tensor img_v, "
    "Tensor txt_q, Tensor txt_k, Tensor txt_v, Tensor? cached_k, Tensor? cached_v, "
    "Tensor txt_q_weight, Tensor txt_k_weight, float eps) -> (Tensor, Tensor, Tensor)")
_lib_def.define(
    "fused_cached_kv_pack(Tensor key0, Tensor value0, Tensor? key1, Tensor? value1, "
    "Tensor cos, Tensor sin) -> (Tensor, Tensor)")
_lib_def.define(
    "fused_norm_scale_shift(Tensor x, Tensor? gamma_opt, Tensor? beta_opt, "
    "Tensor scale, Tensor shift, int norm_type, float eps) -> Tensor")
_lib_def.define("rmsnorm(Tensor x, Tensor weight, float eps) -> Tensor")
_lib_def.define("sgl_per_token_quant_fp8(Tensor input, Tensor! output_q, Tensor! output_s) -> ()")
_lib_def.define(
    "fp8_scaled_mm(Tensor mat_a, Tensor mat_b, Tensor scales_a, Tensor scales_b, "
    "ScalarType out_dtype, Tensor? bias) -> Tensor")

# --- additions of this build ---
_lib_def.define(
    "per_token_quant_fp8(Tensor input, Tensor! output_q, Tensor! output_s, bool exact_division) -> ()")
_lib_def.define(
    "fp8_scaled_mm_gelu_tanh(Tensor mat_a, Tensor mat_b, Tensor scales_a, Tensor scales_b, "
    "ScalarType out_dtype, Tensor? bias) -> Tensor")
_lib_def.define(
    "fp8_scaled_mm_gated_residual(Tensor mat_a, Tensor mat_b, Tensor scales_a, Tensor scales_b, "
    "Tensor residual, Tensor gate, Tensor? bias) -> Tensor")
_lib_def.define(
    "fp8_scaled_mm_gated_residual_(Tensor mat_a, Tensor mat_b, Tensor scales_a, Tensor scales_b, "
    "Tensor(a!) residual, Tensor gate, Tensor? bias) -> ()")
_lib_def.define(
    "fused_norm_scale_shift_fp8(Tensor x, Tensor? gamma_opt, Tensor? beta_opt, Tensor scale, "
    "Tensor shift, int norm_type, float eps, Tensor(a!) output_q, Tensor(b!) output_s, "
    "Tensor(c!)? out, bool exact_division) -> ()")
_lib_def.define(
    "fused_qkv_norm_rope_cache(Tensor qkv, int num_heads, float eps, Tensor q_weight, "
    "Tensor k_weight, Tensor cos, Tensor sin, Tensor(a!)? q_out, Tensor(b!)? k_out, "
    "Tensor(c!)? cache_k, Tensor(d!)? cache_v, int slot, int slot_offset, Tensor(e!)? v_out=None, "
    "int cache_tokens=-1, bool cache_pre_rope=True) -> ()")
_lib_def.define(
    "fp8_qkv_norm_rope_cache(Tensor mat_a, Tensor mat_b, Tensor scales_a, Tensor scales_b, Tensor? bias, "
    "int num_heads, float eps, Tensor q_weight, Tensor k_weight, Tensor cos, Tensor sin, Tensor(a!)? q_out, "
    "Tensor(b!)? k_out, Tensor(c!)? cache_k, Tensor(d!)? cache_v, int slot, int slot_offset, "
    "Tensor(e!)? v_out=None, int cache_tokens=-1, bool cache_pre_rope=True) -> ()")
_lib_def.define(
    "fused_cached_kv_pack_out(Tensor key0, Tensor value0, Tensor? key1, Tensor? value1, "
    "Tensor cos, Tensor sin, Tensor(a!) out_k, Tensor(b!) out_v) -> ()")
_lib_def.define(
    "fused_text_qkv_pack(Tensor txt_q, Tensor txt_k, Tensor txt_v, Tensor txt_q_weight, "
    "Tensor txt_k_weight, float eps, Tensor(a!) out_q, Tensor(b!) out_k, Tensor(c!) out_v) -> ()")

_lib_def.define("sdpa_attention(Tensor query, Tensor key, Tensor value, float? scale=None) -> Tensor")
_lib_def.define(
    "sdpa_attention_out(Tensor query, Tensor key, Tensor value, Tensor(a!) out, float? scale=None) -> ()")

_ops = torch.ops.joyomni_ops


# --------------------------------------------------------------------------
# argument checks, worded like the reference's TORCH_CHECKs (joyomni_ops.h:8-15)
# --------------------------------------------------------------------------
def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _check_input(t: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    _check(t.is_cuda, f"{name} must be a CUDA tensor")
    _check(t.is_contiguous(), f"{name} must be contiguous")
    _check(t.dtype == dtype, f"{name} dtype is {t.dtype}, expected {dtype}")


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


_OUT_CODE = {torch.bfloat16: _lib.JOY_DTYPE_BF16, torch.float16: _lib.JOY_DTYPE_FP16}


# --------------------------------------------------------------------------
# quantiser
# --------------------------------------------------------------------------
def _quant_impl(input, output_q, output_s, rounding):
    for name, t in (("input", input), ("output_q", output_q), ("output_s", output_s)):
        _check(t.is_cuda, f"{name} must be a CUDA tensor")
        _check(t.is_contiguous(), f"{name} must be contiguous")
    _check(input.dim() == 2, "input must be [M, K]")
    _check(output_q.shape == input.shape, "output_q shape must match input")
    _check(output_q.dtype == torch.float8_e4m3fn, "output_q must be torch.float8_e4m3fn")
    _check(output_s.dtype == torch.float32, "output_s must be float32")
    _check(output_s.numel() == input.size(0), "output_s must contain one scale per row")
    _check(input.device == output_q.device and input.device == output_s.device,
           "input and outputs must be on the same device")
    _check(input.dtype in (torch.bfloat16, torch.float16), "input must be bfloat16 or float16")
    M, K = input.shape
    with torch.cuda.device(input.device):
        st = _LIB.joy_per_token_quant_fp8(
            _ptr(input), _OUT_CODE[input.dtype], _ptr(output_q), _ptr(output_s), M, K, rounding,
            _stream(input))
    _lib.check(_LIB, st)


@torch.library.impl(_lib_def, "sgl_per_token_quant_fp8", "CUDA")
def _sgl_per_token_quant_fp8_cuda(input, output_q, output_s):
    # The reference's gfx950 kernel rounds by reciprocal multiply
    # (per_token_quant_fp8_rocm.hip:72-77); keep that contract for this op.
    _quant_impl(input, output_q, output_s, _lib.JOY_QUANT_RECIPROCAL)


@torch.library.impl(_lib_def, "per_token_quant_fp8", "CUDA")
def _per_token_quant_fp8_cuda(input, output_q, output_s, exact_division):
    _quant_impl(input, output_q, output_s,
                _lib.JOY_QUANT_DIVIDE if exact_division else _lib.JOY_QUANT_RECIPROCAL)


# --------------------------------------------------------------------------
# GEMM
# --------------------------------------------------------------------------
def _scaled_mm_checks(mat_a, mat_b, scales_a, scales_b, out_dtype, bias):
    # checks of fp8_gemm.cu:1457-1487
    _check(mat_a.is_cuda, "mat_a must be a CUDA tensor")
    _check(mat_b.is_cuda, "mat_b must be a CUDA tensor")
    _check(mat_a.dim() == 2, "mat_a must be a 2D tensor")
    _check(mat_b.dim() == 2, "mat_b must be a 2D tensor")
    _check(mat_a.stride(1) == 1, "mat_a must be a row major tensor")
    _check(mat_b.stride(0) == 1, "mat_b must be a column major tensor")
    _check(mat_a.size(1) == mat_b.size(0), "mat_a and mat_b shapes cannot be multiplied")
    _check((mat_a.size(1) * mat_a.element_size()) % 16 == 0,
           "mat_a must be multiple of 16 bytes for memory alignment")
    _check((mat_b.size(0) * mat_b.element_size()) % 16 == 0,
           "mat_b must be multiple of 16 bytes for memory alignment")
    _check(mat_a.dtype == torch.float8_e4m3fn, "mat_a must be Float8_e4m3fn")
    _check(mat_b.dtype == torch.float8_e4m3fn, "mat_b must be Float8_e4m3fn")
    _check(out_dtype in (torch.float16, torch.bfloat16), "out_dtype must be Half or BFloat16")
    _check(scales_a.numel() == mat_a.size(0), "size of scales_a is not matched")
    _check(scales_b.numel() == mat_b.size(1), "size of scales_b is not matched")
    _check(scales_a.is_contiguous(), "scales_a must be contiguous")
    _check(scales_b.is_contiguous(), "scales_b msut be contiguous")
    _check(scales_a.dtype == torch.float32, "scales_a must be Float32")
    _check(scales_b.dtype == torch.float32, "scales_b must be Float32")
    if bias is not None:
        _check(bias.numel() == mat_b.size(1), "size of bias is not matched")
        _check(bias.is_contiguous(), "bias must be contiguous")
        _check(bias.dtype == out_dtype, "bias dtype must match output dtype")
    M, K = mat_a.shape
    N = mat_b.size(1)
    # Row stride of A and column stride of B must be K (dense rows).
    _check(M <= 1 or mat_a.stride(0) == K, "mat_a rows must be dense (stride(0) == K)")
    _check(N <= 1 or mat_b.stride(1) == K, "mat_b columns must be dense (stride(1) == K)")
    _check((N * torch.empty((), dtype=out_dtype).element_size()) % 16 == 0,
           "out must be multiple of 16 bytes for memory alignment")
    return M, N, K


def _gemm_workspace(M, N, K, device):
    """Split-K workspace of the small-M GEMM plans (None when the shape uses none); allocated
    from torch's caching allocator like the output, so a captured graph keeps its own."""
    nbytes = _LIB.joy_fp8_scaled_mm_workspace_size(M, N, K)
    if nbytes <= 0:
        return None, 0
    return torch.empty(nbytes, dtype=torch.uint8, device=device), nbytes


def _scaled_mm_impl(mat_a, mat_b, scales_a, scales_b, out_dtype, bias, epilogue):
    M, N, K = _scaled_mm_checks(mat_a, mat_b, scales_a, scales_b, out_dtype, bias)
    out = torch.empty((M, N), device=mat_a.device, dtype=out_dtype)
    with torch.cuda.device(mat_a.device):
        ws, ws_bytes = _gemm_workspace(M, N, K, mat_a.device)
        st = _LIB.joy_fp8_scaled_mm(
            _ptr(mat_a), _ptr(mat_b), _ptr(scales_a), _ptr(scales_b), _ptr(bias), _ptr(out),
            _OUT_CODE[out_dtype], M, N, K, epilogue, _ptr(ws), ws_bytes, _stream(mat_a))
    _lib.check(_LIB, st)
    return out


@torch.library.impl(_lib_def, "fp8_scaled_mm", "CUDA")
def _fp8_scaled_mm_cuda(mat_a, mat_b, scales_a, scales_b, out_dtype, bias=None):
    return _scaled_mm_impl(mat_a, mat_b, scales_a, scales_b, out_dtype, bias, _lib.JOY_EPILOGUE_NONE)


@torch.library.impl(_lib_def, "fp8_scaled_mm_gelu_tanh", "CUDA")
def _fp8_scaled_mm_gelu_cuda(mat_a, mat_b, scales_a, scales_b, out_dtype, bias=None):
    return _scaled_mm_impl(mat_a, mat_b, scales_a, scales_b, out_dtype, bias,
                           _lib.JOY_EPILOGUE_GELU_TANH)


def _gated_residual_impl(mat_a, mat_b, scales_a, scales_b, residual, gate, bias, out):
    """out = residual + fp8_scaled_mm(...) * gate (fused_add_gate, sgl_fused_ops.py:302-305)."""
    out_dtype = residual.dtype
    _check(out_dtype in (torch.float16, torch.bfloat16), "residual must be Half or BFloat16")
    M, N, K = _scaled_mm_checks(mat_a, mat_b, scales_a, scales_b, out_dtype, bias)
    _check(residual.is_cuda and gate.is_cuda, "residual and gate must be CUDA tensors")
    _check(residual.dim() == 2 and tuple(residual.shape) == (M, N), "residual must be [M, N]")
    _check(residual.stride(1) == 1 or N <= 1, "residual rows must be contiguous")
    _check(gate.numel() == N, "size of gate is not matched")
    _check(gate.dtype == out_dtype, "gate dtype must match residual dtype")
    gate = gate.reshape(N)
    if gate.stride(0) != 1 or gate.data_ptr() % 16:
        gate = gate.clone(memory_format=torch.contiguous_format)  # N values: a 16-byte aligned copy
    ld = residual.stride(0) if M > 1 else N
    with torch.cuda.device(mat_a.device):
        ws, ws_bytes = _gemm_workspace(M, N, K, mat_a.device)
        st = _LIB.joy_fp8_scaled_mm_gated_residual(
            _ptr(mat_a), _ptr(mat_b), _ptr(scales_a), _ptr(scales_b), _ptr(bias), _ptr(residual), ld,
            _ptr(gate), _ptr(out), _OUT_CODE[out_dtype], M, N, K, _ptr(ws), ws_bytes, _stream(mat_a))
    _lib.check(_LIB, st)


@torch.library.impl(_lib_def, "fp8_scaled_mm_gated_residual", "CUDA")
def _fp8_scaled_mm_gated_residual_cuda(mat_a, mat_b, scales_a, scales_b, residual, gate, bias=None):
    out = torch.empty(residual.shape, device=residual.device, dtype=residual.dtype)
    _gated_residual_impl(mat_a, mat_b, scales_a, scales_b, residual, gate, bias, out)
    return out


@torch.library.impl(_lib_def, "fp8_scaled_mm_gated_residual_", "CUDA")
def _fp8_scaled_mm_gated_residual_inplace_cuda(mat_a, mat_b, scales_a, scales_b, residual, gate, bias=None):
    _check(residual.is_contiguous(), "an in-place residual must be contiguous")
    _gated_residual_impl(mat_a, mat_b, scales_a, scales_b, residual, gate, bias, residual)


# --------------------------------------------------------------------------
# q/k RMSNorm + RoPE
# --------------------------------------------------------------------------
@torch.library.impl(_lib_def, "fused_qk_norm_rope_3d_paired", "CUDA")
def _fused_qk_norm_rope_3d_paired_cuda(q, k, seq_len, num_heads, eps, q_weight, k_weight, cos,
                                       sin, k_pre_rope=None):
    # checks of fused_qknorm_rope_3d_kernel.cu:285-310
    _check(q.dim() == 3, "q must be 3D [batch, seq_len*num_heads, head_dim]")
    _check(k.dim() == 3, "k must be 3D [batch, seq_len*num_heads, head_dim]")
    _check(q.shape == k.shape, "q and k must have the same shape")
    _check(q_weight.dim() == 1 and k_weight.dim() == 1, "weights must be 1D [head_dim]")
    _check(cos.dim() == 2 and sin.dim() == 2, "cos/sin must be 2D [seq_len, head_dim/2]")
    for name, t in (("q", q), ("k", k), ("q_weight", q_weight), ("k_weight", k_weight),
                    ("cos", cos), ("sin", sin)):
        _check_input(t, name, torch.bfloat16)
    batch, _, head_dim = q.shape
    _check(q.size(1) == seq_len * num_heads, "q.size(1) must equal seq_len*num_heads")
    _check(q_weight.size(0) == head_dim and k_weight.size(0) == head_dim,
           "weight size must match head_dim")
    _check(cos.size(0) == seq_len and cos.size(1) == head_dim // 2,
           "cos shape must be [seq_len, head_dim/2]")
    _check(sin.size(0) == seq_len and sin.size(1) == head_dim // 2,
           "sin shape must be [seq_len, head_dim/2]")
    if k_pre_rope is not None:
        _check(k_pre_rope.shape == k.shape, "k_pre_rope must have the same shape as k")
        _check_input(k_pre_rope, "k_pre_rope", torch.bfloat16)
    with torch.cuda.device(q.device):
        st = _LIB.joy_fused_qk_norm_rope_3d_paired(
            _ptr(q), _ptr(k), batch, seq_len, num_heads, head_dim, float(eps), _ptr(q_weight),
            _ptr(k_weight), _ptr(cos), _ptr(sin), _ptr(k_pre_rope), _stream(q))
    _lib.check(_LIB, st)


def _token_stride(t: torch.Tensor, L: int, H: int, D: int, name: str, device) -> int:
    """Token stride of an output view of L tokens: [L, H, D], [1, L, H, D] or [L, H*D], dense heads.

    The kernel writes exactly L token rows through this stride, so a view with another
    token count (a short or mis-sliced output) is rejected before anything is launched."""
    _check(t.is_cuda and t.device == device, f"{name} must be a CUDA tensor on the device of qkv")
    _check(t.dtype == torch.bfloat16, f"{name} must be a bf16 CUDA tensor")
    x = t
    if x.dim() == 4:
        _check(x.size(0) == 1, f"{name} batch must be 1")
        x = x[0]
    if x.dim() == 2:
        _check(x.size(1) == H * D and x.stride(1) == 1, f"{name} must have dense rows of H*D")
    else:
        _check(x.dim() == 3 and x.size(1) == H and x.size(2) == D, f"{name} must be [L, H, D]")
        _check(x.stride(2) == 1 and x.stride(1) == D, f"{name} must have dense heads")
    _check(x.size(0) == L, f"{name} holds {x.size(0)} tokens, expected {L} (the rows of qkv)")
    return x.stride(0) if L > 1 else H * D


def _norm_rope_out_checks(L, H, D, device, q_weight, k_weight, cos, sin, q_out, k_out, cache_k, cache_v, v_out,
                          cache_tokens):
    """Checks of the norm/RoPE/ring outputs shared by fused_qkv_norm_rope_cache and
    fp8_qkv_norm_rope_cache; returns (token strides of q_out, k_out, v_out, ring slots, slot
    capacity, cached tokens)."""
    for name, t in (("q_weight", q_weight), ("k_weight", k_weight), ("cos", cos), ("sin", sin)):
        _check_input(t, name, torch.bfloat16)
        _check(t.device == device, f"{name} must be on the device of qkv")
    _check(q_weight.numel() == D and k_weight.numel() == D, "weight size must match head_dim")
    _check(cos.shape == (L, D // 2) and sin.shape == (L, D // 2),
           "cos/sin shape must be [seq_len, head_dim/2]")
    strides = [_token_stride(t, L, H, D, name, device) if t is not None else 0
               for name, t in (("q_out", q_out), ("k_out", k_out), ("v_out", v_out))]
    n_slots = cap = 0
    if (cache_k is None) != (cache_v is None):
        raise RuntimeError("cache_k and cache_v must be provided together")
    n_cache = L if cache_tokens is None or int(cache_tokens) < 0 else int(cache_tokens)
    if cache_k is not None:
        for name, t in (("cache_k", cache_k), ("cache_v", cache_v)):
            _check(t.is_cuda and t.device == device and t.dtype == torch.bfloat16,
                   f"{name} must be a bf16 CUDA tensor on the device of qkv")
        _check(cache_k.is_contiguous() and cache_v.is_contiguous(), "cache_k/cache_v must be contiguous")
        _check(cache_k.dim() == 4 and cache_k.shape == cache_v.shape
               and cache_k.shape[2:] == (H, D), "cache must be [num_slots, capacity, H, D]")
        n_slots, cap = cache_k.shape[0], cache_k.shape[1]
    return strides, n_slots, cap, n_cache


@torch.library.impl(_lib_def, "fused_qkv_norm_rope_cache", "CUDA")
def _fused_qkv_norm_rope_cache_cuda(qkv, num_heads, eps, q_weight, k_weight, cos, sin, q_out,
                                    k_out, cache_k, cache_v, slot, slot_offset, v_out=None, cache_tokens=-1,
                                    cache_pre_rope=True):
    _check(qkv.is_cuda, "qkv must be a CUDA tensor")
    _check(qkv.dtype == torch.bfloat16, f"qkv dtype is {qkv.dtype}, expected torch.bfloat16")
    x = qkv[0] if qkv.dim() == 3 else qkv
    _check(qkv.dim() in (2, 3) and (qkv.dim() == 2 or qkv.size(0) == 1),
           "qkv must be [L, 3*H*D] or [1, L, 3*H*D]")
    _check(x.stride(-1) == 1, "qkv rows must be contiguous")
    L, E3 = x.shape
    H = int(num_heads)
    _check(H > 0 and E3 % (3 * H) == 0, "qkv width must be 3*num_heads*head_dim")
    D = E3 // (3 * H)
    strides, n_slots, cap, n_cache = _norm_rope_out_checks(L, H, D, qkv.device, q_weight, k_weight, cos, sin, q_out,
                                                           k_out, cache_k, cache_v, v_out, cache_tokens)
    with torch.cuda.device(qkv.device):
        st = _LIB.joy_fused_qkv_norm_rope_cache(
            _ptr(x), x.stride(0) if L > 1 else E3, L, H, D, float(eps), _ptr(q_weight), _ptr(k_weight), _ptr(cos),
            _ptr(sin), _ptr(q_out), strides[0], _ptr(k_out), strides[1], _ptr(v_out), strides[2], _ptr(cache_k),
            _ptr(cache_v), n_slots, cap, int(slot), int(slot_offset), n_cache, 0 if cache_pre_rope else 1,
            _stream(qkv))
    _lib.check(_LIB, st)


@torch.library.impl(_lib_def, "fp8_qkv_norm_rope_cache", "CUDA")
def _fp8_qkv_norm_rope_cache_cuda(mat_a, mat_b, scales_a, scales_b, bias, num_heads, eps, q_weight, k_weight, cos,
                                  sin, q_out, k_out, cache_k, cache_v, slot, slot_offset, v_out=None,
                                  cache_tokens=-1, cache_pre_rope=True):
    M, N, K = _scaled_mm_checks(mat_a, mat_b, scales_a, scales_b, torch.bfloat16, bias)
    H = int(num_heads)
    _check(H > 0 and N % (3 * H) == 0, "mat_b width must be 3*num_heads*head_dim")
    D = N // (3 * H)
    strides, n_slots, cap, n_cache = _norm_rope_out_checks(M, H, D, mat_a.device, q_weight, k_weight, cos, sin,
                                                           q_out, k_out, cache_k, cache_v, v_out, cache_tokens)
    # the fused epilogue reads the tables 16 bytes at a time: an aligned copy of a misaligned view
    cos = cos if cos.data_ptr() % 16 == 0 else cos.clone()
    sin = sin if sin.data_ptr() % 16 == 0 else sin.clone()
    with torch.cuda.device(mat_a.device):
        nbytes = _LIB.joy_fp8_qkv_norm_rope_cache_scratch_size(M, K, H, D)
        # outputs whose byte offsets pass 2^31 take the unfused path, through an [M, N] bf16 buffer
        if any(t is not None and (M * st_ + H * D) * 2 > 0x7FFFFFFF
               for t, st_ in ((q_out, strides[0]), (k_out, strides[1]), (v_out, strides[2]))):
            nbytes = M * N * 2
        # the tiles that do not take the fused epilogue pass through this [M, N] bf16 buffer
        scratch = torch.empty(nbytes, dtype=torch.uint8, device=mat_a.device) if nbytes > 0 else None
        st = _LIB.joy_fp8_qkv_norm_rope_cache(
            _ptr(mat_a), _ptr(mat_b), _ptr(scales_a), _ptr(scales_b), _ptr(bias), M, K, H, D, float(eps),
            _ptr(q_weight), _ptr(k_weight), _ptr(cos), _ptr(sin), _ptr(q_out), strides[0], _ptr(k_out), strides[1],
            _ptr(v_out), strides[2], _ptr(cache_k), _ptr(cache_v), n_slots, cap, int(slot), int(slot_offset), n_cache,
            0 if cache_pre_rope else 1, _ptr(scratch), nbytes, _stream(mat_a))
    _lib.check(_LIB, st)


# --------------------------------------------------------------------------
# cache read side: joint Q/K/V pack and cached-K rotation (HIP kernels)
# --------------------------------------------------------------------------
def _check_qkv_tensor(t, name, batch, heads, head_dim):
    # check_qkv_tensor of fused_joint_qkv_pack.cu:222-229
    _check(t.is_cuda, f"{name} must be a CUDA tensor")
    _check(t.dtype == torch.bfloat16, f"{name} must be bfloat16")
    _check(t.dim() == 4, f"{name} must be [B,L,H,D]")
    _check(t.size(0) == batch and t.size(2) == heads and t.size(3) == head_dim,
           f"{name} has incompatible shape {list(t.shape)}")
    _check(t.stride(3) == 1, f"{name} last dimension must be contiguous")


def _view(t: Optional[torch.Tensor]):
    """joy_bf16_view of a [1, L, H, D] tensor (None -> NULL)."""
    if t is None:
        return None
    return _lib.Bf16View(t.data_ptr(), t.size(1), t.stride(1), t.stride(2))


def _vref(v):
    return None if v is None else ctypes.byref(v)


# --------------------------------------------------------------------------
# attention core
# --------------------------------------------------------------------------
def _attention_checks(query, key, value, out):
    for name, t in (("query", query), ("key", key), ("value", value), ("out", out)):
        _check(t.is_cuda, f"{name} must be a CUDA tensor")
        _check(t.dim() == 4, f"{name} must be [B, S, H, D]")
        _check(t.dtype == torch.bfloat16, f"{name} must be bfloat16")
        _check(t.stride(3) == 1 or t.size(3) <= 1, f"{name} last dimension must be contiguous")
    B, Lq, H, D = query.shape
    _check(key.shape == value.shape, "key and value must have the same shape")
    _check(key.size(0) == B and key.size(2) == H and key.size(3) == D,
           "query, key and value must agree in batch, heads and head_dim")
    _check(tuple(out.shape) == (B, Lq, H, D), "out must have the shape of query")
    _check(out.stride(2) == D, "out heads must be dense (stride(2) == head_dim)")
    return B, Lq, H, D


def _attention_impl(query, key, value, out, scale):
    B, Lq, H, D = _attention_checks(query, key, value, out)
    sc = float(scale) if scale is not None else 1.0 / math.sqrt(D)
    with torch.cuda.device(query.device):
        for b in range(B):
            qv, kv, vv = _view(query[b:b + 1]), _view(key[b:b + 1]), _view(value[b:b + 1])
            st = _LIB.joy_attention_fwd(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv),
                                        out[b].data_ptr(), out.stride(1), H, D, sc, _stream(query))
            _lib.check(_LIB, st)


@torch.library.impl(_lib_def, "sdpa_attention", "CUDA")
def _sdpa_attention_cuda(query, key, value, scale=None):
    out = torch.empty(query.shape, device=query.device, dtype=query.dtype)
    _attention_impl(query, key, value, out, scale)
    return out


@torch.library.impl(_lib_def, "sdpa_attention_out", "CUDA")
def _sdpa_attention_out_cuda(query, key, value, out, scale=None):
    _attention_impl(query, key, value, out, scale)


@torch.library.impl(_lib_def, "fused_joint_qkv_pack", "CUDA")
def _fused_joint_qkv_pack_cuda(img_q, img_k, img_v, txt_q, txt_k, txt_v, cached_k, cached_v,
                               txt_q_weight, txt_k_weight, eps):
    # checks of fused_joint_qkv_pack.cu:244-284
    _check(img_q.dim() == 4, "img_q must be [B,L,H,D]")
    batch, img_len, heads, head_dim = img_q.shape
    _check(batch == 1, "fused_joint_qkv_pack fast path requires batch=1")
    _check(head_dim == 128, "fused_joint_qkv_pack requires head_dim=128")
    _check(img_len > 0 and heads > 0, "image length and heads must be positive")
    for name, t in (("img_q", img_q), ("img_k", img_k), ("img_v", img_v)):
        _check_qkv_tensor(t, name, batch, heads, head_dim)
    _check(img_k.size(1) == img_len and img_v.size(1) == img_len, "image Q/K/V lengths must match")
    txt_len = txt_q.size(1) if txt_q.dim() == 4 else 0
    for name, t in (("txt_q", txt_q), ("txt_k", txt_k), ("txt_v", txt_v)):
        _check_qkv_tensor(t, name, batch, heads, head_dim)
    _check(txt_len > 0 and txt_k.size(1) == txt_len and txt_v.size(1) == txt_len,
           "text Q/K/V lengths must match and be positive")
    for name, t in (("txt_q_weight", txt_q_weight), ("txt_k_weight", txt_k_weight)):
        _check_input(t, name, torch.bfloat16)
    _check(txt_q_weight.dim() == 1 and txt_q_weight.numel() == head_dim, "txt_q_weight must be [head_dim]")
    _check(txt_k_weight.dim() == 1 and txt_k_weight.numel() == head_dim, "txt_k_weight must be [head_dim]")
    _check((cached_k is None) == (cached_v is None),
           "cached_k and cached_v must either both be present or both be absent")
    cache_len = 0
    if cached_k is not None:
        _check_qkv_tensor(cached_k, "cached_k", batch, heads, head_dim)
        _check_qkv_tensor(cached_v, "cached_v", batch, heads, head_dim)
        cache_len = cached_k.size(1)
        _check(cached_v.size(1) == cache_len, "cached K/V lengths must match")
    out_q = img_q.new_empty((batch, img_len + txt_len, heads, head_dim))
    out_k = img_q.new_empty((batch, cache_len + img_len + txt_len, heads, head_dim))
    out_v = torch.empty_like(out_k)
    views = [_view(t) for t in (img_q, img_k, img_v, txt_q, txt_k, txt_v, cached_k, cached_v)]
    with torch.cuda.device(img_q.device):
        st = _LIB.joy_fused_joint_qkv_pack(
            *[_vref(v) for v in views], _ptr(txt_q_weight), _ptr(txt_k_weight), float(eps), heads,
            head_dim, _ptr(out_q), _ptr(out_k), _ptr(out_v), _stream(img_q))
    _lib.check(_LIB, st)
    return out_q, out_k, out_v


def _cached_pack_checks(key0, value0, key1, value1, cos, sin):
    # checks of fused_joint_qkv_pack.cu:351-381
    _check(key0.dim() == 4, "key0 must be [B,L,H,D]")
    batch, len0, heads, head_dim = key0.shape
    _check(batch == 1, "fused_cached_kv_pack requires batch=1")
    _check(head_dim == 128, "fused_cached_kv_pack requires head_dim=128")
    _check(len0 > 0 and heads > 0, "cache length and heads must be positive")
    _check_qkv_tensor(key0, "key0", batch, heads, head_dim)
    _check_qkv_tensor(value0, "value0", batch, heads, head_dim)
    _check(value0.size(1) == len0, "key0/value0 lengths must match")
    _check((key1 is None) == (value1 is None),
           "key1 and value1 must either both be present or both be absent")
    len1 = 0
    if key1 is not None:
        _check_qkv_tensor(key1, "key1", batch, heads, head_dim)
        _check_qkv_tensor(value1, "value1", batch, heads, head_dim)
        len1 = key1.size(1)
        _check(len1 > 0 and value1.size(1) == len1, "key1/value1 lengths must match and be positive")
    _check_input(cos, "cos", torch.float32)
    _check_input(sin, "sin", torch.float32)
    _check(cos.shape == sin.shape, "cos/sin shapes must match")
    _check(cos.numel() == (len0 + len1) * head_dim,
           f"cos/sin must contain [total_cache_len, head_dim], got {list(cos.shape)}")
    return len0 + len1, heads, head_dim


def _cached_pack_launch(key0, value0, key1, value1, cos, sin, heads, head_dim, out_k, out_v):
    views = [_view(t) for t in (key0, value0, key1, value1)]
    with torch.cuda.device(key0.device):
        st = _LIB.joy_fused_cached_kv_pack(
            *[_vref(v) for v in views], _ptr(cos), _ptr(sin), heads, head_dim, _ptr(out_k), _ptr(out_v),
            _stream(key0))
    _lib.check(_LIB, st)


@torch.library.impl(_lib_def, "fused_cached_kv_pack", "CUDA")
def _fused_cached_kv_pack_cuda(key0, value0, key1, value1, cos, sin):
    total, heads, head_dim = _cached_pack_checks(key0, value0, key1, value1, cos, sin)
    out_k = key0.new_empty((1, total, heads, head_dim))
    out_v = torch.empty_like(out_k)
    _cached_pack_launch(key0, value0, key1, value1, cos, sin, heads, head_dim, out_k, out_v)
    return out_k, out_v


def _check_dense_out(t, name, length, heads, head_dim):
    """A caller-provided pack output: bf16 CUDA [1, length, H, D] (or [length, H, D]), contiguous."""
    _check(t.is_cuda and t.dtype == torch.bfloat16, f"{name} must be a bf16 CUDA tensor")
    _check(t.is_contiguous(), f"{name} must be contiguous")
    x = t[0] if t.dim() == 4 else t
    _check((t.dim() == 3 or t.size(0) == 1) and tuple(x.shape) == (length, heads, head_dim),
           f"{name} must be [1, {length}, {heads}, {head_dim}], got {list(t.shape)}")


@torch.library.impl(_lib_def, "fused_cached_kv_pack_out", "CUDA")
def _fused_cached_kv_pack_out_cuda(key0, value0, key1, value1, cos, sin, out_k, out_v):
    total, heads, head_dim = _cached_pack_checks(key0, value0, key1, value1, cos, sin)
    _check_dense_out(out_k, "out_k", total, heads, head_dim)
    _check_dense_out(out_v, "out_v", total, heads, head_dim)
    _cached_pack_launch(key0, value0, key1, value1, cos, sin, heads, head_dim, out_k, out_v)


@torch.library.impl(_lib_def, "fused_text_qkv_pack", "CUDA")
def _fused_text_qkv_pack_cuda(txt_q, txt_k, txt_v, txt_q_weight, txt_k_weight, eps, out_q, out_k, out_v):
    _check(txt_q.dim() == 4, "txt_q must be [B,L,H,D]")
    batch, txt_len, heads, head_dim = txt_q.shape
    _check(batch == 1, "fused_text_qkv_pack requires batch=1")
    _check(head_dim == 128, "fused_text_qkv_pack requires head_dim=128")
    for name, t in (("txt_q", txt_q), ("txt_k", txt_k), ("txt_v", txt_v)):
        _check_qkv_tensor(t, name, batch, heads, head_dim)
    _check(txt_len > 0 and heads > 0 and txt_k.size(1) == txt_len and txt_v.size(1) == txt_len,
           "text Q/K/V lengths must match and be positive")
    for name, t in (("txt_q_weight", txt_q_weight), ("txt_k_weight", txt_k_weight)):
        _check_input(t, name, torch.bfloat16)
        _check(t.dim() == 1 and t.numel() == head_dim, f"{name} must be [head_dim]")
    for name, t in (("out_q", out_q), ("out_k", out_k), ("out_v", out_v)):
        _check_dense_out(t, name, txt_len, heads, head_dim)
    views = [_view(t) for t in (txt_q, txt_k, txt_v)]
    with torch.cuda.device(txt_q.device):
        st = _LIB.joy_fused_text_qkv_pack(
            *[_vref(v) for v in views], _ptr(txt_q_weight), _ptr(txt_k_weight), float(eps), heads, head_dim,
            _ptr(out_q), _ptr(out_k), _ptr(out_v), _stream(txt_q))
    _lib.check(_LIB, st)


# --------------------------------------------------------------------------
# adaLN norm + modulation (HIP), plain and FP8-emitting
# --------------------------------------------------------------------------
_NORM_DTYPE = {torch.bfloat16: _lib.JOY_DTYPE_BF16, torch.float16: _lib.JOY_DTYPE_FP16,
               torch.float32: _lib.JOY_DTYPE_FP32}


def _norm_args(x, gamma_opt, beta_opt, scale, shift, norm_type):
    # checks of fused_norm_scale_shift.cu:240-262
    _check(x.is_cuda, "x must be a CUDA tensor")
    _check(scale.is_cuda, "scale must be a CUDA tensor")
    _check(shift.is_cuda, "shift must be a CUDA tensor")
    _check(x.dim() == 2, "x must be 2D [M, N]")
    _check(x.stride(-1) == 1, "x last dim must be contiguous")
    M, N = x.shape
    _check(N % 4 == 0, "N must be divisible by 4")
    _check(scale.dim() == 2 and shift.dim() == 2, "scale/shift must be 2D [M, N] or [1, N]")
    _check(scale.size(0) == shift.size(0), "scale/shift row counts must match")
    _check(scale.size(0) == 1 or scale.size(0) == M,
           "scale/shift rows must be 1 (broadcast) or M (per-row modulation)")
    _check(scale.size(1) == N and shift.size(1) == N, "scale/shift last dim must be N")
    _check(scale.stride(-1) == 1 and shift.stride(-1) == 1, "scale/shift last dim must be contiguous")
    _check(x.dtype == scale.dtype and x.dtype == shift.dtype, "x/scale/shift dtype must match")
    _check(norm_type in (0, 1), "norm_type must be 0 (layer) or 1 (rms)")
    _check(x.dtype in _NORM_DTYPE, "Unsupported dtype; use float32/float16/bfloat16")
    if gamma_opt is not None:
        _check(gamma_opt.numel() == N, "gamma must be length N")
        gamma_opt = gamma_opt.to(x.dtype).contiguous()
    if beta_opt is not None:
        _check(beta_opt.numel() == N, "beta must be length N")
        beta_opt = beta_opt.to(x.dtype).contiguous()
    # the kernel reads scale/shift rows densely, as the reference kernel does (:112-117)
    return M, N, gamma_opt, beta_opt, scale.contiguous(), shift.contiguous()


@torch.library.impl(_lib_def, "fused_norm_scale_shift", "CUDA")
def _fused_norm_scale_shift_cuda(x, gamma_opt, beta_opt, scale, shift, norm_type, eps):
    M, N, gamma, beta, scale, shift = _norm_args(x, gamma_opt, beta_opt, scale, shift, norm_type)
    y = torch.empty((M, N), device=x.device, dtype=x.dtype)
    with torch.cuda.device(x.device):
        st = _LIB.joy_fused_norm_scale_shift(
            _ptr(x), x.stride(0) if M > 1 else N, _NORM_DTYPE[x.dtype], _ptr(gamma), _ptr(beta), _ptr(scale),
            _ptr(shift), scale.size(0), _ptr(y), M, N, int(norm_type), float(eps), _stream(x))
    _lib.check(_LIB, st)
    return y


@torch.library.impl(_lib_def, "fused_norm_scale_shift_fp8", "CUDA")
def _fused_norm_scale_shift_fp8_cuda(x, gamma_opt, beta_opt, scale, shift, norm_type, eps, output_q,
                                     output_s, out, exact_division):
    M, N, gamma, beta, scale, shift = _norm_args(x, gamma_opt, beta_opt, scale, shift, norm_type)
    _check(x.dtype in (torch.bfloat16, torch.float16), "x must be bfloat16 or float16")
    _check(output_q.is_cuda and output_q.is_contiguous() and output_q.dtype == torch.float8_e4m3fn
           and output_q.shape == (M, N), "output_q must be a contiguous float8_e4m3fn [M, N] CUDA tensor")
    _check(output_s.is_cuda and output_s.is_contiguous() and output_s.dtype == torch.float32
           and output_s.numel() == M, "output_s must contain one float32 scale per row")
    if out is not None:
        _check(out.is_cuda and out.is_contiguous() and out.dtype == x.dtype and out.shape == (M, N),
               "out must be a contiguous [M, N] CUDA tensor of x's dtype")
    rounding = _lib.JOY_QUANT_DIVIDE if exact_division else _lib.JOY_QUANT_RECIPROCAL
    with torch.cuda.device(x.device):
        st = _LIB.joy_fused_norm_scale_shift_fp8(
            _ptr(x), x.stride(0) if M > 1 else N, _NORM_DTYPE[x.dtype], _ptr(gamma), _ptr(beta), _ptr(scale),
            _ptr(shift), scale.size(0), _ptr(out), _ptr(output_q), _ptr(output_s), rounding, M, N,
            int(norm_type), float(eps), _stream(x))
    _lib.check(_LIB, st)


# --------------------------------------------------------------------------
# rmsnorm: outside the quantised path (the model never calls it); a torch
# device composition of rmsnorm.cu:60-84 keeps the reference import working
# --------------------------------------------------------------------------
@torch.library.impl(_lib_def, "rmsnorm", "CUDA")
def _rmsnorm_cuda(x, weight, eps):
    xf = x.float()
    return ((xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps)) * weight.float()).to(x.dtype)


# --------------------------------------------------------------------------
# FakeTensor kernels (reference __init__.py:39-101) so torch.compile keeps the
# ops opaque inside one graph.
# --------------------------------------------------------------------------
@torch.library.register_fake("joyomni_ops::fused_qk_norm_rope_3d_paired")
def _fake_fused_qk_norm_rope_3d_paired(q, k, seq_len, num_heads, eps, q_weight, k_weight, cos,
                                       sin, k_pre_rope=None):
    return None


@torch.library.register_fake("joyomni_ops::fused_joint_qkv_pack")
def _fake_fused_joint_qkv_pack(img_q, img_k, img_v, txt_q, txt_k, txt_v, cached_k, cached_v,
                               txt_q_weight, txt_k_weight, eps):
    batch, img_len, heads, head_dim = img_q.shape
    txt_len = txt_q.shape[1]
    cache_len = cached_k.shape[1] if cached_k is not None else 0
    out_q = img_q.new_empty((batch, img_len + txt_len, heads, head_dim))
    out_k = img_q.new_empty((batch, cache_len + img_len + txt_len, heads, head_dim))
    return out_q, out_k, torch.empty_like(out_k)


@torch.library.register_fake("joyomni_ops::fused_cached_kv_pack")
def _fake_fused_cached_kv_pack(key0, value0, key1, value1, cos, sin):
    batch, len0, heads, head_dim = key0.shape
    len1 = key1.shape[1] if key1 is not None else 0
    out_key = key0.new_empty((batch, len0 + len1, heads, head_dim))
    return out_key, torch.empty_like(out_key)


@torch.library.register_fake("joyomni_ops::fused_norm_scale_shift")
def _fake_fused_norm_scale_shift(x, gamma, beta, scale, shift, norm_type, eps):
    return torch.empty_like(x)


@torch.library.register_fake("joyomni_ops::fused_norm_scale_shift_fp8")
def _fake_fused_norm_scale_shift_fp8(x, gamma, beta, scale, shift, norm_type, eps, output_q, output_s,
                                     out, exact_division):
    return None


@torch.library.register_fake("joyomni_ops::rmsnorm")
def _fake_rmsnorm(x, weight, eps):
    return torch.empty_like(x)


@torch.library.register_fake("joyomni_ops::sgl_per_token_quant_fp8")
def _fake_sgl_per_token_quant_fp8(input, output_q, output_s):
    return None


@torch.library.register_fake("joyomni_ops::per_token_quant_fp8")
def _fake_per_token_quant_fp8(input, output_q, output_s, exact_division):
    return None


@torch.library.register_fake("joyomni_ops::fp8_scaled_mm")
def _fake_fp8_scaled_mm(mat_a, mat_b, scales_a, scales_b, out_dtype, bias=None):
    return mat_a.new_empty((mat_a.shape[0], mat_b.shape[1]), dtype=out_dtype)


@torch.library.register_fake("joyomni_ops::fp8_scaled_mm_gelu_tanh")
def _fake_fp8_scaled_mm_gelu_tanh(mat_a, mat_b, scales_a, scales_b, out_dtype, bias=None):
    return mat_a.new_empty((mat_a.shape[0], mat_b.shape[1]), dtype=out_dtype)


@torch.library.register_fake("joyomni_ops::fp8_scaled_mm_gated_residual")
def _fake_fp8_scaled_mm_gated_residual(mat_a, mat_b, scales_a, scales_b, residual, gate, bias=None):
    return residual.new_empty(residual.shape)


@torch.library.register_fake("joyomni_ops::fp8_scaled_mm_gated_residual_")
def _fake_fp8_scaled_mm_gated_residual_inplace(mat_a, mat_b, scales_a, scales_b, residual, gate, bias=None):
    return None


@torch.library.register_fake("joyomni_ops::fused_qkv_norm_rope_cache")
def _fake_fused_qkv_norm_rope_cache(qkv, num_heads, eps, q_weight, k_weight, cos, sin, q_out,
                                    k_out, cache_k, cache_v, slot, slot_offset, v_out=None, cache_tokens=-1,
                                    cache_pre_rope=True):
    return None


@torch.library.register_fake("joyomni_ops::fp8_qkv_norm_rope_cache")
def _fake_fp8_qkv_norm_rope_cache(mat_a, mat_b, scales_a, scales_b, bias, num_heads, eps, q_weight, k_weight, cos,
                                  sin, q_out, k_out, cache_k, cache_v, slot, slot_offset, v_out=None,
                                  cache_tokens=-1, cache_pre_rope=True):
    return None


@torch.library.register_fake("joyomni_ops::fused_cached_kv_pack_out")
def _fake_fused_cached_kv_pack_out(key0, value0, key1, value1, cos, sin, out_k, out_v):
    return None


@torch.library.register_fake("joyomni_ops::sdpa_attention")
def _fake_sdpa_attention(query, key, value, scale=None):
    return query.new_empty(query.shape)


@torch.library.register_fake("joyomni_ops::sdpa_attention_out")
def _fake_sdpa_attention_out(query, key, value, out, scale=None):
    return None


@torch.library.register_fake("joyomni_ops::fused_text_qkv_pack")
def _fake_fused_text_qkv_pack(txt_q, txt_k, txt_v, txt_q_weight, txt_k_weight, eps, out_q, out_k, out_v):
    return None


# --------------------------------------------------------------------------
# Python wrappers with the reference's names and signatures (__init__.py:104-153)
# --------------------------------------------------------------------------
def fused_qk_norm_rope_3d_paired(q, k, seq_len, num_heads, eps, q_weight, k_weight, cos, sin,
                                 k_pre_rope=None):
    """Per-head RMSNorm then interleaved RoPE on q and k, written over them (bf16 [B, seq_len * num_heads,
    head_dim]); ``k_pre_rope`` optionally receives k after the norm and before the rotation."""
    _ops.fused_qk_norm_rope_3d_paired(q, k, seq_len, num_heads, eps, q_weight, k_weight, cos, sin,
                                      k_pre_rope)


def fused_joint_qkv_pack(img_q, img_k, img_v, txt_q, txt_k, txt_v, cached_k, cached_v,
                         txt_q_weight, txt_k_weight, eps=1e-6):
    """Joint attention operands in fresh tensors: Q = [image | normed text], K / V = [cache | image | text],
    the text q / k RMS-normalised with two roundings; batch 1, head_dim 128, bf16."""
    return _ops.fused_joint_qkv_pack(img_q, img_k, img_v, txt_q, txt_k, txt_v, cached_k, cached_v,
                                     txt_q_weight, txt_k_weight, eps)


def fused_cached_kv_pack(key0, value0, key1, value1, cos, sin):
    """Cached keys stored before RoPE (one or two segments) rotated with fp32 full-width tables and
    concatenated, values concatenated alongside; batch 1, head_dim 128, bf16."""
    return _ops.fused_cached_kv_pack(key0, value0, key1, value1, cos, sin)


def fused_norm_scale_shift(x, gamma, beta, scale, shift, norm_type, eps=1e-5):
    """LayerNorm or RMSNorm of each row of x (optional affine gamma / beta), then adaLN modulation
    ``* (1 + scale) + shift``; ``norm_type`` is ``"layer"`` or ``"rms"``."""
    nt = 0 if norm_type == "layer" else 1 if norm_type == "rms" else -1
    return _ops.fused_norm_scale_shift(x, gamma, beta, scale, shift, nt, eps)


def fused_norm_scale_shift_fp8(x, gamma, beta, scale, shift, norm_type, eps, output_q, output_s,
                               out=None, exact_division: bool = True):
    """Norm + adaLN modulation quantised per token to e4m3fn in one pass: output_q/output_s are
    bit-identical to ``per_token_quant_fp8(fused_norm_scale_shift(...))``; ``out`` optionally
    receives the modulated row itself."""
    nt = 0 if norm_type == "layer" else 1 if norm_type == "rms" else -1
    _ops.fused_norm_scale_shift_fp8(x, gamma, beta, scale, shift, nt, eps, output_q, output_s, out,
                                    exact_division)


def rmsnorm(x, weight, eps=1e-6):
    """Row-wise RMS normalisation of x [M, N] scaled by weight [N]."""
    return _ops.rmsnorm(x, weight, eps)


def has_fp8() -> bool:
    return hasattr(_ops, "fp8_scaled_mm")


def has_quant() -> bool:
    return hasattr(_ops, "sgl_per_token_quant_fp8")


def sgl_per_token_quant_fp8(input, output_q, output_s):
    _ops.sgl_per_token_quant_fp8(input, output_q, output_s)


def fp8_scaled_mm(mat_a, mat_b, scales_a, scales_b, out_dtype, bias: Optional[torch.Tensor] = None):
    return _ops.fp8_scaled_mm(mat_a, mat_b, scales_a, scales_b, out_dtype, bias)


def per_token_quant_fp8(input, output_q, output_s, exact_division: bool = True):
    """Per-token e4m3fn quantisation; exact_division=True is bit-identical to
    ``_quantize_per_token_impl`` (deploy/xvideo/models/dit/fp8_linear.py:38-43)."""
    _ops.per_token_quant_fp8(input, output_q, output_s, exact_division)


def fp8_scaled_mm_gelu_tanh(mat_a, mat_b, scales_a, scales_b, out_dtype,
                            bias: Optional[torch.Tensor] = None):
    """fp8_scaled_mm followed by GELU-tanh on the rounded output, in one kernel."""
    return _ops.fp8_scaled_mm_gelu_tanh(mat_a, mat_b, scales_a, scales_b, out_dtype, bias)


def fp8_scaled_mm_gated_residual(mat_a, mat_b, scales_a, scales_b, residual, gate,
                                 bias: Optional[torch.Tensor] = None, inplace: bool = False):
    """residual + fp8_scaled_mm(mat_a, mat_b, ...) * gate in one kernel (the block's out-projection /
    FFN-down followed by fused_add_gate); output dtype = residual dtype, gate [N]. Bit-identical to
    ``torch.addcmul(residual, fp8_scaled_mm(...), gate)``. ``inplace=True`` writes into ``residual``
    (contiguous) and returns it."""
    if inplace:
        _ops.fp8_scaled_mm_gated_residual_(mat_a, mat_b, scales_a, scales_b, residual, gate, bias)
        return residual
    return _ops.fp8_scaled_mm_gated_residual(mat_a, mat_b, scales_a, scales_b, residual, gate, bias)


def fused_qkv_norm_rope_cache(qkv, num_heads, eps, q_weight, k_weight, cos, sin, q_out,
                              k_out=None, cache_k=None, cache_v=None, slot=0, slot_offset=0, v_out=None,
                              cache_tokens: int = -1, cache_pre_rope: bool = True):
    """QKV split + q/k RMSNorm + RoPE in one pass.

    Roped Q / K go to ``q_out`` / ``k_out`` (either may be None; without ``q_out`` Q is not read).
    The first ``cache_tokens`` tokens (all when negative; ``kv_cache_write_seq_len``) of K and V
    land in ring slot ``slot`` from row ``slot_offset``: K normalised before rotation when
    ``cache_pre_rope`` (``kv_cache_pre_rope=True``), else rotated. ``v_out`` (optional) receives V
    as well, e.g. the video rows of the joint attention V."""
    _ops.fused_qkv_norm_rope_cache(qkv, num_heads, eps, q_weight, k_weight, cos, sin, q_out, k_out,
                                   cache_k, cache_v, slot, slot_offset, v_out, cache_tokens, cache_pre_rope)


def fp8_qkv_norm_rope_cache(mat_a, mat_b, scales_a, scales_b, bias, num_heads, eps, q_weight, k_weight, cos, sin,
                            q_out, k_out=None, cache_k=None, cache_v=None, slot=0, slot_offset=0, v_out=None,
                            cache_tokens: int = -1, cache_pre_rope: bool = True):
    """The QKV projection (fp8_scaled_mm to bf16 [M, 3*H*D], scales as there) followed by
    fused_qkv_norm_rope_cache on its output (same arguments, cos/sin [M, D/2]), with the same
    results; the GEMM's epilogue writes the norm/RoPE/ring outputs itself where the shape allows,
    so the QKV rows are not stored in between."""
    _ops.fp8_qkv_norm_rope_cache(mat_a, mat_b, scales_a, scales_b, bias, num_heads, eps, q_weight, k_weight, cos,
                                 sin, q_out, k_out, cache_k, cache_v, slot, slot_offset, v_out, cache_tokens,
                                 cache_pre_rope)


def fused_cached_kv_pack_out(key0, value0, key1, value1, cos, sin, out_k, out_v):
    """fused_cached_kv_pack writing into caller-provided dense [1, len0 + len1, H, D] outputs,
    e.g. the cached rows at the head of the joint attention K / V."""
    _ops.fused_cached_kv_pack_out(key0, value0, key1, value1, cos, sin, out_k, out_v)


def fused_text_qkv_pack(txt_q, txt_k, txt_v, txt_q_weight, txt_k_weight, eps, out_q, out_k, out_v):
    """The condition segment of fused_joint_qkv_pack (two-rounding q/k RMSNorm, V copied) written
    into caller-provided dense [1, T, H, D] outputs (the tails of the joint Q / K / V)."""
    _ops.fused_text_qkv_pack(txt_q, txt_k, txt_v, txt_q_weight, txt_k_weight, eps, out_q, out_k, out_v)


def sdpa_attention(query, key, value, scale: Optional[float] = None):
    """softmax(q k^T * scale) v per head on [B, S, H, D] bf16 tensors, non-causal, no mask:
    the reference's ``_sdpa_attention`` (dit.py:154-167) without its transposes. scale defaults
    to 1/sqrt(D) like F.scaled_dot_product_attention; head_dim 128."""
    return _ops.sdpa_attention(query, key, value, scale)


def sdpa_attention_out(query, key, value, out, scale: Optional[float] = None):
    """sdpa_attention writing into ``out`` ([B, S, H, D], dense heads), e.g. rows of a
    [S, H*D] buffer that the out-projection quantiser reads."""
    _ops.sdpa_attention_out(query, key, value, out, scale)
