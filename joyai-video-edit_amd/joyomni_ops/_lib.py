"""ctypes binding of libjoyomni_hip.so (the C ABI declared in include/joyomni_hip.h).

The library is built in-tree next to this file (``joyai-video-edit_amd/csrc/Makefile``).
Loading fails loudly when it is missing: there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
import os

LIB_NAME = "libjoyomni_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

JOY_OK = 0
JOY_ERR_INVALID_ARGUMENT = 1
JOY_ERR_UNSUPPORTED = 2
JOY_ERR_HIP = 3

JOY_DTYPE_BF16 = 0
JOY_DTYPE_FP16 = 1
JOY_DTYPE_FP32 = 2

JOY_NORM_LAYER = 0
JOY_NORM_RMS = 1

JOY_QUANT_DIVIDE = 0
JOY_QUANT_RECIPROCAL = 1

JOY_FP8_NOALLOC_SCRATCH_BYTES = 32 * 1024 * 1024

JOY_EPILOGUE_NONE = 0
JOY_EPILOGUE_GELU_TANH = 1

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float


class Bf16View(ctypes.Structure):
    """joy_bf16_view: bf16 [len, H, D] view, element (t, h, d) at ptr[t*stride_token + h*stride_head + d]."""
    _fields_ = [("ptr", ctypes.c_void_p), ("len", ctypes.c_int64), ("stride_token", ctypes.c_int64),
                ("stride_head", ctypes.c_int64)]


_view = ctypes.POINTER(Bf16View)

# name -> (restype, argtypes); mirrors include/joyomni_hip.h one to one.
SIGNATURES = {
    "joy_abi_version": (_int, []),
    "joy_last_error": (ctypes.c_char_p, []),
    "joy_init": (_int, []),
    "joy_per_token_quant_fp8": (_int, [_vp, _int, _vp, _vp, _i64, _i64, _int, _vp]),
    "joy_fp8_scaled_mm": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _int, _i64, _i64, _i64, _int, _vp, _i64, _vp]),
    "joy_fp8_scaled_mm_workspace_size": (_i64, [_i64, _i64, _i64]),
    "joy_fp8_scaled_mm_noalloc": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _int, _i64, _i64, _i64, _int, _vp]),
    "joy_fp8_scaled_mm_gated_residual": (
        _int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _int, _i64, _i64, _i64, _vp, _i64, _vp]),
    "joy_fused_qk_norm_rope_3d_paired": (
        _int, [_vp, _vp, _i64, _i64, _i64, _i64, _f32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "joy_fused_qkv_norm_rope_cache": (
        _int, [_vp, _i64, _i64, _i64, _i64, _f32, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _vp, _i64,
               _vp, _vp, _i64, _i64, _i64, _i64, _i64, _int, _vp]),
    "joy_fp8_qkv_norm_rope_cache": (
        _int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _i64,
               _vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _int, _vp, _i64, _vp]),
    "joy_fp8_qkv_norm_rope_cache_scratch_size": (_i64, [_i64, _i64, _i64, _i64]),
    "joy_fused_joint_qkv_pack": (
        _int, [_view, _view, _view, _view, _view, _view, _view, _view, _vp, _vp, _f32, _i64, _i64,
               _vp, _vp, _vp, _vp]),
    "joy_fused_text_qkv_pack": (
        _int, [_view, _view, _view, _vp, _vp, _f32, _i64, _i64, _vp, _vp, _vp, _vp]),
    "joy_fused_cached_kv_pack": (
        _int, [_view, _view, _view, _view, _vp, _vp, _i64, _i64, _vp, _vp, _vp]),
    "joy_attention_fwd": (_int, [_view, _view, _view, _vp, _i64, _i64, _i64, _f32, _vp]),
    "joy_fused_norm_scale_shift": (
        _int, [_vp, _i64, _int, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _int, _f32, _vp]),
    "joy_fused_norm_scale_shift_fp8": (
        _int, [_vp, _i64, _int, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _int, _i64, _i64, _int, _f32,
               _vp]),
}

ABI_VERSION = 10


class JoyError(RuntimeError):
    """A non-OK status from the C ABI (argument check failure or HIP launch error)."""


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise ImportError(
            f"{LIB_NAME} not found at {path}; build it first "
            "(python -c 'import __graft_entry__ as g; g.build()' or make -C joyai-video-edit_amd/csrc)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.joy_abi_version() != ABI_VERSION:
        raise ImportError(f"{LIB_NAME} ABI version {lib.joy_abi_version()} != {ABI_VERSION}")
    return lib


def check(lib: ctypes.CDLL, status: int) -> None:
    if status != JOY_OK:
        raise JoyError(lib.joy_last_error().decode())
