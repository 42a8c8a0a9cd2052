"""The C-ABI library loads, exports every symbol include/joyomni_hip.h declares,
and rejects bad arguments before touching the GPU (no compute calls here)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "joyomni_hip.h")

from joyomni_ops import _lib  # noqa: E402  (conftest puts the package dir on sys.path)


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"JOY_API\s+[\w\s\*]+?\b(joy_\w+)\s*\(", text)))


# JOY_HIP_LIB names another build of the library to check (the sanitizer build of
# tests/test_sanitized_capi.py); by default the in-tree library.
LIB_PATH = os.environ.get("JOY_HIP_LIB", _lib.LIB_PATH)


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB_PATH):
        pytest.fail(f"{LIB_PATH} missing: run __graft_entry__.build()")
    return _lib.load(LIB_PATH)


def test_header_declares_expected_entry_points():
    names = declared_functions()
    assert names == sorted(_lib.SIGNATURES), names


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    for name in declared_functions():
        assert name in exported, name
    # nothing else with the joy_ prefix leaks out
    assert {n for n in exported if n.startswith("joy_")} == set(declared_functions())


def test_abi_version(lib):
    assert lib.joy_abi_version() == _lib.ABI_VERSION


def _status(lib, st, code, fragment):
    assert st == code, lib.joy_last_error()
    assert fragment in lib.joy_last_error().decode()


def test_quant_argument_checks(lib):
    p = ctypes.c_void_p(0x1000)
    _status(lib, lib.joy_per_token_quant_fp8(p, 7, p, p, 4, 16, 0, None), 1, "bfloat16 or float16")
    _status(lib, lib.joy_per_token_quant_fp8(p, 0, p, p, 4, 16, 5, None), 1, "rounding")
    _status(lib, lib.joy_per_token_quant_fp8(p, 0, p, None, 4, 16, 0, None), 1, "one scale per row")
    _status(lib, lib.joy_per_token_quant_fp8(p, 0, p, p, -1, 16, 0, None), 1, "[M, K]")
    assert lib.joy_per_token_quant_fp8(None, 0, None, None, 0, 16, 0, None) == 0  # empty: no launch


def test_gemm_argument_checks(lib):
    p = ctypes.c_void_p(0x1000)
    args = lambda **kw: [kw.get("a", p), kw.get("b", p), p, p, None, p, kw.get("dt", 0),  # noqa: E731
                         kw.get("M", 64), kw.get("N", 64), kw.get("K", 64), kw.get("epi", 0),
                         kw.get("ws", None), kw.get("wsb", 0), None]
    _status(lib, lib.joy_fp8_scaled_mm(*args(K=40)), 1, "multiple of 16 bytes")
    _status(lib, lib.joy_fp8_scaled_mm(*args(N=36)), 1, "out must be multiple of 16 bytes")
    _status(lib, lib.joy_fp8_scaled_mm(*args(dt=5)), 1, "Half or BFloat16")
    _status(lib, lib.joy_fp8_scaled_mm(*args(epi=9)), 1, "epilogue")
    _status(lib, lib.joy_fp8_scaled_mm(*args(a=ctypes.c_void_p(0x1008))), 2, "16-byte aligned")
    _status(lib, lib.joy_fp8_scaled_mm(*args(wsb=-1)), 1, "workspace_bytes")
    _status(lib, lib.joy_fp8_scaled_mm(*args(wsb=4096)), 1, "with a workspace")
    _status(lib, lib.joy_fp8_scaled_mm(*args(ws=ctypes.c_void_p(0x1004), wsb=4096)), 1,
            "workspace must be 16-byte aligned")
    assert lib.joy_fp8_scaled_mm(*args(M=0)) == 0


def test_gemm_workspace_size(lib):
    """Host-side plan: split-K only for small M where the tiles leave CUs idle and no narrow-tile
    plan fills them (256-CU MI355X when no device is visible); the size is splits * M * N fp32
    partial sums."""
    size = lib.joy_fp8_scaled_mm_workspace_size
    ws = size(64, 5120, 5120)
    assert ws > 0 and ws % (64 * 5120 * 4) == 0 and 2 <= ws // (64 * 5120 * 4) <= 8
    assert size(10800, 5120, 5120) == 0      # large M: full rounds of 256x256 tiles, no split
    assert size(64, 15360, 5120) == 0        # 240 tiles already cover the CUs
    assert size(64, 5120, 5120 + 64) == 0    # K not a multiple of the plan's K step
    # N % 80 == 0 where one round of 80-column tiles fills the CUs: no split
    assert size(256, 5120, 5120) == 0 and size(200, 5120, 768) == 0 and size(512, 5120, 5120) == 0
    assert size(256, 5136, 5120) > 0         # the same rows with 128x128 tiles split over K
    assert size(512, 5120, 13824) > 0        # long K: larger tiles split over K move fewer bytes
    assert size(0, 5120, 5120) == 0 and size(-1, 8, 64) == 0 and size(64, 36, 64) == 0


def test_gated_residual_argument_checks(lib):
    p, r, g = ctypes.c_void_p(0x1000), ctypes.c_void_p(0x2000), ctypes.c_void_p(0x3000)
    args = lambda **kw: [p, p, p, p, None, kw.get("r", r), kw.get("ld", 64), kw.get("g", g),  # noqa: E731
                         kw.get("out", p), 0, kw.get("M", 64), 64, 64, None, 0, None]
    f = lib.joy_fp8_scaled_mm_gated_residual
    _status(lib, f(*args(r=None)), 1, "residual must be non-null")
    _status(lib, f(*args(g=None)), 1, "gate must be non-null")
    _status(lib, f(*args(ld=32)), 1, "row stride must be >= N")
    _status(lib, f(*args(out=r, ld=72)), 1, "in-place residual must have row stride N")
    _status(lib, f(*args(r=ctypes.c_void_p(0x2001))), 1, "naturally aligned")
    assert f(*args(M=0)) == 0


def test_norm_rope_argument_checks(lib):
    p = ctypes.c_void_p(0x1000)
    _status(lib, lib.joy_fused_qk_norm_rope_3d_paired(p, p, 1, 4, 2, 96, 1e-6, p, p, p, p, None, None),
            1, "Unsupported head_dim")
    _status(lib, lib.joy_fused_qk_norm_rope_3d_paired(p, p, 1, 4, 2, 128, 1e-6, None, p, p, p, None, None),
            1, "non-null")
    f = lib.joy_fused_qkv_norm_rope_cache

    def call(qkv_stride=3 * 256, q=p, q_st=256, v=None, v_st=0, ck=p, cv=p, slots=4, cap=16, slot=0, off=0,
             ntok=4, post=0):
        return f(p, qkv_stride, 4, 2, 128, 1e-6, p, p, p, p, q, q_st, None, 0, v, v_st, ck, cv, slots, cap, slot,
                 off, ntok, post, None)

    _status(lib, call(cv=None), 1, "provided together")
    _status(lib, call(slot=4), 1, "slot 4 out of range")
    _status(lib, call(slot=1, off=13), 1, "do not fit")
    _status(lib, call(ntok=5), 1, "cache_tokens 5 out of range")
    _status(lib, call(ntok=-1), 1, "cache_tokens -1 out of range")
    _status(lib, call(qkv_stride=100, ck=None, cv=None), 1, "row stride")
    _status(lib, call(v=p, v_st=128, ck=None, cv=None), 1, "q_out/k_out/v_out token stride")
    _status(lib, call(v=ctypes.c_void_p(0x1008), v_st=256, ck=None, cv=None), 2, "16-byte aligned")
    _status(lib, call(q=ctypes.c_void_p(0x1008), ck=None, cv=None), 2, "16-byte aligned")
    # only the first cache_tokens tokens must fit the slot (kv_cache_write_seq_len, dit.py:449-451)
    _status(lib, call(q=ctypes.c_void_p(0x1008), slot=1, off=14, ntok=2), 2, "16-byte aligned")
    _status(lib, call(q=ctypes.c_void_p(0x1008), slot=1, off=14, ntok=3), 1, "do not fit")
    # nothing to write is a successful no-op, even with a null qkv
    assert f(None, 3 * 256, 4, 2, 128, 1e-6, None, None, None, None, None, 0, None, 0, None, 0, None, None, 0, 0,
             0, 0, 0, 0, None) == 0


def test_fused_qkv_projection_scratch_checks(lib):
    """The QKV projection with norm/RoPE/ring in its epilogue: the scratch this call needs is checked
    before any launch -- 0 bytes for 4096 rows x 32 heads (whole rounds of tiles) with aligned tables,
    the whole [M, 3E] bf16 buffer with 8-byte aligned ones (unfused path) -- and a shape with a partial
    last round needs it whatever the tables."""
    p, p8 = ctypes.c_void_p(0x10000), ctypes.c_void_p(0x10008)
    f = lib.joy_fp8_qkv_norm_rope_cache
    size = lib.joy_fp8_qkv_norm_rope_cache_scratch_size

    def call(M, cos=p, scratch=None, nbytes=0):
        E = 32 * 128
        return f(p, p, p, p, None, M, 1024, 32, 128, 1e-6, p, p, cos, cos, p, E, p, E, None, 0, None, None, 0, 0,
                 0, 0, M, 0, scratch, nbytes, None)

    assert size(4096, 1024, 32, 128) == 0 and size(4352, 1024, 32, 128) == 4352 * 3 * 4096 * 2
    _status(lib, call(4096, cos=p8), 1, "bytes of scratch needed for this call")
    _status(lib, call(4352), 1, "bytes of scratch needed for this call")
    _status(lib, call(4352, scratch=p, nbytes=-1), 1, "scratch_bytes must be >= 0")


def test_single_hip_runtime_in_process():
    """The library must bind to the HIP runtime torch already loaded (same SONAME),
    so its launches share torch's streams and queues."""
    import torch  # noqa: F401
    import joyomni_ops  # noqa: F401
    maps = open("/proc/self/maps").read().splitlines()
    hip = {line.split()[-1] for line in maps if "libamdhip64" in line}
    assert len(hip) == 1, hip


def _v(lib, ptr, n, st=3 * 2 * 128, sh=128):
    return ctypes.byref(_lib.Bf16View(ptr, n, st, sh))


def test_joint_pack_argument_checks(lib):
    p = 0x1000
    f = lib.joy_fused_joint_qkv_pack
    w = ctypes.c_void_p(p)
    img = [_v(lib, p, 4) for _ in range(3)]
    txt = [_v(lib, p, 2) for _ in range(3)]
    out = [w, w, w]
    _status(lib, f(*img, *txt, None, None, w, w, 1e-6, 2, 64, *out, None), 1, "requires head_dim=128")
    _status(lib, f(*img, *txt, _v(lib, p, 3), None, w, w, 1e-6, 2, 128, *out, None), 1,
            "both be present or both be absent")
    _status(lib, f(*img, *txt, _v(lib, p, 3), _v(lib, p, 2), w, w, 1e-6, 2, 128, *out, None), 1,
            "cached K/V lengths must match")
    _status(lib, f(img[0], _v(lib, p, 3), img[2], *txt, None, None, w, w, 1e-6, 2, 128, *out, None), 1,
            "image Q/K/V lengths must match")
    _status(lib, f(*img, _v(lib, p, 0), txt[1], txt[2], None, None, w, w, 1e-6, 2, 128, *out, None), 1,
            "text Q/K/V lengths must match and be positive")
    _status(lib, f(*img, *txt, None, None, None, w, 1e-6, 2, 128, *out, None), 1, "weight")
    _status(lib, f(None, *img[1:], *txt, None, None, w, w, 1e-6, 2, 128, *out, None), 1, "non-null")


def test_text_pack_argument_checks(lib):
    p = 0x1000
    f = lib.joy_fused_text_qkv_pack
    w = ctypes.c_void_p(p)
    txt = [_v(lib, p, 2) for _ in range(3)]
    _status(lib, f(*txt, w, w, 1e-6, 2, 64, w, w, w, None), 1, "requires head_dim=128")
    _status(lib, f(txt[0], _v(lib, p, 3), txt[2], w, w, 1e-6, 2, 128, w, w, w, None), 1,
            "text Q/K/V lengths must match and be positive")
    _status(lib, f(*txt, None, w, 1e-6, 2, 128, w, w, w, None), 1, "weight")
    _status(lib, f(None, *txt[1:], w, w, 1e-6, 2, 128, w, w, w, None), 1, "non-null")
    _status(lib, f(*txt, w, w, 1e-6, 2, 128, w, None, w, None), 1, "out_q, out_k and out_v")


def test_cached_pack_argument_checks(lib):
    p = 0x1000
    f = lib.joy_fused_cached_kv_pack
    w = ctypes.c_void_p(p)
    k0 = _v(lib, p, 5)
    _status(lib, f(k0, k0, None, None, w, w, 2, 256, w, w, None), 1, "requires head_dim=128")
    _status(lib, f(k0, _v(lib, p, 4), None, None, w, w, 2, 128, w, w, None), 1, "key0/value0 lengths must match")
    _status(lib, f(k0, k0, k0, None, w, w, 2, 128, w, w, None), 1, "key1 and value1")
    _status(lib, f(k0, k0, _v(lib, p, 3), _v(lib, p, 2), w, w, 2, 128, w, w, None), 1,
            "key1/value1 lengths must match and be positive")
    _status(lib, f(_v(lib, p, 0), _v(lib, p, 0), None, None, w, w, 2, 128, w, w, None), 1,
            "cache length and heads must be positive")
    _status(lib, f(k0, k0, None, None, None, w, 2, 128, w, w, None), 1, "cos and sin")


def test_norm_argument_checks(lib):
    p = ctypes.c_void_p(0x1000)
    f = lib.joy_fused_norm_scale_shift
    _status(lib, f(p, 64, 0, None, None, p, p, 1, p, 4, 62, 0, 1e-6, None), 1, "divisible by 4")
    _status(lib, f(p, 64, 0, None, None, p, p, 2, p, 4, 64, 0, 1e-6, None), 1, "broadcast")
    _status(lib, f(p, 64, 0, None, None, p, p, 1, p, 4, 64, 3, 1e-6, None), 1, "norm_type")
    _status(lib, f(p, 64, 9, None, None, p, p, 1, p, 4, 64, 0, 1e-6, None), 1, "Unsupported dtype")
    _status(lib, f(p, 32, 0, None, None, p, p, 1, p, 4, 64, 0, 1e-6, None), 1, "row stride")
    assert f(None, 64, 0, None, None, None, None, 1, None, 0, 64, 0, 1e-6, None) == 0
    g = lib.joy_fused_norm_scale_shift_fp8
    _status(lib, g(p, 64, 2, None, None, p, p, 1, None, p, p, 0, 4, 64, 0, 1e-6, None), 1,
            "bfloat16 or float16")
    _status(lib, g(p, 64, 0, None, None, p, p, 1, None, p, p, 7, 4, 64, 0, 1e-6, None), 1, "rounding")
    _status(lib, g(p, 64, 0, None, None, p, p, 1, None, None, p, 0, 4, 64, 0, 1e-6, None), 1, "output_q")


def test_attention_argument_checks(lib):
    V = _lib.Bf16View
    good = V(0x1000, 8, 256, 128)
    keys = V(0x2000, 16, 256, 128)
    f = lib.joy_attention_fwd
    b = ctypes.byref
    out = ctypes.c_void_p(0x4000)
    _status(lib, f(b(good), b(keys), b(keys), out, 256, 2, 64, 0.1, None), 2, "head_dim=128")
    _status(lib, f(None, b(keys), b(keys), out, 256, 2, 128, 0.1, None), 1, "views must be non-null")
    _status(lib, f(b(good), b(keys), b(V(0x3000, 15, 256, 128)), out, 256, 2, 128, 0.1, None), 1,
            "same sequence length")
    _status(lib, f(b(good), b(V(0, 0, 256, 128)), b(V(0, 0, 256, 128)), out, 256, 2, 128, 0.1, None), 1,
            "empty key sequence")
    _status(lib, f(b(good), b(keys), b(keys), out, 128, 2, 128, 0.1, None), 1, "out token stride")
    _status(lib, f(b(good), b(keys), b(keys), out, 256, 2, 128, -1.0, None), 1, "scale must be positive")
    _status(lib, f(b(V(0x1008, 8, 256, 128)), b(keys), b(keys), out, 256, 2, 128, 0.1, None), 2,
            "16-byte aligned rows")
    assert f(b(V(0, 0, 256, 128)), b(keys), b(keys), out, 256, 2, 128, 0.1, None) == 0  # no queries: no launch


def test_init_is_ok_without_a_device(lib):
    """joy_init resolves per-device state for every visible device; with none visible (this CPU
    container) it has nothing to do and returns JOY_OK."""
    assert lib.joy_init() == _lib.JOY_OK, lib.joy_last_error()
