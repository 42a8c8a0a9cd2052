"""GPU: the QKV projection with its q/k RMSNorm, RoPE and KV-ring write in one op
(fp8_qkv_norm_rope_cache) equals the two-op sequence it replaces -- fp8_scaled_mm into a bf16
[M, 3*H*D] buffer, then fused_qkv_norm_rope_cache on that buffer (dit.py:409-451) -- bit for bit,
on every output: rotated Q and K, the ring slot's K (normalised or rotated) and V, the second V
destination, and the ring rows and slots it must not touch.

Cases cover the three ways a tile reaches the outputs: the persistent kernel's fused epilogue,
the sub-tiles of a last partial round (stored plainly, then the tail kernel), and the fallback of
shapes the fused epilogue does not take (odd head counts, head_dim 64, K % 256 != 0), which runs
the two-op sequence itself. Where the plain GEMM's kernel choice for a shape may differ from the
fused op's tile plan, operands are exact small integers with power-of-two scales, so every GEMM
output is exact whatever the summation order and the comparison isolates the norm/RoPE/ring work.
"""
import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, gen, u16
from oracle import rope as orope
from oracle.fp8 import f32_to_bf16, f32_to_e4m3fn

pytestmark = pytest.mark.gpu


def _fp8(a_f32: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(f32_to_e4m3fn(a_f32)).view(torch.float8_e4m3fn).to(DEV)


def _bf16(a_f32: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(f32_to_bf16(a_f32).view(np.int16)).view(torch.bfloat16).to(DEV)


def _problem(M, K, H, D, seed, exact):
    """Quantised activations [M, K], weight (K, N) column-major, scales, bias, norm weights and RoPE
    tables [M, D/2]."""
    rng = np.random.default_rng(seed)
    N = 3 * H * D
    if exact:
        a = _fp8(rng.integers(-8, 9, (M, K)).astype(np.float32))
        w = _fp8(rng.integers(-8, 9, (N, K)).astype(np.float32))
        sa = torch.from_numpy((2.0 ** rng.integers(-10, -5, M)).astype(np.float32)).to(DEV)
        sw = torch.from_numpy((2.0 ** rng.integers(-8, -4, N)).astype(np.float32)).to(DEV)
    else:
        import joyomni_ops as jo
        g = gen(seed)
        x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
        wf = (0.05 * torch.randn(N, K, generator=g)).to(torch.bfloat16).to(DEV)
        a = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=DEV)
        w = torch.empty(N, K, dtype=torch.float8_e4m3fn, device=DEV)
        sa = torch.empty(M, 1, device=DEV)
        sw = torch.empty(N, 1, device=DEV)
        jo.per_token_quant_fp8(x, a, sa, True)
        jo.per_token_quant_fp8(wf, w, sw, True)
        sa, sw = sa.reshape(M), sw.reshape(N)
    bias = _bf16((rng.integers(-32, 32, N) / 16).astype(np.float32))
    qw = _bf16((1 + 0.1 * rng.standard_normal(D)).astype(np.float32))
    kw = _bf16((1 + 0.1 * rng.standard_normal(D)).astype(np.float32))
    # 3-D RoPE tables of a frames x 16 x ww grid (at least M tokens), first M rows
    frames = max(1, M // 400)
    ww = (M + frames * 16 - 1) // (frames * 16)
    dims = (44, 42, 42) if D == 128 else (24, 20, 20)
    _, _, cb, sb = orope.rope_half_tables(list(range(frames)), 16, ww, dims, 10000.0)
    cos = torch.from_numpy(np.ascontiguousarray(cb[:M]).view(np.int16)).view(torch.bfloat16).to(DEV)
    sin = torch.from_numpy(np.ascontiguousarray(sb[:M]).view(np.int16)).view(torch.bfloat16).to(DEV)
    return a, w.t(), sa, sw, bias, qw, kw, cos, sin


def _outputs(M, H, D, slots, cap, seed):
    g = gen(seed)
    q = torch.randn(M, H, D, generator=g).to(torch.bfloat16).to(DEV)  # garbage: every row is written
    k = torch.randn(M, H, D, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(M, H, D, generator=g).to(torch.bfloat16).to(DEV)
    ck = torch.randn(slots, cap, H, D, generator=g).to(torch.bfloat16).to(DEV)  # other rows must keep these
    cv = torch.randn(slots, cap, H, D, generator=g).to(torch.bfloat16).to(DEV)
    return q, k, v, ck, cv


def _shift_table(t, elems):
    """The same table in a buffer whose first row starts `elems` elements past an aligned address."""
    buf = torch.empty(t.numel() + elems, dtype=t.dtype, device=t.device)
    view = buf[elems:].view(t.shape)
    view.copy_(t)
    return view


def _run_both(M, K, H, D, seed, exact, cache_tokens=-1, pre_rope=True, with_q=True, with_k=True, with_v=True,
              slot=1, offset=3, table_shift=0):
    import joyomni_ops as jo
    a, b, sa, sw, bias, qw, kw, cos, sin = _problem(M, K, H, D, seed, exact)
    if table_shift:
        cos, sin = _shift_table(cos, table_shift), _shift_table(sin, table_shift)
    n = M if cache_tokens < 0 else cache_tokens
    slots, cap = 3, offset + M + 5
    ref = _outputs(M, H, D, slots, cap, seed + 1)
    got = tuple(t.clone() for t in ref)
    y = jo.fp8_scaled_mm(a, b, sa, sw, torch.bfloat16, bias)
    jo.fused_qkv_norm_rope_cache(y, H, 1e-6, qw, kw, cos, sin, ref[0] if with_q else None, ref[1] if with_k else None,
                                 ref[3], ref[4], slot, offset, v_out=ref[2] if with_v else None, cache_tokens=n,
                                 cache_pre_rope=pre_rope)
    jo.fp8_qkv_norm_rope_cache(a, b, sa, sw, bias, H, 1e-6, qw, kw, cos, sin, got[0] if with_q else None,
                               got[1] if with_k else None, got[3], got[4], slot, offset,
                               v_out=got[2] if with_v else None, cache_tokens=n, cache_pre_rope=pre_rope)
    torch.cuda.synchronize()
    for name, r, o in zip(("q_out", "k_out", "v_out", "ring K", "ring V"), ref, got):
        assert torch.equal(u16_t(r), u16_t(o)), f"{name} differs ({M}x{K}, H {H}, D {D})"


def u16_t(t):
    return t.contiguous().view(torch.int16)


@pytest.mark.parametrize("M,K,H,D", [
    (4352, 1024, 32, 128),  # whole rounds through the fused epilogue + q, k and v tiles as quarter sub-tiles
    (2048, 1024, 8, 128),   # less than one round: every tile through the sub-tile launch
    (1000, 2048, 16, 128),  # ragged M
    (777, 512, 5, 128),     # odd head count: fallback
    (300, 1024, 6, 64),     # head_dim 64: fallback
    (640, 640, 4, 128),     # K % 256 != 0: fallback
    (1002, 1024, 8, 128),   # M % 4 != 0 (row scales read 4 at a time by the persistent kernel): fallback
])
def test_exact_equals_gemm_then_norm_rope(M, K, H, D):
    announce("fp8 qkv norm rope exact", M, K, H, D)
    _run_both(M, K, H, D, M + K + H, exact=True)


@pytest.mark.parametrize("pre_rope", [True, False])
def test_partial_cache_and_post_rope_ring(pre_rope):
    """kv_cache_write_seq_len: only the first rows reach the ring (at an offset, in slot 1); the ring K
    before or after RoPE."""
    announce("fp8 qkv norm rope partial cache", pre_rope)
    _run_both(4352, 1024, 32, 128, 11, exact=True, cache_tokens=4000, pre_rope=pre_rope)


def test_cache_only_forward():
    """kv_cache_write_only: no Q / K / V outputs, only the ring."""
    announce("fp8 qkv norm rope cache only")
    _run_both(4352, 1024, 32, 128, 12, exact=True, with_q=False, with_k=False, with_v=False)


def test_block_shape_random_operands():
    """The block's video stream at the benchmark's size (10800 tokens, 40 x 128 heads, K 5120) on
    random quantised operands: the fused op and the two-op sequence run the same GEMM kernels, so
    every output is bit-identical (the whole rounds through the fused epilogue, the last round's
    V tiles as quarter sub-tiles)."""
    announce("fp8 qkv norm rope block shape", 10800, 5120, 40, 128)
    _run_both(10800, 5120, 40, 128, 13, exact=False)


@pytest.mark.parametrize("M", [4352, 4096])  # a partial last round; whole rounds (no scratch otherwise)
def test_tables_not_16_byte_aligned(M):
    """cos / sin rows that start 8 bytes past a 16-byte boundary: the torch op reads an aligned copy
    (fused epilogue), the same bits as the two-op sequence."""
    announce("fp8 qkv norm rope unaligned tables", M)
    _run_both(M, 1024, 32, 128, 14, exact=True, table_shift=4)


def test_capi_unaligned_tables_need_the_full_scratch():
    """Through the C ABI, misaligned tables send the call to the unfused path, which needs the whole
    [M, 3E] bf16 scratch even where the size query says 0 (4096 rows: whole rounds of tiles): with
    no scratch the call fails before any launch and leaves the outputs alone; with M x 3E x 2 bytes
    it gives the two-op sequence's bits."""
    import joyomni_ops as jo
    from joyomni_ops import _lib
    announce("fp8 qkv norm rope C ABI unaligned tables")
    M, K, H, D = 4096, 1024, 32, 128
    N = 3 * H * D
    a, b, sa, sw, bias, qw, kw, cos, sin = _problem(M, K, H, D, 16, exact=True)
    cos, sin = _shift_table(cos, 4), _shift_table(sin, 4)
    assert jo._LIB.joy_fp8_qkv_norm_rope_cache_scratch_size(M, K, H, D) == 0
    slots, cap = 2, M
    ref = _outputs(M, H, D, slots, cap, 17)
    got = tuple(t.clone() for t in ref)
    y = jo.fp8_scaled_mm(a, b, sa, sw, torch.bfloat16, bias)
    jo.fused_qkv_norm_rope_cache(y, H, 1e-6, qw, kw, cos, sin, ref[0], ref[1], ref[3], ref[4], 1, 0, v_out=ref[2])
    before = tuple(t.clone() for t in got)
    st = torch.cuda.current_stream().cuda_stream

    def call(scratch, nbytes):
        return jo._LIB.joy_fp8_qkv_norm_rope_cache(
            a.data_ptr(), b.data_ptr(), sa.data_ptr(), sw.data_ptr(), bias.data_ptr(), M, K, H, D, 1e-6,
            qw.data_ptr(), kw.data_ptr(), cos.data_ptr(), sin.data_ptr(), got[0].data_ptr(), H * D,
            got[1].data_ptr(), H * D, got[2].data_ptr(), H * D, got[3].data_ptr(), got[4].data_ptr(), slots, cap, 1,
            0, M, 0, scratch, nbytes, st)

    rc = call(None, 0)
    assert rc == 1, rc  # JOY_ERR_INVALID_ARGUMENT
    assert b"scratch needed for this call" in jo._LIB.joy_last_error()
    torch.cuda.synchronize()
    for r, o in zip(before, got):
        assert torch.equal(u16_t(r), u16_t(o)), "outputs written by a refused call"
    scratch = torch.empty(M * N * 2, dtype=torch.uint8, device=DEV)
    _lib.check(jo._LIB, call(scratch.data_ptr(), scratch.numel()))
    torch.cuda.synchronize()
    for name, r, o in zip(("q_out", "k_out", "v_out", "ring K", "ring V"), ref, got):
        assert torch.equal(u16_t(r), u16_t(o)), f"{name} differs"


def test_no_ring_rows_written():
    """cache_tokens = 0: the ring keeps every row; Q / K / V are still written."""
    announce("fp8 qkv norm rope no ring rows")
    _run_both(4352, 1024, 32, 128, 15, exact=True, cache_tokens=0)
