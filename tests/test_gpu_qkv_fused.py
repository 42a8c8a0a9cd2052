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


def _run_both(M, K, H, D, seed, exact, cache_tokens=-1, pre_rope=True, with_q=True, with_k=True, with_v=True,
              slot=1, offset=3):
    import joyomni_ops as jo
    a, b, sa, sw, bias, qw, kw, cos, sin = _problem(M, K, H, D, seed, exact)
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
