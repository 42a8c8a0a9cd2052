"""GPU parity: the FP8 GEMM with the block's gated residual in its epilogue
(fp8_scaled_mm_gated_residual) -- bit-exact, as fused_add_gate's torch.addcmul
(sgl_fused_ops.py:302-305) rounds the fp32 sum of residual and the exact product
y * gate once, which is what the epilogue's fma does.

Pins: exact small-integer problems against the GEMM oracle's output put through
torch.addcmul on the CPU (bf16 and fp16); gate = 0 returns the residual and
residual = 0 with gate = 1 returns the plain GEMM, bit for bit; random problems on
every launch shape (small-M, 256x256 rounds plus split remainder, the generic kernel)
equal torch.addcmul over the plain fp8_scaled_mm output, computed on the CPU (IEEE fp32
with fp16 denormals kept, as the reference's CUDA build); the in-place form, a
row-strided residual and an unaligned gate give the same bytes."""
import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, gen, u16
from oracle import gemm as og
from oracle.fp8 import f32_to_bf16, f32_to_e4m3fn

pytestmark = pytest.mark.gpu


def fp8_dev(q_u8):
    return torch.from_numpy(np.ascontiguousarray(q_u8)).view(torch.float8_e4m3fn).to(DEV)


def exact_problem(M, N, K, seed):
    rng = np.random.default_rng(seed)
    qa = f32_to_e4m3fn(rng.integers(-8, 9, (M, K)).astype(np.float32))
    qw = f32_to_e4m3fn(rng.integers(-8, 9, (N, K)).astype(np.float32))
    sa = (2.0 ** rng.integers(-8, 2, M)).astype(np.float32)
    sw = (2.0 ** rng.integers(-8, 2, N)).astype(np.float32)
    bias = f32_to_bf16((rng.integers(-64, 64, N) / 16).astype(np.float32))
    return qa, qw, sa, sw, bias


def operands(qa, qw, sa, sw):
    return (fp8_dev(qa), fp8_dev(qw).t(), torch.from_numpy(sa).to(DEV).reshape(-1, 1),
            torch.from_numpy(sw).to(DEV).reshape(1, -1))


@pytest.mark.parametrize("M,N,K", [(300, 264, 256), (1, 520, 384), (200, 4104, 640), (33, 40, 48),
                                   (513, 520, 384),
                                   # small-M plans with a K split (partials reduced before the epilogue)
                                   (64, 2048, 4096), (500, 4104, 1664)])
def test_exact_problems_bit_exact(M, N, K):
    import joyomni_ops as jo
    announce("gated residual exact", M, N, K)
    qa, qw, sa, sw, bias = exact_problem(M, N, K, M * 3 + N)
    y_bits, _ = og.scaled_mm(qa, qw, sa, sw, bias)
    y = torch.from_numpy(y_bits.view(np.int16)).view(torch.bfloat16)
    g = gen(M + K)
    res = torch.randn(M, N, generator=g).to(torch.bfloat16)
    gate = torch.randn(N, generator=g).to(torch.bfloat16)
    a, b, s_a, s_b = operands(qa, qw, sa, sw)
    bias_d = torch.from_numpy(bias.view(np.int16)).view(torch.bfloat16).to(DEV)
    out = jo.fp8_scaled_mm_gated_residual(a, b, s_a, s_b, res.to(DEV), gate.to(DEV), bias_d)
    zero_gate = jo.fp8_scaled_mm_gated_residual(a, b, s_a, s_b, res.to(DEV), torch.zeros_like(gate, device=DEV),
                                                bias_d)
    plain = jo.fp8_scaled_mm_gated_residual(a, b, s_a, s_b, torch.zeros(M, N, dtype=torch.bfloat16, device=DEV),
                                            torch.ones(N, dtype=torch.bfloat16, device=DEV), bias_d)
    torch.cuda.synchronize()
    exp = torch.addcmul(res, y, gate[None])
    assert np.array_equal(u16(out), u16(exp)), f"{np.count_nonzero(u16(out) != u16(exp))} outputs differ"
    assert np.array_equal(u16(zero_gate), u16(res))
    assert np.array_equal(u16(plain), y_bits)


def test_exact_fp16():
    import joyomni_ops as jo
    announce("gated residual exact fp16")
    M, N, K = 130, 136, 192
    qa, qw, sa, sw, _ = exact_problem(M, N, K, 5)
    y_bits, _ = og.scaled_mm(qa, qw, sa, sw, None, out_dtype="fp16")
    y = torch.from_numpy(y_bits.view(np.int16)).view(torch.float16)
    g = gen(6)
    res = torch.randn(M, N, generator=g).half()
    gate = torch.randn(N, generator=g).half()
    a, b, s_a, s_b = operands(qa, qw, sa, sw)
    out = jo.fp8_scaled_mm_gated_residual(a, b, s_a, s_b, res.to(DEV), gate.to(DEV))
    torch.cuda.synchronize()
    exp = torch.addcmul(res, y, gate[None])
    assert np.array_equal(u16(out), u16(exp))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", [(64, 5120, 5120), (256, 15360, 1024), (400, 15360, 640), (1560, 12288, 256),
                                   (4352, 4352, 256),
                                   (2048, 5120, 13824), (777, 1000, 320),
                                   # persistent 256x256 kernel (K % 256 == 0, M % 4 == 0): a whole
                                   # round plus a sub-tile tail, and a single partial round
                                   (4352, 4352, 512), (2600, 2304, 512),
                                   # narrow 80-column tiles (the condition stream's 512-token
                                   # projections; 64-row tiles with padding rows)
                                   (512, 5120, 5120), (200, 5120, 768)])
def test_random_equals_addcmul_over_plain_gemm(dtype, M, N, K):
    """Large / every-launch-shape problems: the fused epilogue equals torch.addcmul applied to
    fp8_scaled_mm's own output (the same kernel tiling sums each output in the same order)."""
    import joyomni_ops as jo
    announce("gated residual random", dtype, M, N, K)
    g = gen(M + N + K)
    a = (torch.randn(M, K, generator=g) * 2).to(torch.float8_e4m3fn).to(DEV)
    w = (torch.randn(N, K, generator=g) * 2).to(torch.float8_e4m3fn).to(DEV)
    s_a = (torch.rand(M, 1, generator=g) * 0.01 + 1e-3).to(DEV)
    s_b = (torch.rand(1, N, generator=g) * 0.01 + 1e-3).to(DEV)
    bias = (torch.randn(N, generator=g) * 0.1).to(dtype).to(DEV)
    res = torch.randn(M, N, generator=g).to(dtype).to(DEV)
    gate = (torch.randn(N, generator=g) * 0.5).to(dtype).to(DEV)
    y = jo.fp8_scaled_mm(a, w.t(), s_a, s_b, dtype, bias)
    out = jo.fp8_scaled_mm_gated_residual(a, w.t(), s_a, s_b, res, gate, bias)
    inplace = res.clone()
    ret = jo.fp8_scaled_mm_gated_residual(a, w.t(), s_a, s_b, inplace, gate, bias, inplace=True)
    dev_addcmul = torch.addcmul(res, y, gate[None])
    torch.cuda.synchronize()
    exp = torch.addcmul(res.cpu(), y.cpu(), gate.cpu()[None])
    r = res.cpu()
    denormal = int(((r != 0) & (r.float().abs() < torch.finfo(dtype).tiny)).sum())
    print(f"denormal residuals {denormal}; device torch.addcmul differs from the CPU on "
          f"{int((dev_addcmul.cpu() != exp).sum())} outputs")
    assert ret is inplace
    assert torch.equal(out.cpu(), exp), f"{int((out.cpu() != exp).sum())} outputs differ"
    assert torch.equal(inplace.cpu(), exp)


def test_strided_residual_and_unaligned_gate():
    import joyomni_ops as jo
    announce("gated residual strided")
    M, N, K = 300, 512, 256
    g = gen(9)
    a = (torch.randn(M, K, generator=g) * 2).to(torch.float8_e4m3fn).to(DEV)
    w = (torch.randn(N, K, generator=g) * 2).to(torch.float8_e4m3fn).to(DEV)
    s_a = torch.full((M, 1), 0.01, device=DEV)
    s_b = torch.full((1, N), 0.02, device=DEV)
    wide = torch.randn(M, N + 24, generator=g).to(torch.bfloat16).to(DEV)
    res = wide[:, 8:8 + N]                          # row stride N + 24, 16-byte aligned start
    gate_store = torch.randn(N + 1, generator=g).to(torch.bfloat16).to(DEV)
    gate = gate_store[1:]                           # 2-byte aligned: the op copies it
    y = jo.fp8_scaled_mm(a, w.t(), s_a, s_b, torch.bfloat16)
    out = jo.fp8_scaled_mm_gated_residual(a, w.t(), s_a, s_b, res, gate)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), torch.addcmul(res.cpu(), y.cpu(), gate.cpu()[None]))
    with pytest.raises(RuntimeError, match="in-place residual must be contiguous"):
        jo.fp8_scaled_mm_gated_residual(a, w.t(), s_a, s_b, res, gate, inplace=True)
    with pytest.raises(RuntimeError, match="size of gate"):
        jo.fp8_scaled_mm_gated_residual(a, w.t(), s_a, s_b, res.contiguous(), gate[:8])
    with pytest.raises(RuntimeError, match="gate dtype"):
        jo.fp8_scaled_mm_gated_residual(a, w.t(), s_a, s_b, res.contiguous(), gate.half())
