"""Pins the torch restatements of the reference's CPU path (oracle/torch_path.py), which
bench.py times as the CPU baseline and the block test uses as its checker, to the pinned
numpy oracle functions: quantiser bytes and scales bit-exact, the FP8 linear within one bf16
rounding of the fp32 dequantise-then-matmul, the norm/RoPE fallback within the extra rounding
of its normalised q/k (sgl_fused_ops.py:170-199), V and ring V bit-exact."""
import numpy as np
import pytest
import torch

from oracle import gemm as ogemm
from oracle import kvpack as okv
from oracle import normmod as onm
from oracle import qknorm as oqk
from oracle import quant as oquant
from oracle import torch_path
from oracle.fp8 import bf16_to_f32


def u16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def u8(t):
    return t.contiguous().view(torch.uint8).numpy()


def _act(M, K, g):
    x = torch.randn(M, K, generator=g)
    x[:, torch.randperm(K, generator=g)[: max(1, K // 200)]] *= 20  # outlier channels (cfg 0)
    x[3] = 0  # zero row: s = 1e-8 / 448
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("exact", [True, False])
def test_quantize_per_token_bit_exact(exact):
    g = torch.Generator().manual_seed(10)
    x = _act(67, 4096, g)
    q, s = torch_path.quantize_per_token_rounding(x, exact)
    oq, osc = oquant.quant_per_token(u16(x), "bf16", "div" if exact else "rcp")
    assert np.array_equal(u8(q), oq) and np.array_equal(s.reshape(-1).numpy(), osc)
    if exact:
        q2, s2 = torch_path.quantize_per_token(x)
        assert torch.equal(q2.view(torch.uint8), q.view(torch.uint8)) and torch.equal(s2, s)


def test_fp8_linear_within_one_rounding_of_fp32_reference():
    g = torch.Generator().manual_seed(11)
    M, K, N = 48, 512, 384
    x = _act(M, K, g)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    wq, ws = oquant.quant_weight_per_channel(u16(w))
    bias = (torch.randn(N, generator=g) * 0.01).to(torch.bfloat16)
    y = torch_path.fp8_linear(x, torch.from_numpy(wq).view(torch.float8_e4m3fn), torch.from_numpy(ws), bias)
    qa, sa = oquant.quant_per_token(u16(x), "bf16", "div")
    ref = ogemm.reference_fp32(qa, wq, sa, ws, u16(bias))
    got = y.float().numpy()
    # one bf16 rounding plus fp32 summation-order noise (sum |a b| * 2^-22)
    bound = np.abs(ref) * 2.0 ** -8 + ogemm.abs_acc(qa, wq) * sa[:, None] * ws[None, :] * 2.0 ** -20 + 1e-30
    assert np.all(np.abs(got - ref) <= bound)
    # a dropped weight scale or bias misses by far more
    assert np.abs(got - ogemm.reference_fp32(qa, wq, sa, np.ones_like(ws), u16(bias))).max() > 1.0
    assert np.abs(got - ogemm.reference_fp32(qa, wq, sa, ws, None)).max() > 1e-3


def test_qkv_norm_rope_cache_fallback_matches_kernel_oracle():
    g = torch.Generator().manual_seed(12)
    L, H, D, slots, slot = 40, 4, 128, 3, 1
    qkv = torch.randn(L, 3 * H * D, generator=g).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    ang = torch.rand(L, D // 2, generator=g) * 6.28
    cos, sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    ck = torch.zeros(slots, L, H, D, dtype=torch.bfloat16)
    cv = torch.zeros_like(ck)
    q, k = torch_path.qkv_norm_rope_cache(qkv, H, 1e-6, qw, kw, cos, sin, ck, cv, slot)
    oq, ok, okp, ov = oqk.qkv_norm_rope_cache(u16(qkv), H, 1e-6, u16(qw), u16(kw), u16(cos), u16(sin))
    assert np.array_equal(u16(cv[slot]), ov)
    assert not ck[0].any() and not cv[2].any()
    # ring K: both round the same fp32 normalised value once (sum order and rsqrt may move one ulp)
    kp = bf16_to_f32(okp)
    assert np.all(np.abs(bf16_to_f32(u16(ck[slot])) - kp) <= np.abs(kp) * 2.0 ** -8)
    # roped q/k: the fallback rounds the normalised values to bf16 before rotating; bound = that
    # rounding of each pair member plus the final rounding
    qpre = bf16_to_f32(oqk.qkv_norm_rope_cache(u16(qkv), H, 1e-6, u16(qw), u16(qw), np.full_like(u16(cos), 0x3F80),
                                                np.zeros_like(u16(sin)))[0])
    for got, ref, pre in ((q, oq, qpre), (k, ok, kp)):
        a, b = bf16_to_f32(u16(got)), bf16_to_f32(ref)
        pair = np.repeat(np.abs(pre[..., 0::2]) + np.abs(pre[..., 1::2]), 2, axis=-1)
        assert np.all(np.abs(a - b) <= pair * 2.0 ** -8 + np.abs(b) * 2.0 ** -8)
        assert np.mean(a == b) > 0.5  # the two roundings agree on most elements
    # a rotation the wrong way round fails the same bound
    qbad, _ = torch_path.qkv_norm_rope_cache(qkv, H, 1e-6, qw, kw, cos, -sin, ck, cv, slot)
    assert np.abs(bf16_to_f32(u16(qbad)) - bf16_to_f32(oq)).max() > 0.1


def test_block_pieces_match_pinned_oracles():
    g = torch.Generator().manual_seed(13)
    M, N, H, D = 16, 256, 2, 128
    x = torch.randn(M, N, generator=g).to(torch.bfloat16)
    shift = (0.3 * torch.randn(1, N, generator=g)).to(torch.bfloat16)
    scale = (0.3 * torch.randn(1, N, generator=g)).to(torch.bfloat16)
    # adaLN LayerNorm + modulation: the normmod oracle (pinned to torch's own layer_norm)
    y = torch_path._layernorm_modulate_ref(x, shift, scale, 1e-6)
    ref = onm.norm_scale_shift(u16(x), None, None, u16(scale), u16(shift), 0, 1e-6, "bf16")
    assert np.mean(u16(y) == ref) > 0.99
    assert np.all(np.abs(u16(y).astype(np.int32) - ref.astype(np.int32)) <= 1)
    # two-rounding text RMSNorm: the kvpack oracle, bit-exact up to the rsqrt's last ulp
    t = torch.randn(8, H, D, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    r = torch_path._rms_two_round(t, w, 1e-6)
    ref = okv.rms_two_round(u16(t), u16(w), 1e-6)
    assert np.mean(u16(r) == ref) > 0.99
    assert np.all(np.abs(u16(r).astype(np.int32) - ref.astype(np.int32)) <= 1)
    # half-table rotation: the pinned qknorm oracle's rotation of its own normalised values, exactly
    ang = torch.rand(8, D // 2, generator=g) * 6.28
    c, s = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    xt = torch.randn(8, H, D, generator=g).to(torch.bfloat16)
    o, xh = oqk.norm_rope_heads(bf16_to_f32(u16(xt)), bf16_to_f32(u16(w)), bf16_to_f32(u16(c)),
                                bf16_to_f32(u16(s)), 1e-6)
    assert np.array_equal(torch_path._rope_half(torch.from_numpy(xh), c, s).numpy(), o)
