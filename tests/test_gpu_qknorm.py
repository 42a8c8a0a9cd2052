"""GPU parity: q/k RMSNorm + RoPE (in-place reference op) and the fused QKV
split + norm + RoPE + KV-ring write, vs the oracle. Tolerance: 1e-2 relative
(BASELINE) and at most 1 bf16 ulp from the oracle's correctly rounded result
for all but 0.1% of elements; V copies and untouched ring slots bit-exact."""
import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, gen, u16
from oracle import qknorm as oqk
from oracle import rope as orope
from oracle.fp8 import bf16_to_f32

pytestmark = pytest.mark.gpu


def assert_close(got_bits, exp_bits, what):
    a = bf16_to_f32(got_bits).astype(np.float64)
    b = bf16_to_f32(exp_bits).astype(np.float64)
    rel = np.abs(a - b).max() / max(np.abs(b).max(), 1e-12)
    assert rel <= 1e-2, f"{what}: relative error {rel:.3e}"
    ulp = np.abs(got_bits.astype(np.int32) - exp_bits.astype(np.int32))
    same_sign = (got_bits >> 15) == (exp_bits >> 15)
    far = (ulp > 1) & same_sign & (np.abs(b) > 1e-3)
    assert np.count_nonzero(far) <= 1e-3 * a.size, f"{what}: {np.count_nonzero(far)} values > 1 ulp"


def bf(x):
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("B,L,H,D,kpre", [(1, 128, 8, 128, True), (1, 128, 8, 128, False),
                                          (2, 33, 5, 64, True), (1, 17, 3, 256, True),
                                          (1, 1560, 32, 128, True)])
def test_paired_inplace_op(B, L, H, D, kpre):
    announce("qk_norm_rope paired", B, L, H, D, kpre)
    import joyomni_ops as jo
    g = gen(L * H + D)
    q = bf(torch.randn(B, L * H, D, generator=g))
    k = bf(torch.randn(B, L * H, D, generator=g))
    qw, kw = bf(torch.randn(D, generator=g)), bf(torch.randn(D, generator=g))
    cos, sin = bf(torch.randn(L, D // 2, generator=g)), bf(torch.randn(L, D // 2, generator=g))
    qd, kd = q.to(DEV), k.to(DEV)
    kp = torch.empty_like(kd) if kpre else None
    jo.fused_qk_norm_rope_3d_paired(qd, kd, L, H, 1e-6, qw.to(DEV), kw.to(DEV), cos.to(DEV),
                                    sin.to(DEV), kp)
    torch.cuda.synchronize()
    oq_, ok_, okp = oqk.qk_norm_rope_paired(u16(q), u16(k), L, H, 1e-6, u16(qw), u16(kw), u16(cos), u16(sin))
    assert_close(u16(qd), oq_, "q")
    assert_close(u16(kd), ok_, "k")
    if kpre:
        assert_close(u16(kp), okp, "k_pre_rope")


def cfg1_inputs(L, H, D, frames, hh, ww, dims, theta, seed):
    g = gen(seed)
    qkv = bf(torch.randn(L, 3 * H * D, generator=g))
    qw = bf(1 + 0.1 * torch.randn(D, generator=g))
    kw = bf(1 + 0.1 * torch.randn(D, generator=g))
    _, _, cb, sb = orope.rope_half_tables(list(range(frames)), hh, ww, dims, theta)
    cos = torch.from_numpy(cb.view(np.int16)).view(torch.bfloat16)
    sin = torch.from_numpy(sb.view(np.int16)).view(torch.bfloat16)
    return qkv, qw, kw, cos, sin


@pytest.mark.parametrize("case", ["baseline_cfg1", "reference_720p_shape"])
def test_fused_qkv_cache_full_size(case):
    import joyomni_ops as jo
    if case == "baseline_cfg1":
        T, hh, ww, H, D, dims, theta, slots, slot = 3, 45, 80, 40, 128, (44, 42, 42), 10000.0, 4, 1
    else:  # reference production geometry: 32 heads, RoPE 16/56/56, theta 256
        T, hh, ww, H, D, dims, theta, slots, slot = 1, 39, 40, 32, 128, (16, 56, 56), 256.0, 4, 3
    L = T * hh * ww
    announce("fused qkv cache", case, L, H, D)
    qkv, qw, kw, cos, sin = cfg1_inputs(L, H, D, T, hh, ww, dims, theta, L)
    qkv_d = qkv.to(DEV)
    q_out = torch.empty(L, H, D, dtype=torch.bfloat16, device=DEV)
    k_out = torch.empty_like(q_out)
    ck = torch.zeros(slots, L, H, D, dtype=torch.bfloat16, device=DEV)
    cv = torch.zeros_like(ck)
    jo.fused_qkv_norm_rope_cache(qkv_d, H, 1e-6, qw.to(DEV), kw.to(DEV), cos.to(DEV), sin.to(DEV),
                                 q_out, k_out, ck, cv, slot, 0)
    torch.cuda.synchronize()
    E = H * D
    assert torch.equal(cv[slot].reshape(L, E), qkv_d[:, 2 * E:]), "V ring copy differs"
    for s in range(slots):
        if s != slot:
            assert not ck[s].any() and not cv[s].any(), f"slot {s} written"
    toks = np.sort(np.random.default_rng(0).choice(L, 512, replace=False))
    toks[-1] = L - 1
    ti = torch.from_numpy(toks)
    oq_, ok_, okp, ov = oqk.qkv_norm_rope_cache(u16(qkv[ti]), H, 1e-6, u16(qw), u16(kw),
                                                u16(cos[ti]), u16(sin[ti]))
    tid = ti.to(DEV)
    assert_close(u16(q_out[tid]), oq_, "q")
    assert_close(u16(k_out[tid]), ok_, "k")
    assert_close(u16(ck[slot][tid]), okp, "k_pre (cache)")


def test_fused_qkv_strided_outputs_and_offsets():
    """q/k land inside larger joint-attention buffers; cache rows at an offset."""
    announce("fused qkv strided")
    import joyomni_ops as jo
    L, H, D = 77, 6, 128
    qkv, qw, kw, cos, sin = cfg1_inputs(L, H, D, 1, 7, 11, (44, 42, 42), 10000.0, 5)
    qkv_wide = torch.zeros(L, 3 * H * D + 64, dtype=torch.bfloat16)
    qkv_wide[:, : 3 * H * D] = qkv
    qkv_d = qkv_wide.to(DEV)[:, : 3 * H * D]
    joint_q = torch.zeros(L + 20, H, D, dtype=torch.bfloat16, device=DEV)
    joint_k = torch.zeros(L + 30, H, D, dtype=torch.bfloat16, device=DEV)
    ck = torch.zeros(2, 100, H, D, dtype=torch.bfloat16, device=DEV)
    cv = torch.zeros_like(ck)
    jo.fused_qkv_norm_rope_cache(qkv_d, H, 1e-6, qw.to(DEV), kw.to(DEV), cos.to(DEV), sin.to(DEV),
                                 joint_q[:L], joint_k[30:], ck, cv, 0, 10)
    torch.cuda.synchronize()
    oq_, ok_, okp, ov = oqk.qkv_norm_rope_cache(u16(qkv), H, 1e-6, u16(qw), u16(kw), u16(cos), u16(sin))
    assert_close(u16(joint_q[:L]), oq_, "q")
    assert_close(u16(joint_k[30:]), ok_, "k")
    assert not joint_q[L:].any() and not joint_k[:30].any()
    assert_close(u16(ck[0, 10:10 + L]), okp, "k_pre")
    assert np.array_equal(u16(cv[0, 10:10 + L]), ov)
    assert not ck[0, :10].any() and not ck[0, 10 + L:].any() and not ck[1].any()


def test_fused_without_cache_or_k_out():
    announce("fused qkv no cache")
    import joyomni_ops as jo
    L, H, D = 40, 4, 64
    qkv, qw, kw, cos, sin = cfg1_inputs(L, H, D, 1, 5, 8, (24, 20, 20), 10000.0, 6)
    q_out = torch.empty(L, H, D, dtype=torch.bfloat16, device=DEV)
    jo.fused_qkv_norm_rope_cache(qkv.to(DEV), H, 1e-6, qw.to(DEV), kw.to(DEV), cos.to(DEV), sin.to(DEV),
                                 q_out, None, None, None, 0, 0)
    torch.cuda.synchronize()
    oq_, _, _, _ = oqk.qkv_norm_rope_cache(u16(qkv), H, 1e-6, u16(qw), u16(kw), u16(cos), u16(sin))
    assert_close(u16(q_out), oq_, "q")
