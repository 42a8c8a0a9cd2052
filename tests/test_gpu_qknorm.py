"""GPU parity: q/k RMSNorm + RoPE (in-place reference op) and the fused QKV
split + norm + RoPE + KV-ring write, vs the oracle. Tolerance: 1e-2 relative
(the benchmark's tolerance) and at most 1 bf16 ulp from the oracle's correctly rounded result
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


def test_short_or_foreign_outputs_raise_before_launch():
    """An output view with fewer (or more) tokens than qkv rows is rejected before anything runs;
    the canary buffers stay untouched."""
    announce("fused qkv short outputs")
    import joyomni_ops as jo
    L, H, D = 24, 2, 128
    qkv, qw, kw, cos, sin = cfg1_inputs(L, H, D, 1, 4, 6, (44, 42, 42), 10000.0, 7)
    args = (qkv.to(DEV), H, 1e-6, qw.to(DEV), kw.to(DEV), cos.to(DEV), sin.to(DEV))
    full = torch.zeros(L, H, D, dtype=torch.bfloat16, device=DEV)
    canary = torch.zeros(1, L, H, D, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="holds 23 tokens, expected 24"):
        jo.fused_qkv_norm_rope_cache(*args, canary[0, :L - 1], None, None, None, 0, 0)
    with pytest.raises(RuntimeError, match="k_out holds 23 tokens"):
        jo.fused_qkv_norm_rope_cache(*args, full, canary[:, 1:], None, None, 0, 0)
    with pytest.raises(RuntimeError, match="v_out holds 25 tokens"):
        big = torch.zeros(L + 1, H * D, dtype=torch.bfloat16, device=DEV)
        jo.fused_qkv_norm_rope_cache(*args, full, None, None, None, 0, 0, v_out=big)
    with pytest.raises(RuntimeError, match="on the device of qkv"):
        jo.fused_qkv_norm_rope_cache(*args, torch.zeros(L, H, D, dtype=torch.bfloat16), None, None, None, 0, 0)
    torch.cuda.synchronize()
    assert not canary.any() and not full.any()


@pytest.mark.parametrize("pre_rope", [True, False])
def test_fused_qkv_partial_cache_write(pre_rope):
    """kv_cache_write_seq_len (dit.py:449-451): only the first n tokens reach the ring; the ring
    keeps K before RoPE or rotated (kv_cache_pre_rope, dit.py:432-433); Q/K/V outputs cover all L."""
    announce("fused qkv partial cache", pre_rope)
    import joyomni_ops as jo
    L, H, D, n = 96, 4, 128, 61
    qkv, qw, kw, cos, sin = cfg1_inputs(L, H, D, 2, 6, 8, (44, 42, 42), 10000.0, 8)
    q_out = torch.empty(L, H, D, dtype=torch.bfloat16, device=DEV)
    k_out = torch.empty_like(q_out)
    v_out = torch.empty_like(q_out)
    ck = torch.zeros(3, 70, H, D, dtype=torch.bfloat16, device=DEV)
    cv = torch.zeros_like(ck)
    jo.fused_qkv_norm_rope_cache(qkv.to(DEV), H, 1e-6, qw.to(DEV), kw.to(DEV), cos.to(DEV), sin.to(DEV),
                                 q_out, k_out, ck, cv, 2, 9, v_out=v_out, cache_tokens=n, cache_pre_rope=pre_rope)
    torch.cuda.synchronize()
    oq_, ok_, okp, ov = oqk.qkv_norm_rope_cache(u16(qkv), H, 1e-6, u16(qw), u16(kw), u16(cos), u16(sin))
    assert_close(u16(q_out), oq_, "q")
    assert_close(u16(k_out), ok_, "k")
    assert np.array_equal(u16(v_out), ov)
    assert_close(u16(ck[2, 9:9 + n]), (okp if pre_rope else ok_)[:n], "ring k")
    assert np.array_equal(u16(cv[2, 9:9 + n]), ov[:n])
    if not pre_rope:  # the rotated ring K is the attention K itself
        assert torch.equal(ck[2, 9:9 + n], k_out[:n])
    assert not ck[2, :9].any() and not ck[2, 9 + n:].any() and not cv[2, 9 + n:].any()
    assert not ck[:2].any() and not cv[:2].any()


def test_fused_qkv_cache_only_forward():
    """kv_cache_write_only (dit.py:446-459): no Q/K/V outputs, only the ring; Q is not read."""
    announce("fused qkv cache only")
    import joyomni_ops as jo
    L, H, D = 50, 4, 128
    qkv, qw, kw, cos, sin = cfg1_inputs(L, H, D, 1, 5, 10, (44, 42, 42), 10000.0, 9)
    qkv_d = qkv.to(DEV)
    qkv_d[:, : H * D] = float("nan")  # Q is not read: NaNs there cannot reach the ring
    ck = torch.zeros(2, L, H, D, dtype=torch.bfloat16, device=DEV)
    cv = torch.zeros_like(ck)
    jo.fused_qkv_norm_rope_cache(qkv_d, H, 1e-6, qw.to(DEV), kw.to(DEV), cos.to(DEV), sin.to(DEV),
                                 None, None, ck, cv, 1, 0)
    torch.cuda.synchronize()
    _, _, okp, ov = oqk.qkv_norm_rope_cache(u16(qkv), H, 1e-6, u16(qw), u16(kw), u16(cos), u16(sin))
    assert_close(u16(ck[1]), okp, "ring k")
    assert np.array_equal(u16(cv[1]), ov) and not ck[0].any()


def test_fused_qkv_on_source_id_tables_at_production_geometry():
    """Composed [current | ref-video] tables (dit.py:1093-1155, config.py:29-37) at the reference's
    480x832 chunk: 2 x 30 x 52 tokens per segment, 32 heads, RoPE 16/56/56 theta 256, role theta 256
    over 128 dims; the first 3120 tokens (the current chunk) go to the ring."""
    from joyomni_ops import rope
    announce("fused qkv source-id tables")
    import joyomni_ops as jo
    frames, hh, ww, H, D = 2, 30, 52, 32, 128
    n_cur = frames * hh * ww
    L = 2 * n_cur
    g = gen(10)
    qkv = bf(torch.randn(L, 3 * H * D, generator=g))
    qw = bf(1 + 0.1 * torch.randn(D, generator=g))
    kw = bf(1 + 0.1 * torch.randn(D, generator=g))
    cos, sin = rope.visual_rope_half_tables((frames, hh, ww), frames)
    _, _, cb, sb = orope.visual_half_tables((frames, hh, ww), frames)
    assert np.all(np.abs(u16(cos).astype(np.int32) - cb.astype(np.int32)) <= 1)
    q_out = torch.empty(L, H, D, dtype=torch.bfloat16, device=DEV)
    k_out = torch.empty_like(q_out)
    ck = torch.zeros(2, n_cur, H, D, dtype=torch.bfloat16, device=DEV)
    cv = torch.zeros_like(ck)
    jo.fused_qkv_norm_rope_cache(qkv.to(DEV), H, 1e-6, qw.to(DEV), kw.to(DEV), cos.to(DEV), sin.to(DEV),
                                 q_out, k_out, ck, cv, 0, 0, cache_tokens=n_cur)
    torch.cuda.synchronize()
    toks = np.sort(np.random.default_rng(1).choice(L, 384, replace=False))
    toks[0], toks[-1] = 0, L - 1
    ti = torch.from_numpy(toks)
    oq_, ok_, okp, _ = oqk.qkv_norm_rope_cache(u16(qkv[ti]), H, 1e-6, u16(qw), u16(kw), cb[toks], sb[toks])
    tid = ti.to(DEV)
    assert_close(u16(q_out[tid]), oq_, "q")
    assert_close(u16(k_out[tid]), ok_, "k")
    cur = toks < n_cur
    assert_close(u16(ck[0][tid[torch.from_numpy(cur)]]), okp[cur], "ring k (current chunk)")
    assert torch.equal(cv[0].reshape(n_cur, -1), qkv.to(DEV)[:n_cur, 2 * H * D:])
