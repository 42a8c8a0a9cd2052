"""GPU parity: fused_joint_qkv_pack and fused_cached_kv_pack (HIP kernels) vs the
oracle. Copied rows (img Q/K, cached K/V, every V) must be bit-exact; text-norm
and rotated rows within 1e-2 relative (the benchmark's tolerance) and at most 1 bf16 ulp from the
oracle on all but 0.1 % of elements."""
import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, gen, u16
from oracle import kvpack as okv
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


def sq(t):
    """[1, L, H, D] -> [L, H, D] numpy bits."""
    return u16(t[0])


@pytest.mark.parametrize("cache", [True, False])
def test_joint_pack_reference_geometry(cache):
    """The reference test's case (test_parity_light.py:136-173): Q/K/V sliced from
    interleaved projections so every input is a strided view."""
    import joyomni_ops as jo
    announce("joint pack reference geometry", cache)
    g = gen(7)
    img_len, txt_len, cache_len, H, D = 17, 11, 9, 4, 128
    img_qkv = bf(torch.randn(1, img_len, 3, H, D, generator=g))
    txt_qkv = bf(torch.randn(1, txt_len, 3, H, D, generator=g))
    ck = bf(torch.randn(1, cache_len, H, D, generator=g))
    cv = bf(torch.randn(1, cache_len, H, D, generator=g))
    qw, kw = bf(torch.randn(D, generator=g)), bf(torch.randn(D, generator=g))
    di, dt = img_qkv.to(DEV), txt_qkv.to(DEV)
    iq, ik, iv = di.unbind(2)
    tq, tk, tv = dt.unbind(2)
    args = (ck.to(DEV), cv.to(DEV)) if cache else (None, None)
    oq, ok, ov = jo.fused_joint_qkv_pack(iq, ik, iv, tq, tk, tv, *args, qw.to(DEV), kw.to(DEV), 1e-6)
    torch.cuda.synchronize()
    h_iq, h_ik, h_iv = img_qkv.unbind(2)
    h_tq, h_tk, h_tv = txt_qkv.unbind(2)
    eq, ek, ev = okv.joint_qkv_pack(sq(h_iq), sq(h_ik), sq(h_iv), sq(h_tq), sq(h_tk), sq(h_tv),
                                    sq(ck) if cache else None, sq(cv) if cache else None,
                                    u16(qw), u16(kw), 1e-6)
    c = cache_len if cache else 0
    assert oq.shape == (1, img_len + txt_len, H, D) and ok.shape == (1, c + img_len + txt_len, H, D)
    assert np.array_equal(sq(ov), ev), "V pack differs"
    assert np.array_equal(sq(oq)[:img_len], eq[:img_len]), "img Q copy differs"
    assert np.array_equal(sq(ok)[: c + img_len], ek[: c + img_len]), "cache/img K copy differs"
    assert_close(sq(oq)[img_len:], eq[img_len:], "txt Q norm")
    assert_close(sq(ok)[c + img_len:], ek[c + img_len:], "txt K norm")


def test_joint_pack_unaligned_strides():
    """Head stride 129 elements: the kernel's 2-byte path."""
    import joyomni_ops as jo
    announce("joint pack unaligned")
    g = gen(8)
    L, T, C, H, D = 5, 3, 2, 3, 128
    base = lambda n: bf(torch.randn(1, n, H, D + 1, generator=g))[..., :D]  # noqa: E731
    ins = [base(L), base(L), base(L), base(T), base(T), base(T), base(C), base(C)]
    qw, kw = bf(torch.randn(D, generator=g)), bf(torch.randn(D, generator=g))
    dev = [t.to(DEV) for t in ins]
    oq, ok, ov = jo.fused_joint_qkv_pack(*dev, qw.to(DEV), kw.to(DEV), 1e-6)
    torch.cuda.synchronize()
    eq, ek, ev = okv.joint_qkv_pack(*[sq(t) for t in ins], u16(qw), u16(kw), 1e-6)
    assert np.array_equal(sq(ov), ev)
    assert np.array_equal(sq(oq)[:L], eq[:L]) and np.array_equal(sq(ok)[: C + L], ek[: C + L])
    assert_close(sq(oq)[L:], eq[L:], "txt Q norm")
    assert_close(sq(ok)[C + L:], ek[C + L:], "txt K norm")


def test_joint_pack_baseline_size():
    """cfg-4 geometry: 10800 video + 512 condition tokens, 40x128 heads, 3 cached chunks
    (32400 tokens) read from ring slots, video q/k/v straight from the QKV GEMM row."""
    import joyomni_ops as jo
    announce("joint pack baseline size")
    L, T, H, D, slots = 10800, 512, 40, 128, 4
    C = 3 * L
    E = H * D
    g = gen(9)
    img_qkv = bf(torch.randn(L, 3 * E, generator=g)).to(DEV)
    txt_qkv = bf(torch.randn(T, 3 * E, generator=g))
    ring_k = bf(torch.randn(slots, L, H, D, generator=g)).to(DEV)
    ring_v = bf(torch.randn(slots, L, H, D, generator=g)).to(DEV)
    qw, kw = bf(1 + 0.1 * torch.randn(D, generator=g)), bf(1 + 0.1 * torch.randn(D, generator=g))
    i4 = img_qkv.view(1, L, 3, H, D)
    t4 = txt_qkv.to(DEV).view(1, T, 3, H, D)
    ck = ring_k[:3].reshape(1, C, H, D)
    cv = ring_v[:3].reshape(1, C, H, D)
    oq, ok, ov = jo.fused_joint_qkv_pack(i4[:, :, 0], i4[:, :, 1], i4[:, :, 2], t4[:, :, 0], t4[:, :, 1],
                                         t4[:, :, 2], ck, cv, qw.to(DEV), kw.to(DEV), 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(ov[0, :C], cv[0]) and torch.equal(ov[0, C:C + L], i4[0, :, 2])
    assert torch.equal(ov[0, C + L:], t4[0, :, 2])
    assert torch.equal(ok[0, :C], ck[0]) and torch.equal(ok[0, C:C + L], i4[0, :, 1])
    assert torch.equal(oq[0, :L], i4[0, :, 0])
    t3 = txt_qkv.view(T, 3, H, D)
    eq = okv.rms_two_round(u16(t3[:, 0]), u16(qw), 1e-6)
    ek = okv.rms_two_round(u16(t3[:, 1]), u16(kw), 1e-6)
    assert_close(u16(oq[0, L:]), eq, "txt Q norm")
    assert_close(u16(ok[0, C + L:]), ek, "txt K norm")


@pytest.mark.parametrize("two", [True, False])
def test_cached_pack_reference_geometry(two):
    """The reference test's case (test_parity_light.py:176-199), repeat_interleave tables."""
    import joyomni_ops as jo
    announce("cached pack reference geometry", two)
    g = gen(10)
    len0, len1, H, D = 13, 7 if two else 0, 4, 128
    k0, v0 = bf(torch.randn(1, len0, H, D, generator=g)), bf(torch.randn(1, len0, H, D, generator=g))
    k1, v1 = bf(torch.randn(1, max(len1, 1), H, D, generator=g)), bf(torch.randn(1, max(len1, 1), H, D, generator=g))
    cos = torch.randn(len0 + len1, D // 2, generator=g).repeat_interleave(2, dim=-1).contiguous()
    sin = torch.randn(len0 + len1, D // 2, generator=g).repeat_interleave(2, dim=-1).contiguous()
    seg1 = (k1.to(DEV), v1.to(DEV)) if two else (None, None)
    ok, ov = jo.fused_cached_kv_pack(k0.to(DEV), v0.to(DEV), *seg1, cos.to(DEV), sin.to(DEV))
    torch.cuda.synchronize()
    ek, ev = okv.cached_kv_pack(sq(k0), sq(v0), sq(k1) if two else None, sq(v1) if two else None,
                                cos.numpy(), sin.numpy())
    assert ok.shape == (1, len0 + len1, H, D)
    assert np.array_equal(sq(ov), ev), "V pack differs"
    assert_close(sq(ok), ek, "rotated K")


def test_cached_pack_from_ring_slots_baseline_size():
    """Two cached chunks read straight out of KV-ring slots (pre-RoPE K), rotated with
    fp32 full-width tables of the real 3-D RoPE at window-relative positions."""
    import joyomni_ops as jo
    announce("cached pack ring slots baseline size")
    L, H, D, slots = 10800, 40, 128, 4
    g = gen(11)
    ring_k = bf(torch.randn(slots, L, H, D, generator=g)).to(DEV)
    ring_v = bf(torch.randn(slots, L, H, D, generator=g)).to(DEV)
    # chunk 0 at frames 0..2, chunk 1 at frames 3..5 (window-relative temporal ids)
    c32, s32, _, _ = orope.rope_half_tables(list(range(6)), 45, 80, (44, 42, 42), 10000.0)
    cos = torch.from_numpy(np.repeat(c32, 2, axis=1)).contiguous()
    sin = torch.from_numpy(np.repeat(s32, 2, axis=1)).contiguous()
    k0, v0 = ring_k[2][None], ring_v[2][None]
    k1, v1 = ring_k[0][None], ring_v[0][None]
    ok, ov = jo.fused_cached_kv_pack(k0, v0, k1, v1, cos.to(DEV), sin.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(ov[0, :L], ring_v[2]) and torch.equal(ov[0, L:], ring_v[0])
    toks = np.sort(np.random.default_rng(0).choice(2 * L, 384, replace=False))
    toks[-1] = 2 * L - 1
    kcat = torch.cat((ring_k[2], ring_k[0]), 0)[torch.from_numpy(toks).to(DEV)]
    ek = okv.rotate_pairs(u16(kcat), cos.numpy()[toks], sin.numpy()[toks])
    assert_close(u16(ok[0][torch.from_numpy(toks).to(DEV)]), ek, "rotated K")


def test_joint_operands_in_place_equal_reference_sequence():
    """The block's in-place assembly of the joint attention operands -- the fused QKV op
    writing the video rows (v_out), fused_cached_kv_pack_out rotating two ring slots into
    the head of K / V, fused_text_qkv_pack writing the tails -- is byte-identical to the
    reference sequence (fused QKV op into separate q/k, fused_cached_kv_pack, then
    fused_joint_qkv_pack), writes every row (NaN-filled buffers) and leaves the same ring."""
    import joyomni_ops as jo
    announce("joint operands in place")
    hh, ww, T, H, D, slots = 30, 40, 64, 40, 128, 3
    L, E, C = hh * ww, H * D, 2 * hh * ww
    g = gen(12)
    img_qkv = bf(torch.randn(L, 3 * E, generator=g)).to(DEV)
    txt_qkv = bf(torch.randn(T, 3 * E, generator=g)).to(DEV)
    ring_k = bf(torch.randn(slots, L, H, D, generator=g)).to(DEV)
    ring_v = bf(torch.randn(slots, L, H, D, generator=g)).to(DEV)
    qn, kn, tqn, tkn = (bf(1 + 0.1 * torch.randn(D, generator=g)).to(DEV) for _ in range(4))
    _, _, cb, sb = orope.rope_half_tables([2], hh, ww, (44, 42, 42), 10000.0)
    cos_h = torch.from_numpy(cb.view(np.int16)).view(torch.bfloat16).to(DEV)
    sin_h = torch.from_numpy(sb.view(np.int16)).view(torch.bfloat16).to(DEV)
    c32, s32, _, _ = orope.rope_half_tables([0, 1], hh, ww, (44, 42, 42), 10000.0)
    cos_f = torch.from_numpy(np.repeat(c32, 2, axis=1)).contiguous().to(DEV)
    sin_f = torch.from_numpy(np.repeat(s32, 2, axis=1)).contiguous().to(DEV)
    i4, t4 = img_qkv.view(1, L, 3, H, D), txt_qkv.view(1, T, 3, H, D)
    # reference sequence
    rk, rv = ring_k.clone(), ring_v.clone()
    q_img, k_img = (torch.empty(L, H, D, dtype=torch.bfloat16, device=DEV) for _ in range(2))
    jo.fused_qkv_norm_rope_cache(img_qkv, H, 1e-6, qn, kn, cos_h, sin_h, q_img, k_img, rk, rv, 2, 0)
    ck, cv = jo.fused_cached_kv_pack(rk[0][None], rv[0][None], rk[1][None], rv[1][None], cos_f, sin_f)
    Q, K, V = jo.fused_joint_qkv_pack(q_img[None], k_img[None], i4[:, :, 2], t4[:, :, 0], t4[:, :, 1],
                                      t4[:, :, 2], ck, cv, tqn, tkn, 1e-6)
    # in place
    q = torch.full((1, L + T, H, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    k = torch.full((1, C + L + T, H, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    v = torch.full_like(k, float("nan"))
    jo.fused_qkv_norm_rope_cache(img_qkv, H, 1e-6, qn, kn, cos_h, sin_h, q[0, :L], k[0, C:C + L], ring_k, ring_v,
                                 2, 0, v_out=v[0, C:C + L])
    jo.fused_cached_kv_pack_out(ring_k[0][None], ring_v[0][None], ring_k[1][None], ring_v[1][None], cos_f, sin_f,
                                k[:, :C], v[:, :C])
    jo.fused_text_qkv_pack(t4[:, :, 0], t4[:, :, 1], t4[:, :, 2], tqn, tkn, 1e-6, q[:, L:], k[:, C + L:],
                           v[:, C + L:])
    torch.cuda.synchronize()
    assert torch.equal(q, Q) and torch.equal(k, K) and torch.equal(v, V)
    assert torch.equal(ring_k, rk) and torch.equal(ring_v, rv)


def test_pack_argument_errors():
    import joyomni_ops as jo
    announce("pack argument errors")
    x = torch.zeros(1, 4, 2, 128, dtype=torch.bfloat16, device=DEV)
    w = torch.ones(128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="both be present or both be absent"):
        jo.fused_joint_qkv_pack(x, x, x, x, x, x, x, None, w, w, 1e-6)
    with pytest.raises(RuntimeError, match="image Q/K/V lengths must match"):
        jo.fused_joint_qkv_pack(x, x[:, :3], x, x, x, x, None, None, w, w, 1e-6)
    c = torch.ones(4, 128, device=DEV)
    with pytest.raises(RuntimeError, match="key1 and value1"):
        jo.fused_cached_kv_pack(x, x, x, None, c, c)
    with pytest.raises(RuntimeError, match="total_cache_len"):
        jo.fused_cached_kv_pack(x, x, x, x, c, c)
    with pytest.raises(RuntimeError, match=r"out_k must be \[1, 4, 2, 128\]"):
        jo.fused_cached_kv_pack_out(x, x, None, None, c, c, x[:, :3], x)
    with pytest.raises(RuntimeError, match="out_v must be contiguous"):
        wide = torch.zeros(1, 4, 4, 128, dtype=torch.bfloat16, device=DEV)
        jo.fused_text_qkv_pack(x, x, x, w, w, 1e-6, x, x, wide[:, :, :2])
