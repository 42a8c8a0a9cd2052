"""Pins the joint-pack / cached-pack oracle against the reference test's closed
forms (joyomni_ops/tests/test_parity_light.py:136-199) evaluated with torch CPU
ops, and against special cases whose result is known exactly."""
import numpy as np
import torch

from oracle import kvpack as okv
from oracle.fp8 import bf16_to_f32, f32_to_bf16


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def torch_norm_two_round(x, w, eps=1e-6):
    # test_parity_light.py:159-164: fp32 normalise, cast to bf16, multiply by the bf16 weight
    xf = x.float()
    normalized = (xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps)).to(torch.bfloat16)
    return normalized * w


def torch_norm_one_round(x, w, eps=1e-6):
    xf = x.float()
    return (xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps) * w.float()).to(torch.bfloat16)


def test_joint_pack_matches_reference_closed_form():
    g = torch.Generator().manual_seed(0)
    img_len, txt_len, cache_len, H, D = 17, 11, 9, 4, 128  # the reference test's geometry
    img_qkv = torch.randn(img_len, 3, H, D, generator=g).to(torch.bfloat16)
    txt_qkv = torch.randn(txt_len, 3, H, D, generator=g).to(torch.bfloat16)
    ck = torch.randn(cache_len, H, D, generator=g).to(torch.bfloat16)
    cv = torch.randn(cache_len, H, D, generator=g).to(torch.bfloat16)
    qw = torch.randn(D, generator=g).to(torch.bfloat16)
    kw = torch.randn(D, generator=g).to(torch.bfloat16)
    iq, ik, iv = img_qkv.unbind(1)
    tq, tk, tv = txt_qkv.unbind(1)
    oq, ok, ov = okv.joint_qkv_pack(u16(iq), u16(ik), u16(iv), u16(tq), u16(tk), u16(tv), u16(ck), u16(cv),
                                    u16(qw), u16(kw), 1e-6)
    ref_q = torch.cat((iq, torch_norm_two_round(tq, qw)), 0)
    ref_k = torch.cat((ck, ik, torch_norm_two_round(tk, kw)), 0)
    ref_v = torch.cat((cv, iv, tv), 0)
    assert np.array_equal(ov, u16(ref_v))
    # copied rows bit-exact
    assert np.array_equal(oq[:img_len], u16(iq)) and np.array_equal(ok[: cache_len + img_len],
                                                                      u16(torch.cat((ck, ik), 0)))
    # normalised rows: bit-exact except where the fp32 sum order moves a bf16 tie,
    # while a one-rounding norm (a plausible mistake) differs far more often
    for got, ref, one in ((oq[img_len:], ref_q[img_len:], torch_norm_one_round(tq, qw)),
                          (ok[cache_len + img_len:], ref_k[cache_len + img_len:], torch_norm_one_round(tk, kw))):
        miss = np.count_nonzero(got != u16(ref))
        miss_one = np.count_nonzero(u16(one) != u16(ref))
        assert miss <= 2e-3 * got.size, miss
        assert miss_one >= 20 * max(miss, 1), (miss, miss_one)
        assert np.all(np.abs(got.astype(np.int32) - u16(ref).astype(np.int32)) <= 1)


def test_joint_pack_without_cache_and_segment_order():
    L, H, D = 3, 2, 128
    mk = lambda base: f32_to_bf16(np.full((L, H, D), base, np.float32))  # noqa: E731
    w = f32_to_bf16(np.ones(D, np.float32))
    q, k, v = okv.joint_qkv_pack(mk(1), mk(2), mk(3), mk(4), mk(5), mk(6), None, None, w, w, 0.0)
    assert q.shape == (2 * L, H, D) and k.shape == (2 * L, H, D)
    # a constant row with unit weight normalises to exactly 1.0 when eps = 0
    assert np.all(bf16_to_f32(q[L:]) == 1.0) and np.all(bf16_to_f32(k[L:]) == 1.0)
    assert np.all(bf16_to_f32(q[:L]) == 1) and np.all(bf16_to_f32(k[:L]) == 2)
    assert np.all(bf16_to_f32(v[:L]) == 3) and np.all(bf16_to_f32(v[L:]) == 6)


def test_cached_pack_matches_reference_closed_form_bit_exact():
    g = torch.Generator().manual_seed(1)
    len0, len1, H, D = 13, 7, 4, 128  # the reference test's geometry
    k0 = torch.randn(len0, H, D, generator=g).to(torch.bfloat16)
    v0 = torch.randn(len0, H, D, generator=g).to(torch.bfloat16)
    k1 = torch.randn(len1, H, D, generator=g).to(torch.bfloat16)
    v1 = torch.randn(len1, H, D, generator=g).to(torch.bfloat16)
    cos = torch.randn(len0 + len1, D // 2, generator=g).repeat_interleave(2, dim=-1).contiguous()
    sin = torch.randn(len0 + len1, D // 2, generator=g).repeat_interleave(2, dim=-1).contiguous()
    ok, ov = okv.cached_kv_pack(u16(k0), u16(v0), u16(k1), u16(v1), cos.numpy(), sin.numpy())
    # test_parity_light.py:190-197
    src = torch.cat((k0, k1), 0).float()
    pairs = src.reshape(len0 + len1, H, D // 2, 2)
    rotated = torch.stack((-pairs[..., 1], pairs[..., 0]), dim=-1).flatten(-2)
    ref_k = (src * cos.view(-1, 1, D) + rotated * sin.view(-1, 1, D)).to(torch.bfloat16)
    assert np.array_equal(ok, u16(ref_k))
    assert np.array_equal(ov, u16(torch.cat((v0, v1), 0)))


def test_cached_pack_identity_and_quarter_turn():
    rng = np.random.default_rng(3)
    L, H, D = 5, 3, 128
    k = f32_to_bf16(rng.standard_normal((L, H, D)).astype(np.float32))
    v = f32_to_bf16(rng.standard_normal((L, H, D)).astype(np.float32))
    one, zero = np.ones((L, D), np.float32), np.zeros((L, D), np.float32)
    ok, ov = okv.cached_kv_pack(k, v, None, None, one, zero)
    assert np.array_equal(ok, k) and np.array_equal(ov, v)
    ok, _ = okv.cached_kv_pack(k, v, None, None, zero, one)  # rotate by +90 degrees
    kf = bf16_to_f32(k)
    assert np.array_equal(bf16_to_f32(ok[..., 0::2]), -kf[..., 1::2])
    assert np.array_equal(bf16_to_f32(ok[..., 1::2]), kf[..., 0::2])
    # the odd table column is never read (kernel indexing fused_joint_qkv_pack.cu:207-212)
    junk = one.copy()
    junk[:, 1::2] = 7.0
    ok2, _ = okv.cached_kv_pack(k, v, None, None, junk, zero)
    assert np.array_equal(ok2, k)
