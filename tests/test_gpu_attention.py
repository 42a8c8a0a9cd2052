"""GPU parity: joint-attention core (joyomni_ops.sdpa_attention, joy_attention_fwd) vs the
float64 oracle (oracle/attention.py, restating dit.py:154-167).

Tolerance (bf16 output, probabilities rounded to bf16 for the P V product as in bf16
flash attention): |out - ref| <= 2^-8 * (max_j |v[j, h, :]| + |ref|) per element. Exact
cases (single key, identical keys over small-integer values) are checked bit for bit."""
import math

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, gen, u16
from oracle import attention as oa
from oracle.fp8 import bf16_to_f32, f32_to_bf16

pytestmark = pytest.mark.gpu


def _inputs(Lq, Lk, H, seed, scale=1.0):
    g = gen(seed)
    q = (torch.randn(Lq, H, 128, generator=g) * scale).to(torch.bfloat16)
    k = (torch.randn(Lk, H, 128, generator=g) * scale).to(torch.bfloat16)
    v = torch.randn(Lk, H, 128, generator=g).to(torch.bfloat16)
    return q, k, v


def _run(q, k, v, scale=None):
    import joyomni_ops as jo
    out = jo.sdpa_attention(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), scale)
    torch.cuda.synchronize()
    return out[0]


def _check(out, q, k, v, what, scale=None, rows=None):
    ref = oa.sdpa(u16(q if rows is None else q[rows]), u16(k), u16(v), scale)
    got = bf16_to_f32(u16(out if rows is None else out[torch.from_numpy(rows).to(out.device)]))
    vmax = np.abs(bf16_to_f32(u16(v))).max(axis=0)  # [H, D] -> per head max below
    tol = 2.0 ** -8 * (vmax.max(axis=-1)[None, :, None] + np.abs(ref))
    err = np.abs(got - ref)
    assert (err <= tol).all(), f"{what}: {np.count_nonzero(err > tol)} elements beyond tolerance, max err {err.max():.3e}"
    return err.max()


@pytest.mark.parametrize("Lq,Lk,H", [(1, 1, 1), (5, 3, 2), (128, 64, 1), (130, 65, 2), (300, 700, 3),
                                     (257, 129, 4), (64, 1000, 1), (33, 32, 2), (40, 33, 1), (70, 96, 2)])
def test_random_shapes(Lq, Lk, H):
    announce("attention random", Lq, Lk, H)
    q, k, v = _inputs(Lq, Lk, H, Lq * 31 + Lk)
    _check(_run(q, k, v), q, k, v, f"{Lq}x{Lk}x{H}")


@pytest.mark.parametrize("Lq,H", [(330, 7), (256, 3), (225, 2), (40, 9)])
def test_workgroups_straddling_heads(Lq, H):
    """Workgroups take 8 consecutive 32-query blocks of the head-major block list, so one
    workgroup can hold the end of one head and the start of the next (330 queries: 11 blocks per
    head), or padding blocks past Lq (40 queries: 2 of 8 blocks); every row of every head is
    checked."""
    announce("attention straddling heads", Lq, H)
    q, k, v = _inputs(Lq, 300, H, Lq + 17 * H)
    _check(_run(q, k, v), q, k, v, f"{Lq}x300x{H}")


def test_peaked_scores_and_explicit_scale():
    """Large-magnitude q/k (peaked softmax, exp2 range) and a non-default scale."""
    announce("attention peaked")
    q, k, v = _inputs(200, 333, 2, 7, scale=3.0)
    _check(_run(q, k, v), q, k, v, "peaked")
    _check(_run(q, k, v, 0.02), q, k, v, "scale 0.02", scale=0.02)


def test_running_max_jumps_across_tiles():
    """Scores that jump between 64-key tiles, so that the softmax's first pass against the running
    max fails its check and the max-based pass takes over in every way it can: a jump of about 5
    and 7.9 (log2 units, below the slack of 8: the sum check fails, the running max stays), of
    about 12.7 (the running max moves and O is rescaled), a drop of about 20 (tiny probabilities,
    the first pass holds) and of about 200 (probabilities against the old max overflow to inf).
    Key rows carry their level in dimension 0 and queries 4 there, on top of small random parts;
    the last tile is partial (17 keys)."""
    announce("attention running-max jumps")
    g = gen(41)
    Lq, H, tiles = 96, 2, 11
    Lk = 64 * (tiles - 1) + 17
    q = torch.randn(Lq, H, 128, generator=g) * 0.1
    k = torch.randn(Lk, H, 128, generator=g) * 0.1
    v = torch.randn(Lk, H, 128, generator=g)
    q[:, :, 0] = 4.0
    # level of dimension 0 per tile: scores move by 4 * level / sqrt(128) * log2(e) ~ 0.51 * level
    levels = {0: 0.0, 3: 10.0, 4: 15.5, 6: 25.0, 7: -40.0, 8: 400.0, 9: 0.0, 10: 401.0}
    for t, lv in levels.items():
        rows = slice(64 * t, min(64 * (t + 1), Lk))
        k[rows, 0, 0] = lv
        k[rows, 1, 0] = -lv if t in (3, 7) else lv  # head 1: drops where head 0 jumps
    q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
    out = _run(q, k, v)
    assert torch.isfinite(out.float()).all()
    _check(out, q, k, v, "running-max jumps")


def test_single_key_is_exact():
    announce("attention single key")
    q, k, v = _inputs(77, 1, 3, 11)
    assert np.array_equal(u16(_run(q, k, v)), np.broadcast_to(u16(v), (77, 3, 128)))


@pytest.mark.parametrize("Lk", [64, 40])
def test_identical_keys_exact_mean(Lk):
    """Lk identical keys (a full tile; a tile whose second 32-key half is partly past the end):
    every probability is exactly 1, small-integer values sum exactly, so the output is the bf16
    rounding of their mean."""
    announce("attention identical keys", Lk)
    rng = np.random.default_rng(5)
    H = 2
    q = torch.from_numpy(rng.standard_normal((40, H, 128)).astype(np.float32)).to(torch.bfloat16)
    k = torch.from_numpy(np.repeat(rng.standard_normal((1, H, 128)).astype(np.float32), Lk, axis=0)
                         ).to(torch.bfloat16)
    v = torch.from_numpy(rng.integers(-8, 9, (Lk, H, 128)).astype(np.float32)).to(torch.bfloat16)
    exp = f32_to_bf16((bf16_to_f32(u16(v)).astype(np.float64).mean(axis=0)).astype(np.float32))
    assert np.array_equal(u16(_run(q, k, v)), np.broadcast_to(exp, (40, H, 128)))


def test_strided_views_and_out_rows():
    """q/k/v read as head/token-strided slices of fused [L, 3, H, D] rows; output written into
    the rows of a wider [L, H*D + 64] buffer (only the [:, :H*D] part may change)."""
    announce("attention strided")
    import joyomni_ops as jo
    L, H = 190, 2
    g = gen(3)
    qkv = torch.randn(L, 3, H, 128, generator=g).to(torch.bfloat16).to(DEV)
    q, k, v = qkv[None, :, 0], qkv[None, :, 1], qkv[None, :, 2]
    buf = torch.full((L, H * 128 + 64), 7.0, dtype=torch.bfloat16, device=DEV)
    out = buf[:, :H * 128].view(1, L, H, 128)
    jo.sdpa_attention_out(q, k, v, out)
    torch.cuda.synchronize()
    assert bool((buf[:, H * 128:] == 7.0).all())
    _check(out[0], q[0].cpu(), k[0].cpu(), v[0].cpu(), "strided")


def test_batch_of_two():
    announce("attention batch 2")
    import joyomni_ops as jo
    g = gen(4)
    q = torch.randn(2, 70, 2, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(2, 90, 2, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 90, 2, 128, generator=g).to(torch.bfloat16)
    out = jo.sdpa_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    for b in range(2):
        _check(out[b], q[b], k[b], v[b], f"batch {b}")


def test_argument_errors():
    import joyomni_ops as jo
    q = torch.zeros(1, 4, 2, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="head_dim=128"):
        jo.sdpa_attention(q, q, q)
    q = torch.zeros(1, 4, 2, 128, dtype=torch.bfloat16, device=DEV)
    k = torch.zeros(1, 0, 2, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="empty key"):
        jo.sdpa_attention(q, k, k)


def test_cfg4_joint_shape_sampled_queries():
    """The block's joint attention: 10800 + 512 queries over 2 x 10800 cached + 10800 + 512 keys,
    40 heads. 64 sampled queries (queries are independent) against the oracle; torch's SDPA
    (the reference's own call) on the same inputs is held to the same tolerance."""
    announce("attention cfg4 11312 x 32912 x 40")
    Lq, Lk, H = 11312, 32912, 40
    q, k, v = _inputs(Lq, Lk, H, 2024)
    qd, kd, vd = q[None].to(DEV), k[None].to(DEV), v[None].to(DEV)
    import joyomni_ops as jo
    out = jo.sdpa_attention(qd, kd, vd)[0]
    ref_sdpa = torch.nn.functional.scaled_dot_product_attention(
        qd.transpose(1, 2), kd.transpose(1, 2), vd.transpose(1, 2), is_causal=False).transpose(1, 2)[0]
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(9).choice(Lq, 64, replace=False))
    rows[-1] = Lq - 1
    err_ours = _check(out, q, k, v, "cfg4 ours", rows=rows)
    err_sdpa = _check(ref_sdpa, q, k, v, "cfg4 torch sdpa", rows=rows)
    print(f"cfg4 max|err| vs float64: ours {err_ours:.3e}, torch SDPA {err_sdpa:.3e}")


@pytest.mark.parametrize("Lk", [3467, 11267])
def test_reference_production_shape_sampled_queries(Lk):
    """The reference's own production attention (480x832 chunk: 3467 queries over 3467..11267
    keys, 32 heads of 128): 48 sampled queries against the oracle. 3467 = 108 blocks of 32 + 11
    rows: a partial last query block, 108 blocks per head (workgroups straddle heads), and a
    partial last key tile (11267 = 176 tiles of 64 + 3 keys)."""
    announce("attention reference production", 3467, Lk, 32)
    Lq, H = 3467, 32
    q, k, v = _inputs(Lq, Lk, H, 77 + Lk)
    out = _run(q, k, v)
    rows = np.sort(np.random.default_rng(Lk).choice(Lq, 48, replace=False))
    rows[0], rows[-1] = 0, Lq - 1
    _check(out, q, k, v, f"production {Lq}x{Lk}x{H}", rows=rows)
