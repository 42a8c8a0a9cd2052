"""CPU checks of the block-chain restatement (oracle/torch_path.double_stream_block):
its pieces are pinned in their own oracle tests; here the block's structure --
zero gates leave both streams unchanged, the cached K/V segments and the video K/V
reach attention, and the ring outputs are the pre-RoPE K and the raw V."""
import numpy as np
import torch

from oracle import qknorm as oqk
from oracle import torch_path
from oracle.fp8 import bf16_to_f32


def u16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def make_streams(E, H, FFN, g, zero_gates=False):
    out = []
    D = E // H
    for _ in range(2):
        w = {"mod_table": (torch.randn(1, 6, E, generator=g) / E ** 0.5).to(torch.bfloat16),
             "q_norm": (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16),
             "k_norm": (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)}
        if zero_gates:
            w["mod_table"][:, 2] = 0
            w["mod_table"][:, 5] = 0
        for name, (k, n) in {"qkv": (E, 3 * E), "proj": (E, E), "up": (E, FFN), "down": (FFN, E)}.items():
            q, s = torch_path.quantize_per_token((torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16))
            w[f"{name}_q"], w[f"{name}_s"] = q, s.reshape(-1)
            w[f"{name}_b"] = (torch.randn(n, generator=g) * 0.01).to(torch.bfloat16)
        out.append(w)
    return out


def tables(L, D, g):
    ang = torch.rand(L, D // 2, generator=g) * 6.28
    return ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)


def test_zero_gates_leave_streams_unchanged():
    g = torch.Generator().manual_seed(0)
    E, H, FFN, L, T = 256, 2, 512, 24, 8
    streams = make_streams(E, H, FFN, g, zero_gates=True)
    img = torch.randn(L, E, generator=g).to(torch.bfloat16)
    txt = torch.randn(T, E, generator=g).to(torch.bfloat16)
    vec = torch.zeros(1, E, dtype=torch.bfloat16)
    c, s = tables(L, E // H, g)
    oi, ot, _, _ = torch_path.double_stream_block(img, txt, vec, streams, H, c, s)
    assert torch.equal(oi, img) and torch.equal(ot, txt)


def test_ring_outputs_and_qkv_semantics():
    g = torch.Generator().manual_seed(1)
    E, H, FFN, L, T = 256, 2, 512, 24, 8
    D = E // H
    streams = make_streams(E, H, FFN, g)
    img = torch.randn(L, E, generator=g).to(torch.bfloat16)
    txt = torch.randn(T, E, generator=g).to(torch.bfloat16)
    vec = torch.randn(1, E, generator=g).to(torch.bfloat16)
    c, s = tables(L, D, g)
    _, _, k_pre, v = torch_path.double_stream_block(img, txt, vec, streams, H, c, s)
    # recompute the video QKV projection and check the ring outputs against the qknorm oracle
    w = streams[0]
    mod = [m.squeeze(1) for m in (w["mod_table"].float() + vec.float()[:, None]).to(torch.bfloat16).chunk(6, 1)]
    xm = torch_path._layernorm_modulate_ref(img, mod[0], mod[1], 1e-6)
    qkv = torch_path._fp8_linear_ref(xm, w["qkv_q"], w["qkv_s"], w["qkv_b"], False)
    _, _, okp, ov = oqk.qkv_norm_rope_cache(u16(qkv), H, 1e-6, u16(w["q_norm"]), u16(w["k_norm"]), u16(c), u16(s))
    assert np.array_equal(u16(v), ov)
    diff = np.abs(bf16_to_f32(u16(k_pre)) - bf16_to_f32(okp))
    assert diff.max() <= 2.0 ** -7 * np.abs(bf16_to_f32(okp)).max()


def test_cached_segments_change_attention_only_through_keys_and_values():
    g = torch.Generator().manual_seed(2)
    E, H, FFN, L, T = 256, 2, 512, 24, 8
    D = E // H
    streams = make_streams(E, H, FFN, g)
    img = torch.randn(L, E, generator=g).to(torch.bfloat16)
    txt = torch.randn(T, E, generator=g).to(torch.bfloat16)
    vec = torch.randn(1, E, generator=g).to(torch.bfloat16)
    c, s = tables(L, D, g)
    base = torch_path.double_stream_block(img, txt, vec, streams, H, c, s)
    key = torch.randn(16, H, D, generator=g).to(torch.bfloat16)
    val = torch.randn(16, H, D, generator=g).to(torch.bfloat16)
    ones, zeros = torch.ones(16, D), torch.zeros(16, D)
    with_cache = torch_path.double_stream_block(img, txt, vec, streams, H, c, s, [(key, val, ones, zeros)])
    assert not torch.equal(with_cache[0], base[0])          # attention sees the cached tokens
    assert torch.equal(with_cache[2], base[2]) and torch.equal(with_cache[3], base[3])  # ring outputs unchanged


def _set_chunks(streams, values):
    """Write exact modulation chunks (vec = 0 keeps them: mod = bf16(table + 0))."""
    for w in streams:
        for j, v in values.items():
            w["mod_table"][:, j] = v


def test_second_adaln_order_and_ffn_gate():
    """gate1 = 0, shift2 = c, scale2 = -1, gate2 = 1: the FFN input is the row c for every token
    (LN(x) * (1 + scale2) + shift2), so out(x) = x + FFN(c) with FFN(c) = out(0); swapping shift2 with
    scale2, or gate1 with gate2, makes the added term depend on x (dit.py:383-390,525-538)."""
    g = torch.Generator().manual_seed(3)
    E, H, FFN, L, T = 256, 2, 512, 24, 8
    streams = make_streams(E, H, FFN, g)
    c_img = torch.randn(E, generator=g).to(torch.bfloat16)
    _set_chunks(streams[:1], {2: 0.0, 3: c_img, 4: -1.0, 5: 1.0})
    _set_chunks(streams[1:], {2: 0.0, 3: c_img.flip(0), 4: -1.0, 5: 1.0})
    vec = torch.zeros(1, E, dtype=torch.bfloat16)
    img = torch.randn(L, E, generator=g).to(torch.bfloat16)
    txt = torch.randn(T, E, generator=g).to(torch.bfloat16)
    c, s = tables(L, E // H, g)
    oi, ot, _, _ = torch_path.double_stream_block(img, txt, vec, streams, H, c, s)
    zi, zt, _, _ = torch_path.double_stream_block(torch.zeros_like(img), torch.zeros_like(txt), vec, streams, H, c, s)
    assert torch.equal(oi, (img.float() + zi.float()).to(torch.bfloat16))
    assert torch.equal(ot, (txt.float() + zt.float()).to(torch.bfloat16))
    assert torch.equal(zi, zi[:1].expand_as(zi))  # the same FFN(c) on every token
    # FFN(c) = down(gelu(up(c))) with the pinned linear pieces (dit.py:508-513)
    w = streams[0]
    h = torch_path._fp8_linear_ref(c_img[None], w["up_q"], w["up_s"], w["up_b"], False, gelu=True)
    d = torch_path._fp8_linear_ref(h, w["down_q"], w["down_s"], w["down_b"], False)
    assert torch.equal(zi[0], d[0])


def test_first_adaln_order_and_attention_gate():
    """shift1 = c, scale1 = -1, gate1 = 1, gate2 = 0: the QKV input is c on every token, so the
    attention branch does not depend on x: out(x) = x + out(0) (swaps of shift1/scale1 or of the
    gates break it), and out(0) varies over tokens only through RoPE."""
    g = torch.Generator().manual_seed(4)
    E, H, FFN, L, T = 256, 2, 512, 24, 8
    streams = make_streams(E, H, FFN, g)
    c_row = torch.randn(E, generator=g).to(torch.bfloat16)
    _set_chunks(streams, {0: c_row, 1: -1.0, 2: 1.0, 5: 0.0})
    vec = torch.zeros(1, E, dtype=torch.bfloat16)
    img = torch.randn(L, E, generator=g).to(torch.bfloat16)
    txt = torch.randn(T, E, generator=g).to(torch.bfloat16)
    c, s = tables(L, E // H, g)
    oi, ot, _, _ = torch_path.double_stream_block(img, txt, vec, streams, H, c, s)
    zi, zt, _, _ = torch_path.double_stream_block(torch.zeros_like(img), torch.zeros_like(txt), vec, streams, H, c, s)
    assert torch.equal(oi, (img.float() + zi.float()).to(torch.bfloat16))
    assert torch.equal(ot, (txt.float() + zt.float()).to(torch.bfloat16))
    # with identity RoPE every video token sees the same q, k, v: one attention row for all
    ones, zeros = torch.ones_like(c), torch.zeros_like(s)
    ui, _, _, _ = torch_path.double_stream_block(torch.zeros_like(img), torch.zeros_like(txt), vec, streams, H,
                                                 ones, zeros)
    assert torch.equal(ui, ui[:1].expand_as(ui)) and not torch.equal(zi, zi[:1].expand_as(zi))


def _block_inputs(seed, E=256, H=2, FFN=512, L=24, T=8):
    g = torch.Generator().manual_seed(seed)
    streams = make_streams(E, H, FFN, g)
    img = torch.randn(L, E, generator=g).to(torch.bfloat16)
    txt = torch.randn(T, E, generator=g).to(torch.bfloat16)
    vec = torch.randn(1, E, generator=g).to(torch.bfloat16)
    c, s = tables(L, E // H, g)
    return g, streams, img, txt, vec, c, s


def test_write_only_returns_after_the_cache_write():
    """kv_cache_write_only (dit.py:446-459): streams unchanged, cache = the full forward's cache;
    kv_cache_write_seq_len keeps the first tokens (dit.py:449-451)."""
    g, streams, img, txt, vec, c, s = _block_inputs(5)
    H = 2
    full = torch_path.double_stream_block(img, txt, vec, streams, H, c, s)
    wo = torch_path.double_stream_block(img, txt, vec, streams, H, c, s, write_only=True, cache_tokens=10)
    assert wo[0] is img and wo[1] is txt
    assert torch.equal(wo[2], full[2][:10]) and torch.equal(wo[3], full[3][:10])


def test_post_rope_cache_holds_the_rotated_key():
    """kv_cache_pre_rope=False (dit.py:432-433): the cache keeps the rotated K of the qknorm oracle."""
    g, streams, img, txt, vec, c, s = _block_inputs(6)
    H, L = 2, img.shape[0]
    _, _, k_cache, _ = torch_path.double_stream_block(img, txt, vec, streams, H, c, s, cache_pre_rope=False)
    w = streams[0]
    mod = [m.squeeze(1) for m in (w["mod_table"].float() + vec.float()[:, None]).to(torch.bfloat16).chunk(6, 1)]
    qkv = torch_path._fp8_linear_ref(torch_path._layernorm_modulate_ref(img, mod[0], mod[1], 1e-6), w["qkv_q"],
                                     w["qkv_s"], w["qkv_b"], False)
    _, ok, _, _ = oqk.qkv_norm_rope_cache(u16(qkv), H, 1e-6, u16(w["q_norm"]), u16(w["k_norm"]), u16(c), u16(s))
    diff = np.abs(bf16_to_f32(u16(k_cache)) - bf16_to_f32(ok))
    assert k_cache.shape[0] == L and diff.max() <= 2.0 ** -7 * np.abs(bf16_to_f32(ok)).max()


def test_skip_text_stream_ignores_the_condition():
    """skip_text_stream (dit.py:481-487,500-506): txt comes back unchanged and has no influence on
    the video output; with the text stream the condition tokens do influence it."""
    g, streams, img, txt, vec, c, s = _block_inputs(7)
    H = 2
    txt2 = torch.randn(txt.shape, generator=g).to(torch.bfloat16)
    a = torch_path.double_stream_block(img, txt, vec, streams, H, c, s, skip_text_stream=True)
    b = torch_path.double_stream_block(img, txt2, vec, streams, H, c, s, skip_text_stream=True)
    assert a[1] is txt and torch.equal(a[0], b[0])
    full = torch_path.double_stream_block(img, txt, vec, streams, H, c, s)
    assert not torch.equal(full[0], a[0])
    assert torch.equal(full[2], a[2]) and torch.equal(full[3], a[3])


def test_rotated_and_pre_rope_cached_entries_agree():
    """A cached key stored rotated (tables None) gives the block the same result as the pre-RoPE key
    with its tables, rotated by the pinned kvpack oracle (dit.py:216-271)."""
    from oracle import kvpack as okv
    g, streams, img, txt, vec, c, s = _block_inputs(8)
    H, D = 2, 128
    key = torch.randn(16, H, D, generator=g).to(torch.bfloat16)
    val = torch.randn(16, H, D, generator=g).to(torch.bfloat16)
    ang = torch.rand(16, D // 2, generator=g) * 6.28
    cf = ang.cos().repeat_interleave(2, -1)
    sf = ang.sin().repeat_interleave(2, -1)
    rot = torch.from_numpy(okv.rotate_pairs(u16(key), cf.numpy(), sf.numpy()).view(np.int16)).view(torch.bfloat16)
    for skip in (False, True):
        a = torch_path.double_stream_block(img, txt, vec, streams, H, c, s, [(key, val, cf, sf)], skip_text_stream=skip)
        b = torch_path.double_stream_block(img, txt, vec, streams, H, c, s, [(rot, val, None, None)],
                                           skip_text_stream=skip)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_sampled_rows_equal_the_full_block_rows():
    """out_rows computes the same rows as the full block (attention and tail are row-local)."""
    g, streams, img, txt, vec, c, s = _block_inputs(9)
    H = 2
    ri, rt = torch.tensor([0, 5, 23]), torch.tensor([1, 7])
    for skip in (False, True):
        full = torch_path.double_stream_block(img, txt, vec, streams, H, c, s, skip_text_stream=skip)
        part = torch_path.double_stream_block(img, txt, vec, streams, H, c, s, skip_text_stream=skip,
                                              out_rows=(ri, rt))
        assert torch.equal(part[0], full[0][ri]) and torch.equal(part[1], full[1][rt])
        assert torch.equal(part[2], full[2]) and torch.equal(part[3], full[3])
