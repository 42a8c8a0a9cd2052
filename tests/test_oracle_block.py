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
