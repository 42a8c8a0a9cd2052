"""GPU: the ops survive the reference's compile boundary.

The reference runs its whole block loop inside ``torch.compile(_run_double_blocks,
fullgraph=...)`` (``deploy/xvideo/serving/joyomni_streaming.py:404-411``) and registers FakeTensor
kernels for its ops so that the compile keeps them as opaque calls in one graph
(``joyomni_ops/joyomni_ops/__init__.py:36-38``). Two checks:

* the drop-in sequence of the block (adaLN norm emitting FP8 -> QKV GEMM -> fused QKV norm/RoPE
  writing into views of the joint Q / K / V and into the KV ring -> cached rows rotated into the
  head of the joint K / V -> condition rows packed into their tails -> attention -> out-projection
  with the gated residual -> adaLN norm -> FFN-up with GELU -> FFN-down with the gated residual
  in place) as ONE function under ``torch.compile(fullgraph=True, backend="aot_eager")`` gives
  the same bits as the same function run eagerly: the returned tensors and every mutated buffer
  (joint Q / K / V, both ring tensors);
* ``torch.library.opcheck`` on every op of the package with small inputs: schema (declared
  mutations and aliasing), FakeTensor kernel against the real one, and AOT dispatch with dynamic
  shapes. torch's schema check compares tensors with ``allclose``, which has no float8 kernel, so
  for ops with float8 arguments that one check is replaced by the same check done bytewise here
  (every argument the schema does not declare mutable is unchanged after the call).
"""
import pytest
import torch

from gpu_util import DEV, announce, gen

pytestmark = pytest.mark.gpu

E, H, D, FFN = 512, 4, 128, 1536
L, T, C = 240, 32, 240  # video tokens (one 1 x 12 x 20 frame), condition tokens, cached tokens
EPS = 1e-6


def _bf(*shape, g, scale=1.0):
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16).to(DEV)


def _tables(g):
    from joyomni_ops.rope import rope_3d_half_tables
    cos_h, sin_h = rope_3d_half_tables(1, 12, 20, (44, 42, 42), 10000.0, device=DEV)
    ang = torch.rand(C, D, generator=g) * 6.28
    return cos_h, sin_h, ang.cos().to(DEV), ang.sin().to(DEV)


def test_block_sequence_under_torch_compile_fullgraph_matches_eager():
    import joyomni_ops as jo
    from joyomni_ops.dit_block import QuantizedDoubleStreamBlock
    announce("torch.compile fullgraph aot_eager block sequence")
    g = gen(900)
    blk = QuantizedDoubleStreamBlock(E, H, FFN, DEV, g, overlap_streams=False)
    img2 = _bf(L, E, g=g)
    txt2 = _bf(T, E, g=g)
    vec = _bf(1, E, g=g)
    cos_h, sin_h, cf, sf = _tables(g)

    def buffers():
        gb = gen(901)  # identical initial contents for both runs; NaN where every row is rewritten
        q = torch.full((1, L + T, H, D), float("nan"), dtype=torch.bfloat16, device=DEV)
        k = torch.full((1, C + L + T, H, D), float("nan"), dtype=torch.bfloat16, device=DEV)
        v = torch.full_like(k, float("nan"))
        ring_k = _bf(2, L, H, D, g=gb)
        ring_v = _bf(2, L, H, D, g=gb)
        return q, k, v, ring_k, ring_v

    def sequence(img2, txt2, vec, q, k, v, ring_k, ring_v, cos_h, sin_h, cf, sf):
        im = blk.modulation(blk.img, vec)
        tm = blk.modulation(blk.txt, vec)
        # adaLN norm emitting FP8, QKV GEMM (INTEGRATION steps 3 and 5)
        q8, s8 = blk.norm_quant(img2, im[0], im[1], E)
        img_qkv = blk.img.qkv.gemm(q8, s8)
        # video q/k norm + RoPE into views of the joint buffers, K / V into ring slot 0 (step 4, 6)
        jo.fused_qkv_norm_rope_cache(img_qkv, H, EPS, blk.img.q_norm, blk.img.k_norm, cos_h, sin_h,
                                     q[0, :L], k[0, C:C + L], ring_k, ring_v, 0, 0, v_out=v[0, C:C + L])
        # cached chunk (ring slot 1, K before RoPE) rotated into the head of the joint K / V (step 6)
        jo.fused_cached_kv_pack_out(ring_k[1, :C][None], ring_v[1, :C][None], None, None, cf, sf,
                                    k[:, :C], v[:, :C])
        # condition stream: Fp8Linear forward (quant + GEMM), rows packed into the tails (steps 3, 6)
        q8t, s8t = blk.norm_quant(txt2, tm[0], tm[1], E)
        tv = blk.txt.qkv.gemm(q8t, s8t).view(1, T, 3, H, D)
        jo.fused_text_qkv_pack(tv[:, :, 0], tv[:, :, 1], tv[:, :, 2], blk.txt.q_norm, blk.txt.k_norm, EPS,
                               q[:, L:], k[:, C + L:], v[:, C + L:])
        # attention core (step 8)
        attn = jo.sdpa_attention(q, k, v).flatten(2, 3)
        # out-projection with the gated residual, FFN-up + GELU, FFN-down in place (steps 5, 7)
        x = blk.img.proj.gated_residual(attn[0, :L], img2, im[2])
        q8, s8 = blk.norm_quant(x, im[3], im[4], E)
        h = blk.img.up.gemm(q8, s8)
        blk.img.down.gated_residual(h, x, im[5], inplace=True)
        y = blk.txt.proj(attn[0, L:])  # Fp8Linear.forward on the condition rows
        return x, y, attn

    eager_bufs = buffers()
    ref = sequence(img2, txt2, vec, *eager_bufs, cos_h, sin_h, cf, sf)
    torch.cuda.synchronize()
    torch._dynamo.reset()
    compiled = torch.compile(sequence, fullgraph=True, backend="aot_eager")
    comp_bufs = buffers()
    got = compiled(img2, txt2, vec, *comp_bufs, cos_h, sin_h, cf, sf)
    torch.cuda.synchronize()
    names = ("x", "txt projection", "attention")
    for name, a, b in zip(names, got, ref):
        assert not torch.isnan(b.float()).any(), name
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"{name}: compiled differs from eager"
    for name, a, b in zip(("joint Q", "joint K", "joint V", "ring K", "ring V"), comp_bufs, eager_bufs):
        assert not torch.isnan(b.float()).any(), name
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"{name}: compiled differs from eager"
    # a second call reuses the compiled graph (no recompilation) on new inputs
    img2b = _bf(L, E, g=g)
    ref2 = sequence(img2b, txt2, vec, *eager_bufs, cos_h, sin_h, cf, sf)
    got2 = compiled(img2b, txt2, vec, *comp_bufs, cos_h, sin_h, cf, sf)
    torch.cuda.synchronize()
    for name, a, b in zip(names, got2, ref2):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"second call {name}"


# --------------------------------------------------------------------------
# opcheck
# --------------------------------------------------------------------------
def _fp8(t):
    from joyomni_ops.fp8_linear import quantize_per_token
    return quantize_per_token(t.contiguous(), True)


def _cases():
    """(op name, args) with small inputs, one entry per op of the package."""
    g = gen(910)
    ops = torch.ops.joyomni_ops
    cases = []
    x = _bf(33, 512, g=g)
    cases.append((ops.sgl_per_token_quant_fp8, (x, torch.empty(33, 512, dtype=torch.float8_e4m3fn, device=DEV),
                                                torch.empty(33, 1, device=DEV))))
    cases.append((ops.per_token_quant_fp8, (x, torch.empty(33, 512, dtype=torch.float8_e4m3fn, device=DEV),
                                            torch.empty(33, 1, device=DEV), True)))
    a, sa = _fp8(_bf(64, 512, g=g))
    w, sw = _fp8(_bf(256, 512, g=g, scale=0.02))
    b, sb = w.t(), sw.reshape(1, 256)
    bias = _bf(256, g=g, scale=0.01)
    cases.append((ops.fp8_scaled_mm, (a, b, sa, sb, torch.bfloat16, bias)))
    cases.append((ops.fp8_scaled_mm_gelu_tanh, (a, b, sa, sb, torch.bfloat16, bias)))
    res = _bf(64, 256, g=g)
    gate = _bf(256, g=g)
    cases.append((ops.fp8_scaled_mm_gated_residual, (a, b, sa, sb, res, gate, bias)))
    cases.append((ops.fp8_scaled_mm_gated_residual_, (a, b, sa, sb, res.clone(), gate, bias)))
    cos_h, sin_h, cf, sf = _tables(g)
    qw, kw = _bf(D, g=g, scale=0.1) + 1, _bf(D, g=g, scale=0.1) + 1
    cases.append((ops.fused_qk_norm_rope_3d_paired, (_bf(1, L * H, D, g=g), _bf(1, L * H, D, g=g), L, H, EPS, qw, kw,
                                                     cos_h, sin_h, _bf(1, L * H, D, g=g))))
    qkv = _bf(L, 3 * E, g=g)
    cases.append((ops.fused_qkv_norm_rope_cache, (qkv, H, EPS, qw, kw, cos_h, sin_h, _bf(L, H, D, g=g),
                                                  _bf(L, H, D, g=g), _bf(2, L, H, D, g=g), _bf(2, L, H, D, g=g), 1, 0,
                                                  _bf(L, H, D, g=g), -1, True)))
    aq, saq = _fp8(_bf(L, E, g=g))
    wq, swq = _fp8(_bf(3 * E, E, g=g, scale=0.02))
    cases.append((ops.fp8_qkv_norm_rope_cache, (aq, wq.t(), saq, swq.reshape(1, 3 * E), _bf(3 * E, g=g, scale=0.01),
                                                H, EPS, qw, kw, cos_h, sin_h, _bf(L, H, D, g=g), _bf(L, H, D, g=g),
                                                _bf(2, L, H, D, g=g), _bf(2, L, H, D, g=g), 1, 0, _bf(L, H, D, g=g),
                                                -1, True)))
    img = qkv.view(1, L, 3, H, D)
    txt = _bf(1, T, 3, H, D, g=g)
    ck, cv = _bf(1, C, H, D, g=g), _bf(1, C, H, D, g=g)
    cases.append((ops.fused_joint_qkv_pack, (img[:, :, 0], img[:, :, 1], img[:, :, 2], txt[:, :, 0], txt[:, :, 1],
                                             txt[:, :, 2], ck, cv, qw, kw, EPS)))
    half = C // 2
    cases.append((ops.fused_cached_kv_pack, (ck[:, :half], cv[:, :half], ck[:, half:], cv[:, half:], cf, sf)))
    cases.append((ops.fused_cached_kv_pack_out, (ck[:, :half], cv[:, :half], ck[:, half:], cv[:, half:], cf, sf,
                                                 _bf(1, C, H, D, g=g), _bf(1, C, H, D, g=g))))
    cases.append((ops.fused_text_qkv_pack, (txt[:, :, 0], txt[:, :, 1], txt[:, :, 2], qw, kw, EPS,
                                            _bf(1, T, H, D, g=g), _bf(1, T, H, D, g=g), _bf(1, T, H, D, g=g))))
    xn = _bf(48, E, g=g)
    sc, sh = _bf(1, E, g=g, scale=0.2), _bf(1, E, g=g, scale=0.2)
    cases.append((ops.fused_norm_scale_shift, (xn, None, None, sc, sh, 0, EPS)))
    cases.append((ops.fused_norm_scale_shift_fp8, (xn, None, None, sc, sh, 0, EPS,
                                                   torch.empty(48, E, dtype=torch.float8_e4m3fn, device=DEV),
                                                   torch.empty(48, 1, device=DEV), _bf(48, E, g=g), False)))
    cases.append((ops.rmsnorm, (xn, qw.repeat(4), EPS)))
    q4, k4, v4 = _bf(1, 70, H, D, g=g), _bf(1, 150, H, D, g=g), _bf(1, 150, H, D, g=g)
    cases.append((ops.sdpa_attention, (q4, k4, v4, None)))
    cases.append((ops.sdpa_attention_out, (q4, k4, v4, _bf(1, 70, H, D, g=g), None)))
    return cases


def _op_names():
    import joyomni_ops  # noqa: F401
    return sorted(n for n in dir(torch.ops.joyomni_ops) if isinstance(getattr(torch.ops.joyomni_ops, n),
                                                                       torch._ops.OpOverloadPacket))


def _has_fp8(args):
    return any(isinstance(t, torch.Tensor) and t.dtype == torch.float8_e4m3fn for t in args)


def _bytes_of(t):
    return t.detach().contiguous().view(torch.uint8).clone() if t.numel() else t.detach().clone()


def _check_undeclared_args_unchanged(op, args):
    """torch's schema check done bytewise: run the op and require every tensor argument that the
    schema does not declare mutable (``Tensor(a!)``) to hold the same bytes afterwards."""
    schema = op.default._schema
    before = [_bytes_of(t) if isinstance(t, torch.Tensor) else None for t in args]
    cloned = [t.clone() if isinstance(t, torch.Tensor) else t for t in args]
    op(*cloned)
    torch.cuda.synchronize()
    for arg, b, t in zip(schema.arguments, before, cloned):
        if b is None or (arg.alias_info is not None and arg.alias_info.is_write):
            continue
        assert torch.equal(_bytes_of(t), b), f"{schema.name}: argument {arg.name} changed but is not declared mutable"


def test_opcheck_covers_every_op():
    """Every op the package registers has an opcheck case below."""
    assert sorted(op._qualified_op_name.split("::")[1] for op, _ in _cases()) == _op_names()


@pytest.mark.parametrize("index", range(18))
def test_opcheck(index):
    import joyomni_ops  # noqa: F401
    cases = _cases()
    assert len(cases) == 18
    op, args = cases[index]
    announce("opcheck", op._qualified_op_name)
    utils = ("test_schema", "test_autograd_registration", "test_faketensor", "test_aot_dispatch_dynamic")
    if _has_fp8(args):
        _check_undeclared_args_unchanged(op, args)
        utils = utils[1:]
    torch.library.opcheck(op.default, args, test_utils=utils)
    torch.cuda.synchronize()
