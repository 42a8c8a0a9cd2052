"""Host-side mirror of the reference operator package, without a GPU: schemas,
FakeTensor kernels (torch.compile opacity), wrappers and argument errors."""
import pytest
import torch

import joyomni_ops as jo
from joyomni_ops import fp8_linear, rope


REFERENCE_OPS = ["fused_qk_norm_rope_3d_paired", "fused_joint_qkv_pack", "fused_cached_kv_pack",
                 "fused_norm_scale_shift", "rmsnorm", "sgl_per_token_quant_fp8", "fp8_scaled_mm"]


def test_reference_schemas_registered():
    for name in REFERENCE_OPS:
        assert hasattr(torch.ops.joyomni_ops, name)
    assert jo.has_fp8() and jo.has_quant()
    s = str(torch.ops.joyomni_ops.fp8_scaled_mm.default._schema)
    assert "ScalarType out_dtype" in s and "Tensor? bias" in s
    s = str(torch.ops.joyomni_ops.fused_qk_norm_rope_3d_paired.default._schema)
    assert s.startswith("joyomni_ops::fused_qk_norm_rope_3d_paired(Tensor(") and "Tensor(a!)? k_pre_rope" in s
    args = torch.ops.joyomni_ops.fused_qk_norm_rope_3d_paired.default._schema.arguments
    # q, k (as in the reference) and k_pre_rope (which the reference's kernel writes but its schema
    # leaves undeclared) are declared mutable
    assert [a.name for a in args if a.alias_info is not None and a.alias_info.is_write] == ["q", "k", "k_pre_rope"]


def test_fake_kernels_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        a = torch.empty(300, 512, dtype=torch.float8_e4m3fn, device="cuda")
        b = torch.empty(1024, 512, dtype=torch.float8_e4m3fn, device="cuda").t()
        sa = torch.empty(300, 1, device="cuda")
        sb = torch.empty(1, 1024, device="cuda")
        out = jo.fp8_scaled_mm(a, b, sa, sb, torch.bfloat16, None)
        assert out.shape == (300, 1024) and out.dtype == torch.bfloat16
        out = jo.fp8_scaled_mm_gelu_tanh(a, b, sa, sb, torch.bfloat16, None)
        assert out.shape == (300, 1024)
        q = torch.empty(1, 17, 4, 128, dtype=torch.bfloat16, device="cuda")
        t = torch.empty(1, 11, 4, 128, dtype=torch.bfloat16, device="cuda")
        c = torch.empty(1, 9, 4, 128, dtype=torch.bfloat16, device="cuda")
        w = torch.empty(128, dtype=torch.bfloat16, device="cuda")
        oq, ok, ov = jo.fused_joint_qkv_pack(q, q, q, t, t, t, c, c, w, w, 1e-6)
        assert oq.shape == (1, 28, 4, 128) and ok.shape == (1, 37, 4, 128) and ov.shape == ok.shape


def test_cpu_tensors_rejected_like_reference():
    x = torch.zeros(4, 32, dtype=torch.bfloat16)
    q = torch.empty(4, 32, dtype=torch.float8_e4m3fn)
    s = torch.empty(4, 1)
    with pytest.raises(NotImplementedError):
        # no CPU kernel is registered: the op exists only for GPU tensors
        jo.sgl_per_token_quant_fp8(x, q, s)
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        jo._quant_impl(x, q, s, 0)
    a = torch.zeros(4, 32, dtype=torch.float8_e4m3fn)
    with pytest.raises(RuntimeError, match="mat_a must be a CUDA tensor"):
        jo._scaled_mm_impl(a, a.t(), s, s, torch.bfloat16, None, 0)


def test_fp8_linear_api_surface():
    assert fp8_linear.available()
    assert fp8_linear.backend() == "joyomni_ops/gfx950-hip"
    assert fp8_linear.FP8_MAX == 448.0
    for name in ("Fp8Linear", "_quantize_weight_per_channel", "quantize_per_token"):
        assert hasattr(fp8_linear, name)


def test_rope_tables_match_oracle():
    import numpy as np
    from oracle import rope as orope
    cos, sin = rope.rope_3d_half_tables(3, 4, 6, (44, 42, 42), 10000.0)
    _, _, cb, sb = orope.rope_half_tables([0, 1, 2], 4, 6, (44, 42, 42), 10000.0)
    c = cos.view(torch.int16).numpy().view(np.uint16)
    s = sin.view(torch.int16).numpy().view(np.uint16)
    # torch's fp32 cos/sin may differ from the correctly rounded value by 1 ulp,
    # which can move a bf16 rounding by one step.
    assert np.mean(c == cb) > 0.99 and np.mean(s == sb) > 0.99
    assert np.all(np.abs(c.astype(np.int32) - cb.astype(np.int32)) <= 1)


def test_visual_rope_tables_match_oracle():
    """The product's [current | ref-video] tables (dit.py:1093-1166) equal the oracle's bf16 bits
    (up to one step where torch's fp32 cos/sin round differently), at the production dims."""
    import numpy as np
    from oracle import rope as orope
    for kw in ({}, {"ref_image_cache": True}, {"temporal_ids": torch.tensor([3, 4])}):
        cos, sin = rope.visual_rope_half_tables((2, 4, 6), 2, **kw)
        okw = dict(kw)
        if "temporal_ids" in okw:
            okw["temporal_ids"] = okw["temporal_ids"].numpy()
        _, _, cb, sb = orope.visual_half_tables((2, 4, 6), 2, **okw)
        c = cos.view(torch.int16).numpy().view(np.uint16)
        s = sin.view(torch.int16).numpy().view(np.uint16)
        assert cos.shape == (2 * 2 * 4 * 6, 64)
        assert np.mean(c == cb) > 0.99 and np.mean(s == sb) > 0.99
        assert np.all(np.abs(c.astype(np.int32) - cb.astype(np.int32)) <= 1)
        assert np.all(np.abs(s.astype(np.int32) - sb.astype(np.int32)) <= 1)
    # target tokens alone: the plain 3-D tables
    c0, s0 = rope.visual_rope_half_tables((2, 4, 6), None)
    c1, s1 = rope.rope_3d_half_tables(2, 4, 6, (16, 56, 56), 256.0)
    assert torch.equal(c0, c1) and torch.equal(s0, s1)
    with pytest.raises(ValueError, match="temporal ids"):
        rope.visual_rope_tables((2, 4, 6), 3, temporal_ids=torch.tensor([0, 1]))
