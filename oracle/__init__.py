"""CPU oracle for the quantized DiT hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithms of the three device
paths this repository implements on MI355X:

* ``oracle.fp8``     -- bf16/fp16/fp32 bit conversions and the OCP e4m3fn cast.
* ``oracle.quant``   -- per-token activation quantisation (division variant of
  ``deploy/xvideo/models/dit/fp8_linear.py:38-43`` and reciprocal-multiply
  variant of ``joyomni_ops/csrc/per_token_quant_fp8_rocm.hip:60-78``) and
  per-output-channel weight quantisation (``fp8_linear.py:77-85``).
* ``oracle.gemm``    -- dequantise-then-matmul with the row/column scaled
  epilogue of ``joyomni_ops/csrc/fp8_gemm.cu:99-136``.
* ``oracle.qknorm``  -- per-head RMSNorm + interleaved RoPE
  (``joyomni_ops/csrc/fused_qknorm_rope_3d_kernel.cu:68-105``) and the fused
  QKV split / KV-ring write semantics (``deploy/xvideo/models/dit/dit.py:409-451``,
  ``dit.py:867-882``).
* ``oracle.kvpack``  -- joint-attention Q/K/V pack with the two-rounding text
  RMSNorm and the rotation of pre-RoPE cached K
  (``joyomni_ops/csrc/fused_joint_qkv_pack.cu:58-220``).
* ``oracle.attention`` -- the joint-attention core, softmax(q k^T / sqrt(D)) v
  (``deploy/xvideo/models/dit/dit.py:154-167``).
* ``oracle.rope``    -- 3-D (t,h,w) RoPE tables (``deploy/xvideo/models/dit/rope.py:31-52``,
  ``dit.py:896-934``, ``sgl_fused_ops.py:94-119``).
* ``oracle.torch_path`` -- the reference's own CPU torch code path, restated,
  used as the timed CPU baseline in ``bench.py``.
* ``oracle/quant_ref.c`` -- an independent C restatement of the quantiser plus
  an exhaustive checker of the device division formula (built by
  ``oracle/Makefile`` into ``oracle/liboracle.so``).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import anything from here, and only as the checker. The product path
(``joyomni_ops``) never imports it.

Pinning status of every function is listed in each module's header.
"""
