"""GPU parity: the Fp8Linear counterpart end to end (weight quant, act quant, GEMM, GELU)."""
import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, gen, outlier_acts, u16, u8
from oracle import gemm as og
from oracle import quant as oq
from oracle.fp8 import bf16_to_f32

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("gelu,rounding,K", [(False, "reference_rocm", 1024), (True, "reference_rocm", 1024),
                                             (False, "reference_rocm", 8192), (False, "division", 1024)])
def test_fp8_linear_matches_oracle(gelu, rounding, K):
    """Activation rounding as the reference's ROCm path (fp8_linear.py:57-74): reciprocal-multiply
    below K = 8192, division from 8192 up; or division for every K."""
    announce("Fp8Linear", gelu, rounding, K)
    from joyomni_ops.fp8_linear import Fp8Linear, _quantize_weight_per_channel
    g = gen(21)
    N = 768
    lin = torch.nn.Linear(K, N, bias=True)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(N, K, generator=g) * 0.02)
        lin.bias.copy_(torch.randn(N, generator=g) * 0.01)
    lin = lin.to(torch.bfloat16).to(DEV)
    wq, ws = _quantize_weight_per_channel(lin.weight.data)
    qw_ref, sw_ref = oq.quant_weight_per_channel(u16(lin.weight.data))
    assert np.array_equal(u8(wq.t()), qw_ref) and np.array_equal(ws.cpu().numpy().reshape(-1), sw_ref)
    layer = Fp8Linear.from_linear(lin, gelu_tanh=gelu, quant_rounding=rounding)
    variant = "div" if (rounding == "division" or K >= 8192) else "rcp"
    assert layer.exact_division == (variant == "div")
    x = outlier_acts(2 * 150, K, g).reshape(2, 150, K)
    y = layer(x.to(DEV))
    assert y.shape == (2, 150, N)
    qa, sa = oq.quant_per_token(u16(x.reshape(-1, K)), "bf16", variant)
    pre = og.reference_fp32(qa, qw_ref, sa, sw_ref, u16(lin.bias.data))
    rms = float(np.sqrt(np.mean(pre.astype(np.float64) ** 2)))
    got = y.float().cpu().numpy().reshape(-1, N)
    if not gelu:
        assert np.abs(got - pre).max() <= 2e-2 * rms
    else:
        # GELU is 1.13-Lipschitz: the GEMM tolerance carries over, plus the final
        # bf16 rounding of the activation (one ulp of the result).
        ref = og.gelu_tanh(pre)
        ulp = np.spacing(np.abs(ref).astype(np.float32)) * 65536.0
        assert np.all(np.abs(got - ref) <= 1.13 * 2e-2 * rms + ulp)
