"""GPU: the allocation-free FP8 GEMM entry point (joy_fp8_scaled_mm_noalloc) against the
workspace entry point (joy_fp8_scaled_mm), through the C ABI. Both run the same kernels and the
same split-K plan, so the outputs must be bit-identical: the first call of the process captured
into a HIP graph and replayed, calls in a row (the second on a smaller problem, so stale partial
sums of the first would show), a problem that needs no scratch, and the largest split plan of
the device, which fills the whole scratch on a 256-CU MI355X."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, gen, outlier_acts, u16
from oracle import quant as oq

pytestmark = pytest.mark.gpu


def _problem(M, N, K, seed):
    g = gen(seed)
    x = outlier_acts(M, K, g)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    bias = (torch.randn(N, generator=g) * 0.01).to(torch.bfloat16)
    qa, sa = oq.quant_per_token(u16(x), "bf16", "div")
    qw, sw = oq.quant_weight_per_channel(u16(w))
    dev8 = lambda q: torch.from_numpy(np.ascontiguousarray(q)).view(torch.float8_e4m3fn).to(DEV)  # noqa: E731
    return (dev8(qa), dev8(qw), torch.from_numpy(sa).to(DEV), torch.from_numpy(sw).to(DEV), bias.to(DEV))


def _call(lib, fn, a, w, sa, sw, bias, out, M, N, K, epilogue, *ws):
    stream = torch.cuda.current_stream().cuda_stream
    return getattr(lib, fn)(a.data_ptr(), w.data_ptr(), sa.data_ptr(), sw.data_ptr(), bias.data_ptr(),
                            out.data_ptr(), 0, M, N, K, epilogue, *ws, stream)


def _both(lib, M, N, K, epilogue, seed):
    from joyomni_ops import _lib
    a, w, sa, sw, bias = _problem(M, N, K, seed)
    need = lib.joy_fp8_scaled_mm_workspace_size(M, N, K)
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=DEV)
    ref = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
    got = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
    _lib.check(lib, _call(lib, "joy_fp8_scaled_mm", a, w, sa, sw, bias, ref, M, N, K, epilogue,
                          ws.data_ptr(), need))
    _lib.check(lib, _call(lib, "joy_fp8_scaled_mm_noalloc", a, w, sa, sw, bias, got, M, N, K, epilogue))
    torch.cuda.synchronize()
    return need, ref, got


def test_noalloc_first_call_captured_in_a_graph():
    """The first joy_fp8_scaled_mm_noalloc call of the process, captured into a HIP graph after
    joy_init() (which resolves the scratch address, so the captured call makes no runtime query),
    replayed three times with eager work between the replays (a NaN fill of the output and an
    eager no-alloc call on another problem, which leaves other partial sums in the scratch):
    every replay equals the workspace entry point bit for bit. A split-K plan, so the replays
    read and write the scratch. This test runs before the file's other no-alloc calls."""
    import joyomni_ops as jo
    from joyomni_ops import _lib
    lib = jo._LIB
    _lib.check(lib, lib.joy_init())
    M, N, K = 256, 5136, 5120
    announce("noalloc gemm under graph capture", M, N, K)
    a, w, sa, sw, bias = _problem(M, N, K, 300)
    need = lib.joy_fp8_scaled_mm_workspace_size(M, N, K)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    ref = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    _lib.check(lib, _call(lib, "joy_fp8_scaled_mm", a, w, sa, sw, bias, ref, M, N, K, 0, ws.data_ptr(), need))
    got = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
    other = _problem(64, 5120, 5120, 301)
    other_out = torch.empty((64, 5120), dtype=torch.bfloat16, device=DEV)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            _lib.check(lib, _call(lib, "joy_fp8_scaled_mm_noalloc", a, w, sa, sw, bias, got, M, N, K, 0))
    torch.cuda.synchronize()
    for i in range(3):
        got.fill_(float("nan"))
        _lib.check(lib, _call(lib, "joy_fp8_scaled_mm_noalloc", *other, other_out, 64, 5120, 5120, 0))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"replay {i}"


def test_noalloc_matches_workspace_entry_point():
    import joyomni_ops as jo
    lib = jo._LIB
    cases = [(256, 5136, 5120, 0), (64, 5120, 5120, 1), (96, 2048, 4096, 0), (1024, 512, 512, 0),
             (512, 5120, 5120, 0)]
    splits_seen = 0
    for i, (M, N, K, epi) in enumerate(cases):
        announce("noalloc gemm", M, N, K, epi)
        need, ref, got = _both(lib, M, N, K, epi, 100 + i)
        assert need <= jo._lib.JOY_FP8_NOALLOC_SCRATCH_BYTES
        splits_seen += need > 0
        assert not torch.isnan(ref.float()).any()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), (M, N, K)
    assert splits_seen >= 3  # the first three problems take split-K plans (the scratch is used); the
    # last one the narrow-tile plan (no split, no scratch)


def test_noalloc_uses_the_whole_scratch_and_every_plan_fits():
    """A split plan needs at most (CUs / tiles) * tiles * 128 x 256 x 4 bytes = CUs * 128 KiB, the
    32 MiB of the scratch on a 256-CU MI355X: 512 x 4096 x 8192 needs all of it and still matches
    the workspace entry point bit for bit; no small-M shape of the sweep needs more."""
    import joyomni_ops as jo
    from joyomni_ops import _lib
    lib = jo._LIB
    cap = _lib.JOY_FP8_NOALLOC_SCRATCH_BYTES
    worst = max(lib.joy_fp8_scaled_mm_workspace_size(m, n, k) for m in range(16, 513, 16)
                for n in (512, 1024, 2048, 3072, 4096, 5120, 8192, 13824, 15360) for k in (4096, 5120, 8192, 13824))
    assert 0 < worst <= cap, worst
    M, N, K = 512, 4096, 8192
    announce("noalloc gemm full scratch", M, N, K)
    need, ref, got = _both(lib, M, N, K, 0, 200)
    assert 0 < need <= worst <= cap, (need, worst, cap)
    # the bound is "every plan fits"; on a 256-CU MI355X the largest plan fills the scratch exactly
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert need == worst == cap, (need, worst, cap)
    assert not torch.isnan(ref.float()).any()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
