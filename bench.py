"""Benchmark of the MI355X quantised DiT hot path (one JSON line on stdout).

Headline (``value``): benchmark cfg 1 -- fused QKV split + per-head q/k RMSNorm +
3-D RoPE + 4-slot KV-ring write over L=10800 tokens, 40x128 heads, in GB/s of
algorithmic HBM traffic. One step = one launch over the whole chunk, inputs
resident in HBM. Also reported in the same line: the cfg 2 FP8 GEMM sweep at
M=10800 (TFLOP/s, fraction of dense FP8 MFMA peak), the cfg 3 small-M GEMMs
(GB/s) and the activation quantiser (GB/s), each timed with HIP events on the
launch stream, plus the reference's CPU torch path timed on the host cores on a
bounded sample (``cpu_baseline``).

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--no-cpu] [--only qkv|gemm|...]
       [--tunableop results.csv]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "joyai-video-edit_amd"))
sys.path.insert(0, ROOT)

METRIC = "FP8 GEMM TFLOP/s (% fp8 MFMA peak); QKV-norm-RoPE GB/s (% HBM peak)"
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E, AMD published
PEAK_FP8_TFLOPS = 5000.0      # MI355X dense FP8 MFMA, AMD published (no sparsity)
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA, AMD published (no sparsity)

L_TOK, HEADS, HEAD_DIM = 10800, 40, 128
E = HEADS * HEAD_DIM
RING_SLOTS, SLOT = 4, 1
GEMM_SHAPES = [("qkv", 5120, 15360), ("out_proj", 5120, 5120), ("ffn_up", 5120, 13824),
               ("ffn_down", 13824, 5120)]
SMALL_M = [64, 256, 512]


def qkv_bytes(L: int) -> int:
    """Algorithmic bytes of one fused launch: read q,k,v (bf16) + cos/sin half tables +
    q/k weights; write q_rope, k_rope, k_pre -> cache, v -> cache."""
    return 3 * L * E * 2 + L * (HEAD_DIM // 2) * 2 * 2 + 2 * HEAD_DIM * 2 + 4 * L * E * 2


def gemm_bytes(M, N, K) -> int:
    return M * K + K * N + 2 * M * N + 4 * M + 4 * N + 2 * N


def quant_bytes(M, K) -> int:
    return 2 * M * K + M * K + 4 * M


EAGER = False  # --eager: plain launches instead of one HIP graph (for counter runs)
STEADY_S = 0.05  # seconds of back-to-back replays before each timed replay

# MI355X has a 256 MiB memory-side cache (MALL) in front of HBM: a launch whose working set fits
# in it, replayed on the same buffers, is partly served from it. Memory-bound benchmarks whose
# working set is smaller than this cycle through enough independent buffer sets that each set
# is evicted before it is used again.
MALL_BYTES = 256 << 20


def buffer_sets(bytes_per_set: int) -> int:
    """Number of buffer sets so that the sets together span >= 3 x the MALL."""
    return max(1, -(-3 * MALL_BYTES // max(1, bytes_per_set)))


class Rotation:
    """Calls fn(set) on successive sets; each call during graph capture bakes in its own set.
    With keep=True the tensor each call returns stays alive until the same set comes round
    again, so an op that allocates its output writes a different buffer on every call of a
    rotation (otherwise the allocator hands the same block back each time and the output can
    stay resident in the MALL)."""

    def __init__(self, sets, fn, keep=False):
        self.sets, self.fn, self.i = sets, fn, 0
        self.kept = [None] * len(sets) if keep else None

    def __call__(self):
        j = self.i % len(self.sets)
        r = self.fn(self.sets[j])
        if self.kept is not None:
            self.kept[j] = r
        self.i += 1


def time_launches(fn, steps: int, warmup: int):
    """Average per-launch time (s) of `fn` (one kernel launch) over `steps` launches.

    The `steps` launches are captured once into a HIP graph on a side stream and
    the graph is replayed between two events recorded on that same stream, so the
    figure is device time without Python dispatch gaps. Before the timed replay the
    graph is replayed back to back for at least STEADY_S seconds: after any pause
    (host-side set-up of the next case) the part takes ~30 ms of continuous load to
    settle its clock, and a GEMM timed inside that window ran 10-20 % slower than
    at steady state, which penalised whichever leg of a comparison ran first.
    Falls back to eager launches on the current stream if capture is refused.
    """
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    if EAGER:
        return _time_eager(fn, steps)
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    try:
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                for _ in range(steps):
                    fn()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):  # replay runs on the current stream
            start.record(stream)
            graph.replay()  # warm replay
            end.record(stream)
            torch.cuda.synchronize()
            warm = max(0, min(400, int(STEADY_S / max(start.elapsed_time(end) / 1e3, 1e-6))))
            for _ in range(warm):  # back to back until the clock has settled
                graph.replay()
            start.record(stream)
            graph.replay()
            end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / 1e3 / steps
    except Exception as exc:  # pragma: no cover - capture refused
        print(f"bench: graph capture failed ({exc!r}); timing eager launches", file=sys.stderr)
    return _time_eager(fn, steps)


def _time_eager(fn, steps: int):
    import torch
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3 / steps


class TunedReference:
    """PyTorch TunableOp around a reference torch._scaled_mm leg, with the reference's own settings
    (deploy/tune_rocm_fp8.py:46-66: tuning on, untuned-GEMM recording off, at most 10 ms and 30
    iterations per candidate). The first call of each shape inside the context tunes it (the
    warm-up calls of time_launches, before the graph capture); TunableOp is switched off again on
    exit, so the untuned legs elsewhere keep hipBLASLt's default selection. The deployment loads
    the table with tuning off (serve_joyomni_streaming.py:77-102): the same kernels, chosen here
    in-process instead of from a file."""

    configured = False

    @classmethod
    def configure(cls, csv=None):
        from torch.cuda import tunable
        import tempfile
        path = csv or os.path.join(tempfile.gettempdir(), f"joy_bench_tunableop_{os.getpid()}.csv")
        # results go to that file at exit (a temporary one unless --tunableop names one)
        tunable.set_filename(path, insert_device_ordinal=False)
        tunable.record_untuned_enable(False)
        tunable.set_max_tuning_duration(10)
        tunable.set_max_tuning_iterations(30)
        cls.configured = True

    def __enter__(self):
        from torch.cuda import tunable
        if not TunedReference.configured:
            TunedReference.configure()
        tunable.enable(True)
        tunable.tuning_enable(True)
        return self

    def __exit__(self, *exc):
        from torch.cuda import tunable
        tunable.tuning_enable(False)
        tunable.enable(False)
        return False


def progress(msg: str) -> None:
    """One line on stderr per finished section, so a long run shows it is alive."""
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def load_traffic(name: str):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    calibrated on a copy kernel), committed as profiles/hbm_traffic.json."""
    p = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get(name, {}).get("bytes_per_launch")


def bench_qkv(steps, warmup):
    import torch
    import joyomni_ops as jo
    from joyomni_ops.rope import rope_3d_half_tables
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(0)
    qkv = torch.randn(L_TOK, 3 * E, generator=g).to(torch.bfloat16).to(dev)
    qw = (1 + 0.1 * torch.randn(HEAD_DIM, generator=g)).to(torch.bfloat16).to(dev)
    kw = (1 + 0.1 * torch.randn(HEAD_DIM, generator=g)).to(torch.bfloat16).to(dev)
    cos, sin = rope_3d_half_tables(3, 45, 80, (44, 42, 42), 10000.0, device=dev)
    q_out = torch.empty(L_TOK, HEADS, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    k_out = torch.empty_like(q_out)
    ck = torch.empty(RING_SLOTS, L_TOK, HEADS, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    cv = torch.empty_like(ck)

    def step():
        jo.fused_qkv_norm_rope_cache(qkv, HEADS, 1e-6, qw, kw, cos, sin, q_out, k_out, ck, cv, SLOT, 0)

    t = time_launches(step, steps, warmup)
    return t, qkv_bytes(L_TOK)


def bench_qkv_projection(steps, warmup):
    """The video stream's QKV projection at the block's size (10800 tokens, K 5120, N 3 x 40 x 128)
    with its q/k RMSNorm, RoPE and KV-ring write, as one op (fp8_qkv_norm_rope_cache: the norm, the
    rotation and the ring write in the GEMM's epilogue) and as the two-op sequence it replaces
    (fp8_scaled_mm into a bf16 [M, 3E] buffer, then fused_qkv_norm_rope_cache on it; dit.py:409-451),
    with the GEMM alone beside them. Q, K and V go into views of joint buffers behind 21600 cached rows
    and the ring slot, as in the block."""
    import torch
    import joyomni_ops as jo
    dev = torch.device("cuda:0")
    M, K, N = L_TOK, E, 3 * E
    g = torch.Generator().manual_seed(3)
    x = outlier_acts(M, K, g).to(dev)
    wf = (0.02 * torch.randn(N, K, generator=g)).to(torch.bfloat16).to(dev)
    a, sa = jo_quant(x)
    w, sw = jo_quant(wf)
    b, swr = w.t(), sw.reshape(1, N)
    bias = (0.01 * torch.randn(N, generator=g)).to(torch.bfloat16).to(dev)
    qw = (1 + 0.1 * torch.randn(HEAD_DIM, generator=g)).to(torch.bfloat16).to(dev)
    kw = (1 + 0.1 * torch.randn(HEAD_DIM, generator=g)).to(torch.bfloat16).to(dev)
    from joyomni_ops.rope import rope_3d_half_tables
    cos, sin = rope_3d_half_tables(3, 45, 80, (44, 42, 42), 10000.0, device=dev)
    C = 2 * L_TOK
    q = torch.empty(1, M + 512, HEADS, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    kk = torch.empty(1, C + M + 512, HEADS, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    vv = torch.empty_like(kk)
    ck = torch.empty(RING_SLOTS, M, HEADS, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    cv = torch.empty_like(ck)
    outs = (q[0, :M], kk[0, C:C + M], ck, cv, SLOT, 0)

    def two_op():
        y = jo.fp8_scaled_mm(a, b, sa, swr, torch.bfloat16, bias)
        jo.fused_qkv_norm_rope_cache(y, HEADS, 1e-6, qw, kw, cos, sin, *outs, v_out=vv[0, C:C + M])

    def fused():
        jo.fp8_qkv_norm_rope_cache(a, b, sa, swr, bias, HEADS, 1e-6, qw, kw, cos, sin, *outs, v_out=vv[0, C:C + M])

    def gemm_only():
        jo.fp8_scaled_mm(a, b, sa, swr, torch.bfloat16, bias)

    n = min(steps, 20)
    res = {}
    for name, fn in (("two_op", two_op), ("fused", fused), ("gemm_only", gemm_only)):
        res[name + "_us"] = time_launches(fn, n, warmup) * 1e6
    res["shape"] = f"M{M} K{K} N{N}"
    res["fused_speedup_vs_two_op"] = res["two_op_us"] / res["fused_us"]
    res["fused_tflops"] = 2.0 * M * N * K / (res["fused_us"] * 1e-6) / 1e12
    return res


def bench_gemm(steps, warmup):
    import torch
    import joyomni_ops as jo
    dev = torch.device("cuda:0")
    res = []
    for name, K, N in GEMM_SHAPES:
        g = torch.Generator().manual_seed(K + N)
        M = L_TOK
        # benchmark cfg 2 draws its operands like cfg 0: activations N(0,1) with 0.5 % of the
        # channels scaled x20 (outliers), weights N(0, 0.02)
        x = outlier_acts(M, K, g).to(dev)
        w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(dev)
        bias = (torch.randn(N, generator=g) * 0.01).to(torch.bfloat16).to(dev)
        qa = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=dev)
        sa = torch.empty(M, 1, device=dev)
        qw = torch.empty(N, K, dtype=torch.float8_e4m3fn, device=dev)
        sw = torch.empty(N, 1, device=dev)
        jo.per_token_quant_fp8(x, qa, sa, True)
        jo.per_token_quant_fp8(w, qw, sw, True)
        swr = sw.reshape(1, N)
        wt = qw.t()
        fn = jo.fp8_scaled_mm_gelu_tanh if name == "ffn_up" else jo.fp8_scaled_mm
        t = time_launches(lambda: fn(qa, wt, sa, swr, torch.bfloat16, bias), steps, warmup)
        flops = 2 * M * N * K
        rec = {"shape": name, "M": M, "K": K, "N": N, "ms": t * 1e3,
               "tflops": flops / t / 1e12, "frac_fp8_peak": flops / t / 1e12 / PEAK_FP8_TFLOPS,
               "epilogue": "bias+gelu_tanh" if name == "ffn_up" else "bias",
               "reference_path": "_scaled_mm + F.gelu" if name == "ffn_up" else "_scaled_mm"}
        # the reference's own ROCm GEMM call (fp8_linear.py:124-132 -> hipBLASLt), same inputs; for
        # FFN-up the reference then applies F.gelu(approximate="tanh") as its own kernel (dit.py:87-89)
        def reference_path():
            y = torch._scaled_mm(qa, wt, scale_a=sa, scale_b=swr, bias=bias, out_dtype=torch.bfloat16,
                                 use_fast_accum=True)
            if name == "ffn_up":
                y = torch.nn.functional.gelu(y, approximate="tanh")
            return y
        try:
            tr = time_launches(reference_path, steps, warmup)
            rec["reference_hipblaslt_tflops"] = flops / tr / 1e12
            rec["speedup_vs_reference_gpu"] = tr / t
            with TunedReference():
                tt = time_launches(reference_path, steps, warmup)
            rec["reference_hipblaslt_tuned_tflops"] = flops / tt / 1e12
            rec["speedup_vs_reference_gpu_tuned"] = tt / t
        except Exception as exc:  # pragma: no cover - depends on the torch build
            rec["reference_hipblaslt_tflops"] = None
            rec["reference_hipblaslt_error"] = str(exc)[:200]
        res.append(rec)
        progress(f"cfg2 {name} {M}x{K}x{N}: {t * 1e6:.1f} us, {rec['tflops']:.0f} TFLOP/s "
                 f"({rec['frac_fp8_peak']:.3f} of FP8 peak); hipBLASLt {rec.get('reference_hipblaslt_tflops') or 0:.0f}, "
                 f"tuned {rec.get('reference_hipblaslt_tuned_tflops') or 0:.0f} TFLOP/s")
        del x, w, qa, qw
    tot_flops = sum(2 * r["M"] * r["N"] * r["K"] for r in res)
    tot_t = sum(r["ms"] for r in res) / 1e3
    ref_t = [2 * r["M"] * r["N"] * r["K"] / r["reference_hipblaslt_tflops"] / 1e12
             for r in res if r.get("reference_hipblaslt_tflops")]
    ref_agg = tot_flops / sum(ref_t) / 1e12 if len(ref_t) == len(res) else None
    tuned_t = [2 * r["M"] * r["N"] * r["K"] / r["reference_hipblaslt_tuned_tflops"] / 1e12
               for r in res if r.get("reference_hipblaslt_tuned_tflops")]
    tuned_agg = tot_flops / sum(tuned_t) / 1e12 if len(tuned_t) == len(res) else None
    return res, tot_flops / tot_t / 1e12, ref_agg, tuned_agg


def outlier_acts(M, K, g):
    """Benchmark cfg 0 activations (also cfg 2's, "same seeded distributions as config 0"):
    N(0,1) bf16 with 0.5 % of the channels scaled x20."""
    import torch
    x = torch.randn(M, K, generator=g)
    x[:, torch.randperm(K, generator=g)[: K // 200]] *= 20
    return x.to(torch.bfloat16)


def bench_cfg0(steps, warmup):
    """Benchmark cfg 0: one Fp8Linear forward (per-token activation quant + FP8 GEMM + bias) at
    256 x 4096 -> 4096, the shape the CPU baseline times; W streams from HBM (rotated copies)."""
    import torch
    import joyomni_ops as jo
    from joyomni_ops.fp8_linear import Fp8Linear
    dev = torch.device("cuda:0")
    M, K, N = 256, 4096, 4096
    g = torch.Generator().manual_seed(0)
    x = torch.randn(M, K, generator=g)
    x[:, torch.randperm(K, generator=g)[: K // 200]] *= 20
    x = x.to(torch.bfloat16).to(dev)
    lin = torch.nn.Linear(K, N)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(N, K, generator=g) * 0.02)
        lin.bias.copy_(torch.randn(N, generator=g) * 0.01)
    layers = [Fp8Linear.from_linear(lin.to(torch.bfloat16).to(dev))]
    layers += [Fp8Linear(layers[0].weight_fp8.clone(), layers[0].weight_scale, layers[0].bias)
               for _ in range(buffer_sets(N * K) - 1)]
    t = time_launches(Rotation(layers, lambda f: f(x)), steps, warmup)
    qx, sx = jo_quant(x)
    t_mm = time_launches(Rotation(layers, lambda f: jo.fp8_scaled_mm(
        qx, f.weight_fp8, sx, f.weight_scale, torch.bfloat16, f.bias)), steps, warmup)
    return {"workload": f"cfg0 Fp8Linear forward {M}x{K} -> {N} (act quant + GEMM + bias)", "us": t * 1e6,
            "tflops": 2 * M * N * K / t / 1e12, "gbs": gemm_bytes(M, N, K) / t / 1e9,
            "weight_copies": len(layers), "gemm_only_us": t_mm * 1e6}


def jo_quant(x):
    import torch
    import joyomni_ops as jo
    q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty(x.shape[0], 1, device=x.device)
    jo.sgl_per_token_quant_fp8(x, q, s)
    return q, s


def bench_clock(steps, warmup):
    """The QKV GEMM (cfg 2) launched back to back on the bench's random operands, then on all-zero
    operands, then on the random ones again; each launch timed with HIP events on the stream. Under
    rocprofv3 --pmc SQ_BUSY_CYCLES the per-dispatch busy cycles over these durations give the shader
    clock per operand kind (the part is power-limited; switching activity sets the clock)."""
    import torch
    import joyomni_ops as jo
    dev = torch.device("cuda:0")
    M, K, N = L_TOK, 5120, 15360
    g = torch.Generator().manual_seed(K + N)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    bias = (torch.randn(N, generator=g) * 0.01).to(torch.bfloat16).to(dev)
    qa, sa = jo_quant(x)
    qw, sw = jo_quant(w)
    za, zw = torch.zeros_like(qa), torch.zeros_like(qw)
    stream = torch.cuda.current_stream()
    out = {}
    for name, a, b in (("random", qa, qw), ("zeros", za, zw), ("random_again", qa, qw)):
        for _ in range(warmup):
            jo.fp8_scaled_mm(a, b.t(), sa, sw.reshape(1, N), torch.bfloat16, bias)
        ts = []
        for _ in range(steps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            jo.fp8_scaled_mm(a, b.t(), sa, sw.reshape(1, N), torch.bfloat16, bias)
            e1.record(stream)
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e3)
        out[name] = {"us": ts, "median_us": sorted(ts)[len(ts) // 2]}
    return {"workload": f"QKV GEMM {M}x{K}x{N}, bf16 out + bias", "launches": out}


# The reference's own production GEMM shapes (M, K, N), tuned for gfx950 by
# deploy/tune_rocm_fp8.py:23-36 (hidden 4096, FFN 16384).
REFERENCE_TUNED_SHAPES = [(m, k, n) for m in (1024, 1560, 3120)
                          for k, n in ((4096, 12288), (4096, 4096), (4096, 16384), (16384, 4096))]


def bench_reference_shapes(steps, warmup):
    """This kernel vs the reference's ROCm GEMM (torch._scaled_mm -> hipBLASLt, fp8_linear.py:124-132)
    on the reference's tuned shapes; each launch reads a different weight copy (as consecutive layers do)."""
    import torch
    import joyomni_ops as jo
    dev = torch.device("cuda:0")
    out = []
    for M, K, N in REFERENCE_TUNED_SHAPES:
        g = torch.Generator().manual_seed(M + K + N)
        x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
        w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(dev)
        bias = (torch.randn(N, generator=g) * 0.01).to(torch.bfloat16).to(dev)
        qa = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=dev)
        sa = torch.empty(M, 1, device=dev)
        qw = torch.empty(N, K, dtype=torch.float8_e4m3fn, device=dev)
        sw = torch.empty(N, 1, device=dev)
        jo.per_token_quant_fp8(x, qa, sa, True)
        jo.per_token_quant_fp8(w, qw, sw, True)
        del x, w
        weights = [qw] + [qw.clone() for _ in range(buffer_sets(N * K) - 1)]
        swr = sw.reshape(1, N)
        t = time_launches(Rotation(weights, lambda q: jo.fp8_scaled_mm(qa, q.t(), sa, swr, torch.bfloat16, bias)),
                          steps, warmup)
        def reference_path():
            return time_launches(Rotation(weights, lambda q: torch._scaled_mm(
                qa, q.t(), scale_a=sa, scale_b=swr, bias=bias, out_dtype=torch.bfloat16, use_fast_accum=True)),
                steps, warmup)
        tr = reference_path()
        with TunedReference():  # the table the reference deploys for exactly these shapes
            tt = reference_path()
        flops = 2 * M * N * K
        out.append({"M": M, "K": K, "N": N, "us": t * 1e6, "tflops": flops / t / 1e12,
                    "reference_hipblaslt_us": tr * 1e6, "reference_hipblaslt_tflops": flops / tr / 1e12,
                    "speedup_vs_reference_gpu": tr / t, "reference_hipblaslt_tuned_us": tt * 1e6,
                    "speedup_vs_reference_gpu_tuned": tt / t})
        progress(f"refgemm {M}x{K}x{N}: {t * 1e6:.1f} us; hipBLASLt {tr * 1e6:.1f} us, tuned {tt * 1e6:.1f} us "
                 f"({tt / t:.3f}x)")
        del weights
    return out


def bench_small_m(steps, warmup):
    """cfg 3: the weights dominate the bytes; each launch reads a different copy of W (as
    consecutive layers do), so W streams from HBM rather than from the MALL."""
    import torch
    import joyomni_ops as jo
    dev = torch.device("cuda:0")
    out = []
    for N in (15360, 5120):
        K = 5120
        g = torch.Generator().manual_seed(N)
        w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(dev)
        qw0 = torch.empty(N, K, dtype=torch.float8_e4m3fn, device=dev)
        sw = torch.empty(N, 1, device=dev)
        jo.per_token_quant_fp8(w, qw0, sw, True)
        del w
        weights = [qw0] + [qw0.clone() for _ in range(buffer_sets(N * K) - 1)]
        bias = torch.zeros(N, dtype=torch.bfloat16, device=dev)
        for M in SMALL_M:
            x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
            qa = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=dev)
            sa = torch.empty(M, 1, device=dev)
            jo.per_token_quant_fp8(x, qa, sa, True)
            step = Rotation(weights, lambda qw: jo.fp8_scaled_mm(qa, qw.t(), sa, sw.reshape(1, N),
                                                                 torch.bfloat16, bias))
            t = time_launches(step, steps, warmup)
            # the reference's ROCm GEMM (torch._scaled_mm -> hipBLASLt, fp8_linear.py:124-132), same rotation
            tr = time_launches(Rotation(weights, lambda qw: torch._scaled_mm(
                qa, qw.t(), scale_a=sa, scale_b=sw.reshape(1, N), bias=bias, out_dtype=torch.bfloat16,
                use_fast_accum=True)), steps, warmup)
            b = gemm_bytes(M, N, K)
            flops = 2 * M * N * K
            # the binding roof: HBM below the ridge point (625 FLOP/B), the FP8 MFMA peak above it
            t_roof = max(b / (PEAK_HBM_GBS * 1e9), flops / (PEAK_FP8_TFLOPS * 1e12))
            bound = "hbm" if b / (PEAK_HBM_GBS * 1e9) >= flops / (PEAK_FP8_TFLOPS * 1e12) else "mfma"
            out.append({"M": M, "K": K, "N": N, "us": t * 1e6, "gbs": b / t / 1e9,
                        "frac_hbm_peak": b / t / 1e9 / PEAK_HBM_GBS, "tflops": flops / t / 1e12,
                        "flop_per_byte": flops / b, "roofline_bound": bound, "frac_roofline": t_roof / t,
                        "weight_copies": len(weights),
                        "reference_hipblaslt_us": tr * 1e6, "speedup_vs_reference_gpu": tr / t})
            progress(f"cfg3 M {M} x N {N}: {t * 1e6:.1f} us ({bound}-bound, {t_roof / t:.3f} of roofline); "
                     f"hipBLASLt {tr * 1e6:.1f} us")
        del weights
    return out


def bench_quant(steps, warmup):
    import torch
    import joyomni_ops as jo
    dev = torch.device("cuda:0")
    out = []
    for K in (5120, 13824):
        M = L_TOK
        b = quant_bytes(M, K)
        x0 = torch.randn(M, K, generator=torch.Generator().manual_seed(K)).to(torch.bfloat16).to(dev)
        sets = [(x0 if i == 0 else x0.clone(), torch.empty(M, K, dtype=torch.float8_e4m3fn, device=dev),
                 torch.empty(M, 1, device=dev)) for i in range(buffer_sets(b))]
        t = time_launches(Rotation(sets, lambda st: jo.per_token_quant_fp8(st[0], st[1], st[2], True)),
                          steps, warmup)
        out.append({"M": M, "K": K, "us": t * 1e6, "gbs": b / t / 1e9, "frac_hbm_peak": b / t / 1e9 / PEAK_HBM_GBS,
                    "buffer_sets": len(sets)})
        del sets, x0
    return out


def bench_pack(steps, warmup):
    """Cache read side at cfg-4 geometry: fused_cached_kv_pack over two KV-ring
    slots (2 x 10800 tokens, fp32 full-width tables) and fused_joint_qkv_pack of
    3 cached chunks + 10800 video tokens (strided views of the QKV GEMM row) +
    512 condition tokens (two-rounding RMSNorm)."""
    import torch
    import joyomni_ops as jo
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(3)
    L, T, C = L_TOK, 512, 3 * L_TOK
    ring_k = torch.randn(RING_SLOTS, L, HEADS, HEAD_DIM, generator=g).to(torch.bfloat16).to(dev)
    ring_v = torch.randn(RING_SLOTS, L, HEADS, HEAD_DIM, generator=g).to(torch.bfloat16).to(dev)
    cos = torch.rand(2 * L, HEAD_DIM, generator=g).to(dev)
    sin = torch.rand(2 * L, HEAD_DIM, generator=g).to(dev)
    out = []
    t = time_launches(lambda: jo.fused_cached_kv_pack(ring_k[2][None], ring_v[2][None], ring_k[0][None],
                                                      ring_v[0][None], cos, sin), steps, warmup)
    b = 2 * (2 * L) * E * 2 + 2 * (2 * L) * HEAD_DIM * 4 + 2 * (2 * L) * E * 2
    out.append({"op": "fused_cached_kv_pack", "tokens": 2 * L, "us": t * 1e6, "gbs": b / t / 1e9,
                "frac_hbm_peak": b / t / 1e9 / PEAK_HBM_GBS, "algorithmic_bytes": b})
    img = torch.randn(L, 3 * E, generator=g).to(torch.bfloat16).to(dev).view(1, L, 3, HEADS, HEAD_DIM)
    txt = torch.randn(T, 3 * E, generator=g).to(torch.bfloat16).to(dev).view(1, T, 3, HEADS, HEAD_DIM)
    w = torch.ones(HEAD_DIM, dtype=torch.bfloat16, device=dev)
    ck = ring_k[:3].reshape(1, C, HEADS, HEAD_DIM)
    cv = ring_v[:3].reshape(1, C, HEADS, HEAD_DIM)
    t = time_launches(lambda: jo.fused_joint_qkv_pack(img[:, :, 0], img[:, :, 1], img[:, :, 2], txt[:, :, 0],
                                                      txt[:, :, 1], txt[:, :, 2], ck, cv, w, w, 1e-6),
                      steps, warmup)
    b = (3 * (L + T) + 2 * C) * E * 2 + 2 * HEAD_DIM * 2 + ((L + T) + 2 * (C + L + T)) * E * 2
    out.append({"op": "fused_joint_qkv_pack", "tokens": {"cache": C, "video": L, "condition": T},
                "us": t * 1e6, "gbs": b / t / 1e9, "frac_hbm_peak": b / t / 1e9 / PEAK_HBM_GBS,
                "algorithmic_bytes": b})
    return out


def bench_norm(steps, warmup):
    """adaLN LayerNorm + modulation at cfg-4 geometry (M = 10800 tokens, hidden 5120, one
    broadcast modulation row): the plain op (bf16 out) and the FP8-emitting variant that
    replaces norm -> bf16 -> per-token quant. Buffer sets rotate past the MALL."""
    import torch
    import joyomni_ops as jo
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(4)
    M, N = L_TOK, E
    x0 = torch.randn(M, N, generator=g).to(torch.bfloat16).to(dev)
    sc = (0.2 * torch.randn(1, N, generator=g)).to(torch.bfloat16).to(dev)
    sh = (0.2 * torch.randn(1, N, generator=g)).to(torch.bfloat16).to(dev)
    out = []
    b = 2 * M * N + 2 * M * N + 2 * 2 * N
    xs = [x0] + [x0.clone() for _ in range(buffer_sets(b) - 1)]
    t = time_launches(Rotation(xs, lambda x: jo.fused_norm_scale_shift(x, None, None, sc, sh, "layer", 1e-6),
                               keep=True), steps, warmup)
    out.append({"op": "fused_norm_scale_shift", "M": M, "N": N, "us": t * 1e6, "gbs": b / t / 1e9,
                "frac_hbm_peak": b / t / 1e9 / PEAK_HBM_GBS, "algorithmic_bytes": b, "buffer_sets": len(xs)})
    for exact in (False, True):
        b = 2 * M * N + M * N + 4 * M + 2 * 2 * N
        sets = [(x, torch.empty(M, N, dtype=torch.float8_e4m3fn, device=dev), torch.empty(M, 1, device=dev))
                for x in xs[:buffer_sets(b)]]
        t = time_launches(Rotation(sets, lambda st: jo.fused_norm_scale_shift_fp8(
            st[0], None, None, sc, sh, "layer", 1e-6, st[1], st[2], None, exact)), steps, warmup)
        out.append({"op": "fused_norm_scale_shift_fp8", "rounding": "division" if exact else "reciprocal",
                    "M": M, "N": N, "us": t * 1e6, "gbs": b / t / 1e9,
                    "frac_hbm_peak": b / t / 1e9 / PEAK_HBM_GBS, "algorithmic_bytes": b, "buffer_sets": len(sets)})
        del sets
    return out


def bench_block(steps, warmup, n_cached=2, attention_backend="hip"):
    """Benchmark cfg 4: one two-stream MMDiT block's quantised chain, video 10800 + condition 512
    tokens, hidden 5120, 40 x 128 heads, FFN 13824, random-init weights; the video chunk's K/V go
    into ring slot 0 and the block attends to ``n_cached`` cached chunks of 10800 tokens read from
    other ring slots (rotated on read into joint K / V buffers that persist across calls: the
    latency is that of a call reusing the assembled cached rows, as the denoising steps after the
    first on a chunk, and the first step's, which assembles them, is reported beside it). Per-stage
    device time from HIP events on the launch stream,
    for a block queued behind two others (the host runs ahead of the device, as within a forward);
    SDPA is reported separately (excluded from kernel time, included in block latency)."""
    import torch
    from joyomni_ops.dit_block import CachedChunk, JointKV, KVRing, QuantizedDoubleStreamBlock
    from joyomni_ops.rope import rope_3d_half_tables, rotary_pos_embed_3d
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(5)
    T_COND, FFN = 512, 13824
    blk = QuantizedDoubleStreamBlock(E, HEADS, FFN, dev, g, attention_backend=attention_backend)
    img = torch.randn(1, L_TOK, E, generator=g).to(torch.bfloat16).to(dev)
    txt = torch.randn(1, T_COND, E, generator=g).to(torch.bfloat16).to(dev)
    vec = torch.randn(1, E, generator=g).to(torch.bfloat16).to(dev)
    frames = torch.arange(3 * n_cached, 3 * n_cached + 3)
    cos, sin = rope_3d_half_tables(3, 45, 80, (44, 42, 42), 10000.0, device=dev, frame_ids=frames)
    ring = KVRing(RING_SLOTS, L_TOK, HEADS, HEAD_DIM, dev)
    cached = []
    # one full-width table over every cached token, cut into the chunks' rows (the reference builds
    # cached_freqs_cis once per forward for all blocks, dit.py:1196-1217)
    cf_all, sf_all = rotary_pos_embed_3d(torch.arange(0, 3 * n_cached), 45, 80, (44, 42, 42), 10000.0)
    cf_all, sf_all = cf_all.contiguous().to(dev), sf_all.contiguous().to(dev)
    for c in range(n_cached):
        slot = RING_SLOTS - 1 - c
        ring.k[slot].normal_()
        ring.v[slot].normal_()
        ring.lengths[slot] = L_TOK
        rows = slice(c * L_TOK, (c + 1) * L_TOK)
        cached.append(CachedChunk(slot, cf_all[rows], sf_all[rows]))
    stages = ["qkv", "qkv_norm_rope", "cached_kv", "joint_pack", "attention", "proj_ffn"]
    stream = torch.cuda.current_stream()
    ev = {}

    def mark(name):
        ev[name].record(stream)

    # the joint K / V buffers persist across calls, as across the denoising steps of a chunk: the
    # cached chunks' rows are assembled by the first call and reused by the next ones (the
    # reference memoises the same assembly, dit.py:1168-1217); ``first`` forces the assembly
    joint = JointKV()

    def run(timed, first=False):
        if first:
            joint.invalidate()
        if timed:
            ev["start"].record(stream)
        blk.forward(img, txt, vec, cos, sin, ring=ring, write_slot=0, cached=cached,
                    mark=mark if timed else None, joint=joint)

    for _ in range(warmup):
        run(False)
    torch.cuda.synchronize()
    acc = {k: 0.0 for k in stages}
    acc_first = {k: 0.0 for k in stages}
    lat = lat_first = 0.0
    for _ in range(steps):
        ev = {k: torch.cuda.Event(enable_timing=True) for k in ["start"] + stages}
        e0, e1, e2, e3 = (torch.cuda.Event(enable_timing=True) for _ in range(4))
        # each timed block is queued behind two untimed ones, as consecutive blocks of a forward
        # run: its stages start on a busy device (settled clock, no host launch gaps inside it).
        # The latency comes from a block bracketed by two events only: every event recorded
        # between kernels leaves the device idle for ~5.5 us (kernel trace), so the block with
        # the per-stage events gives the stage split, not the latency.
        run(False)
        run(False)
        run(True)
        run(False)
        e0.record(stream)
        run(False)
        e1.record(stream)
        torch.cuda.synchronize()
        lat += e0.elapsed_time(e1)
        prev = "start"
        for k in stages:
            acc[k] += ev[prev].elapsed_time(ev[k])
            prev = k
        # the first call on a chunk's cached rows: they are assembled inside the block
        ev = {k: torch.cuda.Event(enable_timing=True) for k in ["start"] + stages}
        run(False)
        run(True, first=True)
        run(False)
        e2.record(stream)
        run(False, first=True)
        e3.record(stream)
        torch.cuda.synchronize()
        lat_first += e2.elapsed_time(e3)
        prev = "start"
        for k in stages:
            acc_first[k] += ev[prev].elapsed_time(ev[k])
            prev = k
    per = {k: v / steps for k, v in acc.items()}
    per_first = {k: v / steps for k, v in acc_first.items()}
    total = lat / steps
    gemm_flops = 0
    for M in (L_TOK, T_COND):
        gemm_flops += 2 * M * (E * 3 * E + E * E + E * FFN + FFN * E)
    return {"attention_backend": attention_backend,
            "workload": f"cfg4 block: video {L_TOK} + condition {T_COND} tokens, hidden {E}, "
                        f"{HEADS}x{HEAD_DIM} heads, FFN {FFN}, {n_cached} cached chunks of {L_TOK} tokens "
                        f"(ring write of the chunk every call; cached rows of the joint K / V reused "
                        f"across calls as across denoising steps, or assembled in the call: *_first_step)",
            "block_latency_ms": total, "attention_ms": per["attention"],
            "kernel_ms_excl_attention": total - per["attention"], "stages_ms": per,
            "stages_sum_ms": sum(per.values()),
            "block_latency_first_step_ms": lat_first / steps, "stages_first_step_ms": per_first,
            "gemm_stage_tflops": gemm_flops / ((per["qkv"] + per["proj_ffn"]) / 1e3) / 1e12,
            "attention_kv_tokens": n_cached * L_TOK + L_TOK + T_COND}


def bench_attention(steps, warmup):
    """The block's joint attention core (dit.py:154-167): video 10800 + condition 512
    queries over 2 cached chunks + video + condition = 32912 keys, 40 heads x 128, bf16. This
    build's kernel (joy_attention_fwd, reading the token-major joint operands in place) vs the
    reference's own call, F.scaled_dot_product_attention on the transposed views (ROCm backend of
    this torch), on the same inputs; each step one launch, timed with HIP events on the stream."""
    import torch
    import joyomni_ops as jo
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(6)
    Lq, Lk = L_TOK + 512, 3 * L_TOK + 512
    q = torch.randn(1, Lq, HEADS, HEAD_DIM, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(1, Lk, HEADS, HEAD_DIM, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(1, Lk, HEADS, HEAD_DIM, generator=g).to(torch.bfloat16).to(dev)
    out = torch.empty_like(q)
    steps_a, warm_a = max(2, min(steps, 10)), max(1, min(warmup, 3))
    t = time_launches(lambda: jo.sdpa_attention_out(q, k, v, out), steps_a, warm_a)
    tr = time_launches(lambda: torch.nn.functional.scaled_dot_product_attention(
        q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), is_causal=False), steps_a, warm_a)
    flops = 4 * Lq * Lk * HEAD_DIM * HEADS
    return {"workload": f"joint attention: {Lq} queries x {Lk} keys x {HEADS} heads x {HEAD_DIM}, bf16, "
                        "non-causal, no mask", "ms": t * 1e3, "tflops": flops / t / 1e12,
            "frac_bf16_peak": flops / t / 1e12 / PEAK_BF16_TFLOPS,
            "reference_sdpa_ms": tr * 1e3, "reference_sdpa_tflops": flops / tr / 1e12,
            "speedup_vs_reference_gpu": tr / t, "steps": steps_a}


def bench_copy(steps, warmup):
    """Plain 1 GiB device-to-device copy: the calibration kernel for the
    FETCH_SIZE / WRITE_SIZE counters (known 1 GiB read + 1 GiB write)."""
    import torch
    dev = torch.device("cuda:0")
    src = torch.empty(1 << 29, dtype=torch.bfloat16, device=dev).fill_(1)
    dst = torch.empty_like(src)
    t = time_launches(lambda: dst.copy_(src), steps, warmup)
    return {"bytes": 2 * src.numel() * 2, "us": t * 1e6, "gbs": 2 * src.numel() * 2 / t / 1e9}


def cpu_baseline_qkv():
    """Reference CPU torch path (oracle/torch_path.py) on a bounded token sample."""
    import torch
    from oracle import torch_path
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    Ls = L_TOK  # the whole chunk
    g = torch.Generator().manual_seed(0)
    qkv = torch.randn(Ls, 3 * E, generator=g).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(HEAD_DIM, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(HEAD_DIM, generator=g)).to(torch.bfloat16)
    ang = torch.rand(Ls, HEAD_DIM // 2, generator=g)
    cos, sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    ck = torch.empty(RING_SLOTS, Ls, HEADS, HEAD_DIM, dtype=torch.bfloat16)
    cv = torch.empty_like(ck)
    torch_path.qkv_norm_rope_cache(qkv, HEADS, 1e-6, qw, kw, cos, sin, ck, cv, SLOT)  # warm-up
    times = []
    t_end = time.perf_counter() + 20.0
    while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 15):
        t0 = time.perf_counter()
        torch_path.qkv_norm_rope_cache(qkv, HEADS, 1e-6, qw, kw, cos, sin, ck, cv, SLOT)
        times.append(time.perf_counter() - t0)
    times.sort()
    t = times[len(times) // 2]
    return {"value": qkv_bytes(Ls) / t / 1e9, "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"full chunk {Ls} tokens x 40 heads x 128, median of {len(times)} runs, "
                      f"torch CPU restatement of sgl_fused_ops.py:170-199 + cache copy"}


def cpu_baselines_more():
    """Host-core timings (torch CPU restatements, oracle/torch_path.py) of the other hot-path kernels
    on bounded samples of their bench workloads, reported beside the GPU figures."""
    import torch
    import torch.nn.functional as F
    from oracle import torch_path
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(5)

    def median_time(fn, reps=5):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[len(ts) // 2]

    out = {}
    M, K = L_TOK, E
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    t = median_time(lambda: torch_path.quantize_per_token_rounding(x, True))
    out["act_quant"] = {"value": quant_bytes(M, K) / t / 1e9, "unit": "GB/s", "cores": cores, "kind": "port",
                        "us": t * 1e6, "sample": f"full M {M} x K {K}, division (fp8_linear.py:38-43), median of 5"}
    sc = (0.2 * torch.randn(1, K, generator=g)).to(torch.bfloat16)
    sh = (0.2 * torch.randn(1, K, generator=g)).to(torch.bfloat16)
    t = median_time(lambda: torch_path._layernorm_modulate_ref(x, sh, sc, 1e-6))
    b = 2 * M * K + 2 * M * K + 2 * 2 * K
    out["adaln_norm"] = {"value": b / t / 1e9, "unit": "GB/s", "cores": cores, "kind": "port", "us": t * 1e6,
                         "sample": f"full M {M} x N {K}, fp32 layer_norm * (1 + scale) + shift -> bf16, median of 5"}
    del x
    Lq, Lk = 1024, 3 * L_TOK + 512  # one head's 1024 queries over the whole joint key sequence
    q = torch.randn(1, 1, Lq, HEAD_DIM, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 1, Lk, HEAD_DIM, generator=g).to(torch.bfloat16)
    v = torch.randn(1, 1, Lk, HEAD_DIM, generator=g).to(torch.bfloat16)
    t = median_time(lambda: F.scaled_dot_product_attention(q.float(), k.float(), v.float()), reps=3)
    out["attention"] = {"value": 4 * Lq * Lk * HEAD_DIM / t / 1e12, "unit": "TFLOP/s", "cores": cores,
                        "kind": "port", "us": t * 1e6,
                        "sample": f"1 head, {Lq} queries x {Lk} keys x {HEAD_DIM} (fp32 F.scaled_dot_product_attention "
                                  f"on the bf16 inputs, dit.py:154-167), median of 3"}
    return out


def cpu_baseline_gemm():
    import torch
    from oracle import torch_path
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    Ms, K, N = 256, 4096, 4096  # benchmark cfg 0
    g = torch.Generator().manual_seed(0)
    x = torch.randn(Ms, K, generator=g)
    x[:, torch.randperm(K, generator=g)[: K // 200]] *= 20
    x = x.to(torch.bfloat16)
    wq, ws = torch_path.quantize_per_token((torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16))
    bias = (torch.randn(N, generator=g) * 0.01).to(torch.bfloat16)
    torch_path.fp8_linear(x, wq, ws, bias)
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        torch_path.fp8_linear(x, wq, ws, bias)
        times.append(time.perf_counter() - t0)
    t = sorted(times)[2]
    return {"value": 2 * Ms * N * K / t / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "us": t * 1e6,
            "sample": f"cfg0 single FP8 linear {Ms}x{K} -> {N}, median of 5: per-token quant (division) + "
                      "fp32 dequantise-then-matmul + bias -> bf16"}


def summary(rec):
    """Compact digest of the line's sections (rounded figures), printed as its last key."""
    r = lambda v, n=1: None if v is None else round(v, n)  # noqa: E731
    out = {}
    if "roofline" in rec:
        out["cfg1_qkv_norm_rope"] = {"us": r(rec["ms_per_step"] * 1e3), "gbs": rec["value"],
                                     "frac_hbm": rec["roofline"]["frac"]}
    if "gemm_cfg2" in rec:
        gc = rec["gemm_cfg2"]
        out["cfg2_gemm"] = {"tflops": gc["aggregate_tflops"], "frac_fp8": gc["roofline"]["frac"],
                            "hipblaslt": gc["reference_hipblaslt_aggregate_tflops"],
                            "hipblaslt_tuned": gc["reference_hipblaslt_tuned_aggregate_tflops"],
                            "shapes_us_tflops_hipblaslt_tuned": {
                                x["shape"]: [r(x["ms"] * 1e3), r(x["tflops"], 0), r(x.get("reference_hipblaslt_tflops"), 0),
                                             r(x.get("reference_hipblaslt_tuned_tflops"), 0)] for x in gc["shapes"]}}
    if "gemm_reference_shapes" in rec:
        gr = rec["gemm_reference_shapes"]
        out["refgemm_12"] = {"us": r(gr["total_us"], 0), "hipblaslt_us": r(gr["reference_hipblaslt_total_us"], 0),
                             "hipblaslt_tuned_us": r(gr["reference_hipblaslt_tuned_total_us"], 0),
                             "speedup_tuned_per_shape": [r(x["speedup_vs_reference_gpu_tuned"], 3) for x in gr["shapes"]]}
    if "gemm_cfg3_small_m" in rec:
        out["cfg3_M_N_us_bound_frac_hipblaslt_us"] = [
            [x["M"], x["N"], r(x["us"]), x["roofline_bound"], r(x["frac_roofline"], 3), r(x["reference_hipblaslt_us"])]
            for x in rec["gemm_cfg3_small_m"]]
    if "qkv_projection" in rec:
        qp = rec["qkv_projection"]
        out["qkv_projection_us"] = {"fused": r(qp["fused_us"], 0), "two_op": r(qp["two_op_us"], 0),
                                    "gemm_only": r(qp["gemm_only_us"], 0)}
    if "cfg0_linear" in rec:
        out["cfg0_linear_us"] = r(rec["cfg0_linear"]["us"])
    if "act_quant" in rec:
        out["act_quant_frac_hbm"] = [r(x["frac_hbm_peak"], 3) for x in rec["act_quant"]]
    if "adaln_norm" in rec:
        out["adaln_norm_frac_hbm"] = [r(x["frac_hbm_peak"], 3) for x in rec["adaln_norm"]]
    if "kv_pack" in rec:
        out["kv_pack_frac_hbm"] = [r(x["frac_hbm_peak"], 3) for x in rec["kv_pack"]]
    if "attention_core" in rec:
        a = rec["attention_core"]
        out["attention"] = {"ms": r(a["ms"], 2), "frac_bf16": r(a["frac_bf16_peak"], 3),
                            "torch_sdpa_ms": r(a["reference_sdpa_ms"], 2)}
    if "block_cfg4" in rec:
        b = rec["block_cfg4"]
        out["block_cfg4_ms"] = {"hip_attention": r(b["block_latency_ms"], 2),
                                "hip_attention_first_step": r(b["block_latency_first_step_ms"], 2),
                                "attention": r(b["attention_ms"], 2)}
        if "block_cfg4_torch_sdpa" in rec:
            bs = rec["block_cfg4_torch_sdpa"]
            out["block_cfg4_ms"].update({"torch_sdpa_attention": r(bs["block_latency_ms"], 2),
                                         "torch_sdpa_attention_part": r(bs["attention_ms"], 2)})
    if "cpu_baseline" in rec:
        out["cpu_baseline_gbs"] = r(rec["cpu_baseline"]["value"], 2)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--eager", action="store_true", help="time plain launches (no HIP graph)")
    ap.add_argument("--only", default="all",
                    choices=["all", "qkv", "qkvproj", "gemm", "cfg0", "refgemm", "small", "quant", "pack", "norm", "attn", "block",
                             "copy", "clock"])
    ap.add_argument("--tunableop", metavar="CSV", default=None,
                    help="tune the reference's torch._scaled_mm legs with PyTorch TunableOp first, with the "
                         "reference's settings (deploy/tune_rocm_fp8.py: 10 ms, 30 iterations), results to CSV")
    args = ap.parse_args()
    global EAGER
    EAGER = args.eager
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the hot path has no multi-GPU component in this tier.", file=sys.stderr)
        sys.exit(2)

    import torch
    import joyomni_ops  # noqa: F401  (fails loudly if the HIP library is missing)
    TunedReference.configure(args.tunableop)
    props = torch.cuda.get_device_properties(0)
    rec = {"metric": METRIC, "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
           "data": "synthetic (seeded N(0,1) qkv, N(1,0.1) norm weights, real 3-D RoPE tables)",
           "config": {"workload": "cfg1: fused QKV split + q/k RMSNorm + 3-D RoPE (44/42/42, theta 1e4) "
                                  "+ KV-ring write (4 slots), outputs q_rope, k_rope, k_pre->cache, v->cache",
                      "seq_len": L_TOK, "heads": HEADS, "head_dim": HEAD_DIM, "grid_thw": [3, 45, 80],
                      "parallelism": "single GPU"},
           "device": {"name": props.name, "arch": getattr(props, "gcnArchName", "?"),
                      "cus": props.multi_processor_count}}
    if args.only in ("all", "qkv"):
        t, b = bench_qkv(args.steps, args.warmup)
        gbs = b / t / 1e9
        rec.update({"value": round(gbs, 1), "ms_per_step": t * 1e3})
        rec["roofline"] = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                           "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": load_traffic("qkv_norm_rope"),
                           "algorithmic_bytes": b, "kernel": "qk_norm_rope_kernel<128>"}
        progress(f"cfg1 qkv norm/rope {t * 1e6:.1f} us, {gbs:.0f} GB/s")
    if args.only in ("all", "gemm"):
        # all `steps` calls in one graph: a graph replay carries a fixed start-up cost, which a
        # short graph spreads over few calls (and an op of two launches pays about twice)
        res, agg, ref_agg, tuned_agg = bench_gemm(args.steps, max(2, args.warmup // 2))
        best = max(res, key=lambda r: r["tflops"])
        rec["gemm_cfg2"] = {"shapes": res, "aggregate_tflops": round(agg, 1),
                            "reference_hipblaslt_aggregate_tflops": round(ref_agg, 1) if ref_agg else None,
                            "reference_hipblaslt_tuned_aggregate_tflops": round(tuned_agg, 1) if tuned_agg else None,
                            "activations": "cfg 0 distribution: N(0,1) with 0.5 % of channels x20",
                            "roofline": {"bound": "mfma", "achieved": round(agg, 1), "peak": PEAK_FP8_TFLOPS,
                                         "unit": "TFLOP/s", "frac": round(agg / PEAK_FP8_TFLOPS, 4),
                                         "traffic": load_traffic("fp8_gemm_qkv"),
                                         "best_shape": best["shape"]}}
        progress(f"cfg2 GEMMs {agg:.0f} TFLOP/s aggregate")
        if "value" not in rec:
            rec.update({"value": round(agg, 1), "unit": "TFLOP/s", "ms_per_step": sum(r["ms"] for r in res)})
    if args.only in ("all", "qkvproj"):
        rec["qkv_projection"] = bench_qkv_projection(args.steps, args.warmup)
        qp = rec["qkv_projection"]
        progress(f"QKV projection + norm/RoPE/ring: fused {qp['fused_us']:.0f} us, two ops {qp['two_op_us']:.0f} us "
                 f"(GEMM alone {qp['gemm_only_us']:.0f} us)")
    if args.only in ("all", "cfg0"):
        rec["cfg0_linear"] = bench_cfg0(args.steps, args.warmup)
        progress(f"cfg0 linear {rec['cfg0_linear']['us']:.1f} us")
    if args.only in ("all", "refgemm"):
        rs = bench_reference_shapes(args.steps, max(2, args.warmup // 2))
        t_ours = sum(r["us"] for r in rs)
        t_ref = sum(r["reference_hipblaslt_us"] for r in rs)
        t_tuned = sum(r["reference_hipblaslt_tuned_us"] for r in rs)
        rec["gemm_reference_shapes"] = {"shapes": rs, "total_us": t_ours, "reference_hipblaslt_total_us": t_ref,
                                        "speedup_vs_reference_gpu": t_ref / t_ours,
                                        "reference_hipblaslt_tuned_total_us": t_tuned,
                                        "speedup_vs_reference_gpu_tuned": t_tuned / t_ours}
        progress(f"reference tuned GEMM shapes: {t_ours:.0f} us vs hipBLASLt {t_ref:.0f} us untuned, "
                 f"{t_tuned:.0f} us TunableOp-tuned")
    if args.only in ("all", "small"):
        rec["gemm_cfg3_small_m"] = bench_small_m(args.steps, args.warmup)
        progress("cfg3 small-M GEMMs done")
    if args.only in ("all", "quant"):
        rec["act_quant"] = bench_quant(args.steps, args.warmup)
        progress("act quant done")
    if args.only in ("all", "pack"):
        rec["kv_pack"] = bench_pack(args.steps, args.warmup)
        progress("cache read-side packs done")
    if args.only in ("all", "norm"):
        rec["adaln_norm"] = bench_norm(args.steps, args.warmup)
        progress("adaLN norm done")
    if args.only in ("all", "attn"):
        rec["attention_core"] = bench_attention(args.steps, args.warmup)
        progress(f"attention {rec['attention_core']['ms']:.2f} ms "
                 f"(torch SDPA {rec['attention_core']['reference_sdpa_ms']:.2f} ms)")
    if args.only in ("all", "block"):
        rec["block_cfg4"] = bench_block(max(3, args.steps // 10), max(1, args.warmup // 5))
        progress(f"cfg4 block {rec['block_cfg4']['block_latency_ms']:.2f} ms "
                 f"(first step on a chunk's cache {rec['block_cfg4']['block_latency_first_step_ms']:.2f} ms)")
        # BASELINE cfg 4 as stated: the attention core is the reference's F.scaled_dot_product_attention
        # (dit.py:154-167), inside the block latency
        rec["block_cfg4_torch_sdpa"] = bench_block(max(3, args.steps // 10), max(1, args.warmup // 5),
                                                   attention_backend="torch_sdpa")
        progress(f"cfg4 block with torch SDPA attention {rec['block_cfg4_torch_sdpa']['block_latency_ms']:.2f} ms "
                 f"(attention {rec['block_cfg4_torch_sdpa']['attention_ms']:.2f} ms)")
    if args.only == "copy":
        rec["copy"] = bench_copy(args.steps, args.warmup)
    if args.only == "clock":
        rec["clock"] = bench_clock(max(args.steps, 13), max(args.warmup, 1))
    from torch.cuda import tunable
    rec["tunableop"] = {"file": args.tunableop, "tuned_results": len(tunable.get_results()),
                        "settings": "reference deploy/tune_rocm_fp8.py: 10 ms, 30 iterations"}
    if not args.no_cpu:
        if args.only in ("all", "qkv"):
            rec["cpu_baseline"] = cpu_baseline_qkv()
        if args.only in ("all", "gemm", "cfg0"):
            rec["cpu_baseline_gemm"] = cpu_baseline_gemm()
        if args.only == "all":
            rec["cpu_baselines_more"] = cpu_baselines_more()
    rec["summary"] = summary(rec)  # last key: the part of the line a tail of it keeps
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
