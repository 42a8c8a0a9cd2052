"""Resource properties of the generated gfx950 code that the kernels' performance relies on,
read from the compiler's own kernel metadata (device code compiled with the Makefile's flags,
no GPU needed):

* no kernel of the hot path touches scratch memory (register spills): the attention core, the
  fused QKV norm/RoPE/ring kernel, the packs, the adaLN norms, the quantisers and the GEMM
  kernels. Two persistent GEMM kernels keep a few spills outside their K loops (the fused QKV
  epilogue 12 bytes, the gated-residual epilogue with bf16 output 20 bytes); the general
  fallback kernel fp8_gemm_4w, which the model's shapes do not use, 20 bytes;
* the attention core fits two waves per SIMD (its 512-thread workgroups, one per CU: at most 256
  VGPRs per lane in all) with its two double-buffered K / V tiles in LDS (128 KiB).
"""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "joyai-video-edit_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# the device-side flags of csrc/Makefile (HIPFLAGS without the host-only ones)
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "--cuda-device-only", "-S"]
SOURCES = ["attention", "qkv_norm_rope", "kv_pack", "norm_modulate", "quant_fp8", "fp8_gemm"]


def kernel_metadata(asm):
    """{kernel name: {private_segment_fixed_size, vgpr_spill_count, vgpr_count, agpr_count,
    group_segment_fixed_size}} from the amdhsa.kernels metadata of one assembly file."""
    meta = asm[asm.index("amdhsa.kernels:"):]
    out = {}
    for block in re.split(r"\n  - ", meta):
        m = re.search(r"\.name:\s+(\S+)", block)
        if not m:
            continue
        fields = {}
        for key in ("private_segment_fixed_size", "vgpr_spill_count", "vgpr_count", "agpr_count",
                    "group_segment_fixed_size"):
            f = re.search(r"\." + key + r":\s+(\d+)", block)
            fields[key] = int(f.group(1)) if f else 0
        out[m.group(1)] = fields
    return out


@pytest.fixture(scope="module")
def kernels():
    if not os.path.exists(HIPCC) and shutil.which("hipcc") is None:
        pytest.skip("hipcc not available")
    hipcc = HIPCC if os.path.exists(HIPCC) else shutil.which("hipcc")
    with tempfile.TemporaryDirectory() as tmp:
        procs = {}
        for src in SOURCES:
            out = os.path.join(tmp, src + ".s")
            procs[src] = (subprocess.Popen([hipcc, *FLAGS, "-o", out, os.path.join(CSRC, src + ".hip")],
                                           stdout=subprocess.PIPE, stderr=subprocess.PIPE), out)
        result = {}
        for src, (p, out) in procs.items():
            _, err = p.communicate(timeout=600)
            assert p.returncode == 0, f"{src}.hip: {err.decode()[-2000:]}"
            result[src] = kernel_metadata(open(out).read())
    return result


# scratch bytes allowed per kernel (mangled-name substring), everything else: none
ALLOWED_SCRATCH = {
    "fp8_gemm_4qILb1ELi4ELi256E": 12,   # fused QKV epilogue, spills outside the K loop
    "fp8_gemm_4qILb1ELi2ELi256E": 20,   # gated residual, bf16 output, spills outside the K loop
    "fp8_gemm_4w": 20,                  # general fallback (shapes the model does not use)
}


def test_every_source_compiles_its_kernels(kernels):
    for src in SOURCES:
        assert kernels[src], f"{src}.hip: no kernels in the generated code"
    assert any("attn_fwd_d128" in k for k in kernels["attention"])
    assert any("fp8_gemm_4q" in k for k in kernels["fp8_gemm"])


def test_no_scratch_in_hot_kernels(kernels):
    bad = []
    for src, ks in kernels.items():
        for name, f in ks.items():
            limit = next((v for key, v in ALLOWED_SCRATCH.items() if key in name), 0)
            if f["private_segment_fixed_size"] > limit:
                bad.append(f"{src}: {name} uses {f['private_segment_fixed_size']} bytes of scratch "
                           f"({f['vgpr_spill_count']} VGPR spills), allowed {limit}")
    assert not bad, "\n".join(bad)


def test_attention_occupancy_and_lds(kernels):
    (name, f), = [(k, v) for k, v in kernels["attention"].items() if "attn_fwd_d128" in k]
    assert f["vgpr_count"] <= 256, f"{name}: {f['vgpr_count']} VGPRs per lane, two waves per SIMD need <= 256"
    assert f["group_segment_fixed_size"] == 2 * 2 * 2 * 64 * 256, "K / V tiles: 2 buffers x 2 head slots x K, V"
