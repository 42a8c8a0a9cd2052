"""bench.py's contract on the CPU: more than one GPU is refused with a message and exit status 2
before anything touches a device, and the committed per-launch HBM traffic that the JSON line
reports for the headline kernel and the cfg-2 GEMM loads."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2, (r.returncode, r.stderr[-400:])
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""  # no JSON line


def test_committed_traffic_loads():
    sys.path.insert(0, ROOT)
    import bench
    with open(os.path.join(ROOT, "profiles", "hbm_traffic.json")) as f:
        d = json.load(f)
    for name in ("qkv_norm_rope", "fp8_gemm_qkv"):
        b = bench.load_traffic(name)
        assert isinstance(b, int) and b >= d[name]["algorithmic_bytes"] * 0.99, (name, b)
    # the headline kernel's traffic stays within 1 % of its algorithmic bytes
    assert d["qkv_norm_rope"]["ratio_to_algorithmic"] < 1.01
    assert bench.load_traffic("no_such_kernel") is None
