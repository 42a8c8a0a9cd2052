"""The C-ABI tests (tests/test_capi.py: argument checks, exports, workspace sizing) run against a
build of the library whose host code carries AddressSanitizer and UndefinedBehaviorSanitizer
(``make -C joyai-video-edit_amd/csrc sanitize``), in a child process with the ASan runtime
preloaded. Any sanitizer report aborts the child and fails this test. No kernel is launched."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "joyai-video-edit_amd", "csrc")
SAN_LIB = os.path.join(CSRC, "_build", "san", "libjoyomni_hip_san.so")
HIPCC = "/opt/rocm/bin/hipcc"


def test_capi_under_address_and_ub_sanitizers():
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    jobs = str(min(16, os.cpu_count() or 4))
    subprocess.run(["make", "-j", jobs, "-C", CSRC, "sanitize"], check=True, capture_output=True)
    asan_rt = subprocess.run([HIPCC, "-print-file-name=libclang_rt.asan-x86_64.so"], check=True,
                             capture_output=True, text=True).stdout.strip()
    assert os.path.exists(asan_rt), asan_rt
    env = dict(os.environ, JOY_HIP_LIB=SAN_LIB, LD_PRELOAD=asan_rt,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([sys.executable, "-m", "pytest", os.path.join(ROOT, "tests", "test_capi.py"), "-q",
                        "-p", "no:cacheprovider", "-m", "not gpu"],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert " passed" in out
