"""The host layout / plan code of libsgl_rocm_kv under AddressSanitizer and
UndefinedBehaviorSanitizer: tests/native/layout_fuzz.cpp replays reference
goldens and fuzzes every group-1 entry point (small, boundary and
overflowing values), the page allocator under random traffic and the
checksum; tests/native/bootstrap_fuzz.cpp round-trips and mutates bootstrap
frames through the wire-format decoder. Any out-of-bounds access, overflow
UB or violated invariant fails the run. Host code only (g++, no device
code)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "sglang-rs_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_layout_fuzz_under_asan_ubsan(tmp_path):
    exe = tmp_path / "layout_fuzz"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", "-I" + os.path.join(ROOT, "include"),
           "-I" + CSRC, os.path.join(ROOT, "tests", "native", "layout_fuzz.cpp"),
           os.path.join(CSRC, "kv_layout.cpp"), os.path.join(CSRC, "kv_plan.cpp"), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=240)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=240, env=env)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "layout fuzz ok" in r.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_bootstrap_fuzz_under_asan_ubsan(tmp_path):
    exe = tmp_path / "bootstrap_fuzz"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", "-I" + os.path.join(ROOT, "include"),
           "-I" + CSRC, os.path.join(ROOT, "tests", "native", "bootstrap_fuzz.cpp"),
           os.path.join(CSRC, "kv_bootstrap.cpp"), os.path.join(CSRC, "kv_layout.cpp"),
           os.path.join(CSRC, "kv_plan.cpp"), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=240)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=240, env=env)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "bootstrap fuzz ok" in r.stdout
