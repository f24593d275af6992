"""The library's host code — the GGUF index reader (gguf.cpp) and the device
layout (layout.cpp) — built with g++ under AddressSanitizer and UBSan with a
driver (tests/support/host_sanitize.cpp) that reads every fixture file whole,
every prefix of the small ones and 20,000 seeded mutations of each, and lays
out blocks of every format; any report fails. Host only: no GPU call.
"""

import glob
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "charlotte_amd", "csrc")


def test_host_code_is_clean_under_asan_and_ubsan(tmp_path):
    if shutil.which("g++") is None or not os.path.isdir("/opt/rocm/include"):
        pytest.skip("no host compiler or HIP headers")
    exe = str(tmp_path / "host_sanitize")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
           "-D__HIP_PLATFORM_AMD__", "-I", CSRC, "-I", os.path.join(ROOT, "include"), "-I", "/opt/rocm/include",
           os.path.join(ROOT, "tests", "support", "host_sanitize.cpp"), os.path.join(CSRC, "gguf.cpp"),
           os.path.join(CSRC, "layout.cpp"), "-o", exe, "-lpthread"]
    build = subprocess.run(cmd, capture_output=True, text=True)
    assert build.returncode == 0, build.stderr[-3000:]
    files = sorted(glob.glob(os.path.join(ROOT, "tests", "golden", "gguf", "*.gguf")))
    files.append(os.path.join(ROOT, "tests", "golden", "matmul_rows.gguf"))
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1")
    r = subprocess.run([exe, *files], capture_output=True, text=True, env=env, timeout=900)
    assert r.returncode == 0 and "host ok" in r.stdout, (r.stdout[-1000:], r.stderr[-4000:])
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-4000:]
