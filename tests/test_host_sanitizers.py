"""The host twins' index arithmetic under AddressSanitizer and
UndefinedBehaviorSanitizer (CPU): csrc/host.cpp and a driver
(tests/native/host_sanitize.cpp) are built with -fsanitize=address,undefined
and run over every mask kind, GQA, ragged and single-row shapes, document
labels and block tables with out-of-range entries and over-long counts."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_host_twins_under_asan_ubsan(tmp_path):
    exe = tmp_path / "host_sanitize"
    cmd = ["g++", "-O1", "-g", "-std=c++17", "-pthread", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "native", "host_sanitize.cpp"),
           os.path.join(ROOT, "pallas-flexattn_amd", "csrc", "host.cpp"), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    res = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr[-4000:]
    assert res.stdout.strip() == "ok 6", res.stdout
