"""The RoPE kernels' division by a launch-constant divisor (fastdiv.hpp,
Granlund and Montgomery's multiply-high form) against the hardware division,
on the host: every divisor up to 2^16, 200000 random ones and the powers of
two and their neighbours, each on the dividends that expose a wrong
multiplier or shift (tests/cpp/test_fastdiv.cpp)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_fastdiv_matches_division(tmp_path):
    exe = tmp_path / "test_fastdiv"
    subprocess.run(["g++", "-O2", "-std=c++17", "-o", str(exe), os.path.join(HERE, "cpp", "test_fastdiv.cpp")],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert " 0 failures" in r.stdout
