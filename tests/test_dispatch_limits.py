"""The launch-size check every kernel launch goes through (dispatch_fits /
grid_for in csrc/rows.hpp), on the host: at most 2^31 - 1 workgroups per
grid dimension and fewer than 2^32 work-items, the 32-bit grid size of the
dispatch packet (tests/cpp/test_dispatch.cpp)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_dispatch_limits(tmp_path):
    exe = tmp_path / "test_dispatch"
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Werror", "-o", str(exe),
                    os.path.join(HERE, "cpp", "test_dispatch.cpp")], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert " 0 failures" in r.stdout
