"""The workspace bookkeeping (per-stream buffers, graph-pinned retirement,
no growth under capture) checked on the CPU: tests/cpp/test_workspace_pool.cpp
drives ml_framework_amd/csrc/workspace_pool.h with a fake backend."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_workspace_pool_rules(tmp_path):
    exe = tmp_path / "test_workspace_pool"
    src = os.path.join(ROOT, "tests", "cpp", "test_workspace_pool.cpp")
    inc = os.path.join(ROOT, "ml_framework_amd", "csrc")
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-fsanitize=address,undefined",
                    f"-I{inc}", src, "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stderr
    assert "all checks passed" in out.stdout
