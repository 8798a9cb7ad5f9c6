"""The tile GEMM's per-stream workspace rules (csrc/g4_workspace.h), on the CPU: a C++ driver with
fake allocator, drain and capture-query calls checks that growth inside a capture is refused, that
a buffer a capture saw is retired instead of freed, that other buffers are freed only after their
stream drains, and that a destroyed stream's handle starts without a buffer."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "gemma4-webgpu-engine_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_workspace_lifetime_rules(tmp_path):
    exe = tmp_path / "ws_check"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-I", CSRC,
                    os.path.join(HERE, "workspace_policy_check.cc"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.strip() == "ok", out.stdout + out.stderr
