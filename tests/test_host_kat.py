"""Host-logic known-answer tests (C++, no GPU): builds tests/cpp/test_host.cpp
against libeinsum_ir.so and runs it."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "einsum_ir_amd")


def test_host_known_answers(tmp_path):
    exe = str(tmp_path / "test_host")
    subprocess.check_call(["g++", "-O1", "-std=c++17", "-Wall",
                           "-I" + os.path.join(PKG, "csrc", "host"), "-I" + os.path.join(ROOT, "include"),
                           os.path.join(ROOT, "tests", "cpp", "test_host.cpp"), "-o", exe,
                           "-L" + PKG, "-leinsum_ir", "-Wl,-rpath," + PKG])
    res = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "0 failures" in res.stdout
