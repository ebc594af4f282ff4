"""CPU tests of the C++ harnesses' float64 host evaluation
(einsum_ir_amd/csrc/bench/bench_util.h): builds tests/cpp/test_bench_util.cpp
with g++ and runs it (no GPU call; libeinsum_ir_hip.so is linked for the
device-buffer helpers the header declares but the test does not call)."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "einsum_ir_amd")


def test_bench_util_host_evaluation(tmp_path):
    exe = str(tmp_path / "test_bench_util")
    subprocess.check_call(["g++", "-O1", "-std=c++17", "-Wall", "-I" + os.path.join(ROOT, "include"),
                           os.path.join(ROOT, "tests", "cpp", "test_bench_util.cpp"), "-o", exe,
                           "-L" + PKG, "-leinsum_ir_hip", "-Wl,-rpath," + PKG])
    res = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "0 failures" in res.stdout


def test_harness_programs_are_built():
    for name in ("bench_binary", "bench_unary", "bench_expression", "bench_tree"):
        path = os.path.join(PKG, "bin", name)
        assert os.access(path, os.X_OK), path
        # no arguments: the usage text and a failure status, before any GPU call
        res = subprocess.run([path], capture_output=True, text=True, timeout=60)
        assert res.returncode != 0 and "usage" in res.stderr
