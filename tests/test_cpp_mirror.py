"""Runs the C++ mirror's test binary (tests/cpp/test_kernel_backend.cpp):
the `cpu` suite here, the `gpu` suite on an MI355X.  The binary is built by
__graft_entry__.build() (make -C tests/cpp); a missing binary is a failure."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "_build", "test_kernel_backend")


def _run(suite: str) -> None:
    assert os.path.exists(BIN), f"{BIN} is not built: run __graft_entry__.build() (make -C tests/cpp)"
    r = subprocess.run([BIN, suite], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, f"C++ {suite} suite failed:\n{r.stdout}\n{r.stderr}"


def test_cpp_mirror_cpu_suite():
    _run("cpu")


@pytest.mark.gpu
def test_cpp_mirror_gpu_suite():
    _run("gpu")
