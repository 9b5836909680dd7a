"""Runs the C++ host layer's test binaries: tests/cpp/test_kernel_backend.cpp
(the mirror of the kernel boundary) and tests/cpp/test_gguf.cpp (the GGUF
loader); the `cpu` suites here, the `gpu` suites on an MI355X.  The binaries
are built by __graft_entry__.build() (make -C tests/cpp); a missing binary is
a failure."""
import os
import subprocess

import pytest

BUILD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "_build")


def _run(binary: str, suite: str) -> None:
    path = os.path.join(BUILD, binary)
    assert os.path.exists(path), f"{path} is not built: run __graft_entry__.build() (make -C tests/cpp)"
    r = subprocess.run([path, suite], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, f"C++ {binary} {suite} suite failed:\n{r.stdout}\n{r.stderr}"


def test_cpp_mirror_cpu_suite():
    _run("test_kernel_backend", "cpu")


def test_gguf_loader_cpu_suite():
    _run("test_gguf", "cpu")


@pytest.mark.gpu
def test_cpp_mirror_gpu_suite():
    _run("test_kernel_backend", "gpu")


@pytest.mark.gpu
def test_gguf_loader_gpu_suite():
    _run("test_gguf", "gpu")
