"""Build libokq.so (the gfx950 k-quant linear path) in-tree with hipcc.

``python -m ocelotl_amd.build`` compiles every ``csrc/*.hip`` for gfx950 and
links ``ocelotl_amd/libokq.so``.  The library is loaded by
``ocelotl_amd.okq`` and travels with the source tree; no JIT cache is used.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libokq.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed-FP32 VALU ops (v_pk_*_f32) are disabled on purpose: some of their
# forms have given wrong results on these GPUs without any error.
COMMON = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(HERE, "..", "include"),
]
# Per-file extra flags.  okq_prep.hip holds the bit-exact dequant/quantize
# kernels, okq_gemv.hip writes its FMAs out so that every instantiation rounds
# alike: no FMA contraction in either.
EXTRA = {"okq_prep.hip": ["-ffp-contract=off"], "okq_gemv.hip": ["-ffp-contract=off"],
         # MFMA accumulators in VGPRs where they fit: the per-super-block sums
         # then feed the f32 scaling without AGPR round trips
         "okq_gemm_wide.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
         "okq_gemm_pair.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
         "okq_gemm_q8.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
         "okq_gemm_q6.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def sources():
    return sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, src.replace(".hip", ".o"))
    cmd = [HIPCC, *COMMON, *EXTRA.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


HOST_SRC = [os.path.join(HERE, "host", f)
            for f in ("kernel_backend.cpp", "gguf.cpp", "dequant_policy.cpp", "dequant_host.cpp")]
HOST_LIB = os.path.join(HERE, "libocelotl_hip.so")
CXX = os.environ.get("CXX", "g++")


def build_host(verbose: bool = False) -> str:
    """The C++ host layer (host/kernel_backend.*: the mirror of the kernel
    boundary; host/gguf.*: the GGUF loader), a plain C++17 library over okq.h
    linked against libokq.so."""
    tmp = HOST_LIB + ".tmp"
    # no FMA contraction: the host decoders round every product on its own
    cmd = [CXX, "-std=c++17", "-O2", "-ffp-contract=off", "-Wall", "-Wextra", "-fPIC", "-shared",
           "-I", os.path.join(HERE, "..", "include"),
           "-I", os.path.join(HERE, "host"), *HOST_SRC, "-o", tmp, "-L", HERE, "-lokq", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"host library build failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, HOST_LIB)
    if verbose:
        print(f"built {HOST_LIB}")
    return HOST_LIB


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    build_host(verbose)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
