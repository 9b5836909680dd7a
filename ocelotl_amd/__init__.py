"""ocelotl_amd -- MI355X (gfx950) k-quant linear path for Ocelotl.

Q8_0 / Q4_K / Q5_K / Q6_K GGUF weights, dequantized and contracted against
activations by hand-written HIP kernels in ``libokq.so`` (C-ABI:
``include/okq.h``).  ``ocelotl_amd.okq`` is the ctypes binding,
``ocelotl_amd.backend`` the Python mirror of the reference's KernelBackend
linear surface, ``ocelotl_amd.build`` the in-tree hipcc build.  The C++ host
layer (``host/``: the KernelBackend mirror and the GGUF tensor-payload
loader) builds into ``libocelotl_hip.so``.
"""
__all__ = ["okq", "backend", "build"]
