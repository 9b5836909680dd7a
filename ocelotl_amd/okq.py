"""ctypes binding of ``libokq.so`` (the C-ABI declared in ``include/okq.h``).

The library must have been built in-tree (``python -m ocelotl_amd.build`` or
``__graft_entry__.build()``); there is no fallback: :func:`lib` raises
:class:`LibraryMissing` when the shared object is absent.
"""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libokq.so")

# okq_status
OK, E_SHAPE, E_TYPE, E_ALIGN, E_NODEV, E_LAUNCH, E_ARG, E_ALLOC = range(8)
STATUS_NAMES = {0: "OKQ_OK", 1: "OKQ_E_SHAPE", 2: "OKQ_E_TYPE", 3: "OKQ_E_ALIGN", 4: "OKQ_E_NODEV",
                5: "OKQ_E_LAUNCH", 6: "OKQ_E_ARG", 7: "OKQ_E_ALLOC"}

# Exported symbols and their signatures: (restype, argtypes).
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_u32 = ctypes.c_uint32
_int = ctypes.c_int
_linear_sig = (_int, [_vp, _i64, _i64, _u32, _vp, _u64, _i64, _vp, _vp, _vp])
SIGNATURES = {
    "okq_backend_name": (ctypes.c_char_p, []),
    "okq_last_error": (ctypes.c_size_t, [ctypes.c_char_p, ctypes.c_size_t]),
    "okq_type_info": (_int, [_u32, ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "okq_row_bytes": (_int, [_u32, _i64, ctypes.POINTER(_i64)]),
    "okq_tensor_bytes": (_int, [_u32, ctypes.POINTER(_i64), _int, ctypes.POINTER(_u64)]),
    "okq_init": (_int, [_int]),
    "okq_device_count": (_int, [ctypes.POINTER(_int)]),
    "okq_alloc": (_int, [ctypes.POINTER(_vp), ctypes.c_size_t]),
    "okq_free": (_int, [_vp]),
    "okq_memcpy_h2d": (_int, [_vp, _vp, ctypes.c_size_t, _vp]),
    "okq_memcpy_d2h": (_int, [_vp, _vp, ctypes.c_size_t, _vp]),
    "okq_sync": (_int, [_vp]),
    "okq_dequantize": (_int, [_u32, _vp, _i64, _vp, _vp]),
    "okq_linear_out_by_in_q": _linear_sig,
    "okq_linear_out_by_in_q_bf16": _linear_sig,
    "okq_linear_out_by_in_q_noalloc": _linear_sig,
    "okq_gemv": _linear_sig,
    "okq_gemm": _linear_sig,
    "okq_gemm_bf16": _linear_sig,
    "okq_gemv_multi": (_int, [_vp, _i64, _i64, _u32, _int, _vp, _vp, _vp, _vp, _vp, _vp]),
    "okq_linear_multi_q": (_int, [_vp, _i64, _i64, _int, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "okq_get_rows_q": (_int, [_u32, _vp, _u64, _i64, _i64, _vp, _i64, _vp, _vp]),
    "okq_rmsnorm": (_int, [_vp, _i64, _i64, _vp, ctypes.c_float, _vp, _vp]),
    "okq_rmsnorm_linear_q_multi": (_int, [_vp, _i64, _i64, _vp, ctypes.c_float, _u32, _int, _vp, _vp, _vp, _vp,
                                          _vp, _vp]),
    "okq_mlp_gated_silu_q": (_int, [_vp, _i64, _i64, _i64, _u32, _vp, _u64, _u32, _vp, _u64, _u32, _vp, _u64,
                                    _vp, _vp, _vp, _vp]),
    "okq_set_launch_events": (_int, [_vp, _vp]),
    "okq_quantize": (_int, [_u32, _vp, _i64, _vp, _vp]),
    "okq_fill_normal": (_int, [_u64, _i64, _i64, ctypes.c_float, _vp, _vp]),
    "okq_f32_to_bf16": (_int, [_vp, _i64, _vp, _vp]),
}


class LibraryMissing(RuntimeError):
    pass


class OkqStatusError(RuntimeError):
    """A non-OK okq_status with the library's message."""

    def __init__(self, status: int, message: str, call: str):
        super().__init__(f"{call}: {STATUS_NAMES.get(status, status)}: {message}")
        self.status = status
        self.message = message
        self.call = call


_lock = threading.Lock()
_lib = None


def lib() -> ctypes.CDLL:
    """Load libokq.so once (raises LibraryMissing if it was not built)."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise LibraryMissing(f"{LIB_PATH} not found: build it with `python -m ocelotl_amd.build`")
            handle = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
        return _lib


def last_error() -> str:
    buf = ctypes.create_string_buffer(1024)
    lib().okq_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(status: int, call: str) -> None:
    if status != OK:
        raise OkqStatusError(status, last_error(), call)


def call(name: str, *args) -> int:
    """Call an entry point and raise OkqStatusError on a non-OK status."""
    rc = getattr(lib(), name)(*args)
    check(rc, name)
    return rc


def backend_name() -> str:
    return lib().okq_backend_name().decode()
