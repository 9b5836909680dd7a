"""C-ABI surface of libokq.so (CPU only: no compute launches).

Checks that the library loads, exports every function include/okq.h
declares, and that the host-side contract (type table, GGUF byte lengths,
validation before launch, error codes) behaves as the reference's
validate_linear_out_by_in (crates/kernels/src/lib.rs:2443-2497) does.
"""
import ctypes
import os
import re

import pytest

from ocelotl_amd import okq

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    src = open(os.path.join(ROOT, "include", "okq.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(okq_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for must in ("okq_linear_out_by_in_q", "okq_dequantize", "okq_gemv", "okq_gemm", "okq_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol(okqlib):
    missing = [n for n in declared_functions() if not hasattr(okqlib, n)]
    assert not missing, missing
    assert set(declared_functions()) == set(okq.SIGNATURES), "ctypes signatures out of sync with okq.h"


def test_backend_name():
    assert okq.backend_name() == "hip-gfx950"


@pytest.mark.parametrize("t,elems,nbytes", [(8, 32, 34), (12, 256, 144), (14, 256, 210), (0, 1, 4), (1, 1, 2),
                                            (30, 1, 2), (2, 32, 18), (3, 32, 20), (6, 32, 22), (7, 32, 24),
                                            (10, 256, 84), (11, 256, 110), (13, 256, 176)])
def test_type_info(okqlib, t, elems, nbytes):
    e, b = ctypes.c_int64(), ctypes.c_int64()
    assert okqlib.okq_type_info(t, ctypes.byref(e), ctypes.byref(b)) == okq.OK
    assert (e.value, b.value) == (elems, nbytes)


def test_unknown_type_is_unsupported(okqlib):
    e, b = ctypes.c_int64(), ctypes.c_int64()
    assert okqlib.okq_type_info(9, ctypes.byref(e), ctypes.byref(b)) == okq.E_TYPE  # Q8_1: no block format here
    assert "(9)" in okq.last_error()
    assert okqlib.okq_type_info(99, ctypes.byref(e), ctypes.byref(b)) == okq.E_TYPE


def test_row_and_tensor_bytes(okqlib):
    out = ctypes.c_int64()
    for t, k, want in ((8, 4096, 4352), (12, 4096, 2304), (14, 4096, 3360), (12, 14336, 8064), (14, 14336, 11760)):
        assert okqlib.okq_row_bytes(t, k, ctypes.byref(out)) == okq.OK
        assert out.value == want
    assert okqlib.okq_row_bytes(12, 4000, ctypes.byref(out)) == okq.E_SHAPE
    shape = (ctypes.c_int64 * 2)(4096, 128256)
    tb = ctypes.c_uint64()
    assert okqlib.okq_tensor_bytes(14, shape, 2, ctypes.byref(tb)) == okq.OK
    assert tb.value == 430_940_160
    # the Gemma4 fixture's Q4_K token embedding [2560, 262144]
    shape = (ctypes.c_int64 * 2)(2560, 262144)
    assert okqlib.okq_tensor_bytes(12, shape, 2, ctypes.byref(tb)) == okq.OK
    assert tb.value == 2560 // 256 * 144 * 262144
    shape = (ctypes.c_int64 * 3)(256, 2**40, 2**40)
    assert okqlib.okq_tensor_bytes(12, shape, 3, ctypes.byref(tb)) == okq.E_SHAPE


def _linear(okqlib, rows, k, t, wbytes, n, x=1 << 12, w=1 << 12, out=1 << 12):
    return okqlib.okq_linear_out_by_in_q(x, rows, k, t, w, wbytes, n, None, out, None)


def test_linear_validation_happens_before_launch(okqlib):
    # weight byte length must equal out * row_bytes(in)
    assert _linear(okqlib, 1, 4096, 12, 2304 * 10 - 1, 10) == okq.E_SHAPE
    assert "does not match out_features*row_bytes" in okq.last_error()
    # in_features must be block aligned
    assert _linear(okqlib, 1, 4000, 12, 0, 10) == okq.E_SHAPE
    # unsupported type -> Unsupported: the dequantize-only block formats too
    for t in (2, 3, 6, 7, 10, 11, 0, 9):
        assert _linear(okqlib, 1, 4096, t, 0, 10) == okq.E_TYPE
        assert "supported: Q8_0, Q4K, Q5K, Q6K" in okq.last_error()
    # rows == 0 is a no-op even with null pointers (reference accepts empty slices)
    assert okqlib.okq_linear_out_by_in_q(None, 0, 4096, 12, None, 2304 * 10, 10, None, None, None) == okq.OK
    # null pointers with work to do
    assert okqlib.okq_linear_out_by_in_q(None, 1, 4096, 12, None, 2304 * 10, 10, None, None, None) == okq.E_ARG
    # misaligned activations
    assert _linear(okqlib, 1, 4096, 12, 2304 * 10, 10, x=(1 << 12) + 4) == okq.E_ALIGN
    # 32-bit launch limits
    assert _linear(okqlib, 1, 256, 12, 144 * (1 << 31), 1 << 31) == okq.E_SHAPE


def test_compute_without_gpu_reports_nodev(okqlib):
    cnt = ctypes.c_int()
    assert okqlib.okq_device_count(ctypes.byref(cnt)) == okq.OK
    if cnt.value > 0:
        pytest.skip("a GPU is present")
    assert okqlib.okq_init(0) == okq.E_NODEV
    # valid arguments, no device: refused with E_NODEV, nothing launched
    assert _linear(okqlib, 1, 4096, 12, 2304 * 10, 10) == okq.E_NODEV


def test_python_mirror_maps_errors():
    from ocelotl_amd import backend as B
    with pytest.raises(B.UnsupportedError):
        B.block_info(9)  # Q8_1: no block format here
    assert B.block_info(B.GgmlTensorType.Q6K) == (256, 210)
    assert B.block_info(B.GgmlTensorType.Q5K) == (256, 176)
    assert B.tensor_byte_len(B.GgmlTensorType.Q4K, [4096, 14336]) == 14336 * 2304
    with pytest.raises(B.KernelError) as ei:
        B.tensor_byte_len(B.GgmlTensorType.Q4K, [4000, 2])
    assert ei.value.backend == "hip-gfx950"
