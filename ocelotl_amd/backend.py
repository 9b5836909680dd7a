"""Host-side mirror of Ocelotl's kernel dispatch boundary for the k-quant path.

This mirrors, in Python over the C-ABI, the parts of the reference's
``KernelBackend`` trait (``crates/kernels/src/lib.rs:84-495``) and core error
types (``crates/core/src/lib.rs:15-99``) that the quantized linear touches:

* :class:`HipKernelBackend` -- ``name()`` = ``"hip-gfx950"``, ``context()``
  (``Device::Gpu{ordinal}``), ``upload``/``alloc`` (``lib.rs:171-181``),
  ``linear_out_by_in`` over host slices (``lib.rs:106-116``) and ``linear_d``
  over device-resident tensors (``lib.rs:186-217``), both taking a
  :class:`QuantizedWeight` in place of the f32 ``weight_out_by_in``; plus
  ``dequantize`` (no reference signature exists; same argument style).
* :class:`DeviceTensor` -- an f32 device buffer (``tensor.rs:45-268``:
  ``len``, ``to_host_owned``, ``write_from_host_slice``).
* :class:`KernelError` / :class:`UnsupportedError` -- the reference's error
  structs, raised before any launch, exactly where the reference validates.

Device memory and streams come from PyTorch (plumbing only); every compute
call goes through ``libokq.so``.  There is no CPU fallback: without a gfx950
device the calls raise.
"""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from . import okq


# ---------------------------------------------------------------------------
# core types (crates/core/src/lib.rs)
# ---------------------------------------------------------------------------

class OcelotlError(Exception):
    """OcelotlError (crates/core/src/lib.rs:15-31)."""


class KernelError(OcelotlError):
    """KernelError{backend, message} (crates/core/src/lib.rs:69-74)."""

    def __init__(self, backend: str, message: str):
        super().__init__(f"kernel error on backend `{backend}`: {message}")
        self.backend = backend
        self.message = message


class UnsupportedError(OcelotlError):
    """UnsupportedError{feature, requested, supported} (lib.rs:51-61)."""

    def __init__(self, feature: str, requested: Optional[str], supported: Sequence[str]):
        req = f" (requested `{requested}`)" if requested is not None else ""
        super().__init__(f"unsupported feature `{feature}`{req}: supported = [{', '.join(supported)}]")
        self.feature = feature
        self.requested = requested
        self.supported = list(supported)


@dataclass(frozen=True)
class Device:
    """Device::Cpu | Device::Gpu{ordinal} (crates/core/src/lib.rs:438-441)."""
    kind: str
    ordinal: int = 0

    @staticmethod
    def gpu(ordinal: int) -> "Device":
        return Device("gpu", ordinal)


@dataclass(frozen=True)
class KernelContext:
    device: Device


class GgmlTensorType(enum.IntEnum):
    """Raw GGML type ids (crates/loader/src/gguf_inspect.rs:170-206), the
    subset this path understands plus the unquantized float types."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q2K = 10
    Q3K = 11
    Q4K = 12
    Q5K = 13
    Q6K = 14
    BF16 = 30


# Weight formats the linear kernels execute.
QUANTIZED = (GgmlTensorType.Q8_0, GgmlTensorType.Q4K, GgmlTensorType.Q5K, GgmlTensorType.Q6K)
# Every block format dequantize and the row gather accept.
BLOCK_FORMATS = (GgmlTensorType.Q4_0, GgmlTensorType.Q4_1, GgmlTensorType.Q5_0, GgmlTensorType.Q5_1,
                 GgmlTensorType.Q8_0, GgmlTensorType.Q2K, GgmlTensorType.Q3K, GgmlTensorType.Q4K,
                 GgmlTensorType.Q5K, GgmlTensorType.Q6K)
BACKEND = "hip-gfx950"


def _status_to_error(err: okq.OkqStatusError, type_id: Optional[int] = None) -> OcelotlError:
    if err.status == okq.E_TYPE:
        return UnsupportedError("quantized_tensor_type", None if type_id is None else str(type_id),
                                [t.name for t in QUANTIZED])
    if err.status == okq.E_NODEV:
        return UnsupportedError("gpu_backend", "gfx950", [])
    return KernelError(BACKEND, err.message)


def _call(name: str, *args, type_id: Optional[int] = None) -> None:
    try:
        okq.call(name, *args)
    except okq.OkqStatusError as e:
        raise _status_to_error(e, type_id) from None


def block_info(tensor_type: int):
    """(elements, bytes) per block -- the byte_len the GGUF inspector leaves
    as None for quantized types (gguf_inspect.rs:208-219)."""
    e, b = ctypes.c_int64(), ctypes.c_int64()
    _call("okq_type_info", int(tensor_type), ctypes.byref(e), ctypes.byref(b), type_id=int(tensor_type))
    return e.value, b.value


def tensor_byte_len(tensor_type: int, shape_ne: Sequence[int]) -> int:
    """Byte length of a GGUF tensor given its ne-order shape."""
    arr = (ctypes.c_int64 * len(shape_ne))(*shape_ne)
    out = ctypes.c_uint64()
    _call("okq_tensor_bytes", int(tensor_type), arr, len(shape_ne), ctypes.byref(out), type_id=int(tensor_type))
    return out.value


# ---------------------------------------------------------------------------
# device buffers (crates/kernels/src/tensor.rs)
# ---------------------------------------------------------------------------

def _torch():
    import torch  # plumbing only: device memory and streams
    return torch


class DeviceTensor:
    """f32 device buffer (the Device residency of tensor.rs:87-268)."""

    def __init__(self, t):
        torch = _torch()
        if t.dtype != torch.float32 or not t.is_cuda:
            raise KernelError(BACKEND, "DeviceTensor must be a float32 device tensor")
        self.t = t.contiguous().view(-1)

    def len(self) -> int:  # noqa: A003 -- mirrors DeviceTensor::len
        return self.t.numel()

    def ptr(self) -> int:
        return self.t.data_ptr()

    def to_host_owned(self) -> np.ndarray:
        return self.t.detach().cpu().numpy().copy()

    def write_from_host_slice(self, src) -> None:
        src = np.ascontiguousarray(src, dtype=np.float32).reshape(-1)
        if src.size != self.len():
            raise KernelError(BACKEND, f"write_from_host_slice length {src.size} != tensor length {self.len()}")
        self.t.copy_(_torch().from_numpy(src))


@dataclass
class QuantizedWeight:
    """A GGUF weight tensor resident on the device, in its on-disk layout:
    shape [ne0 = in_features, ne1 = out_features] (gguf_inspect.rs:118-130)."""
    tensor_type: GgmlTensorType
    ne0: int
    ne1: int
    data: object  # torch.uint8 device tensor of byte_len bytes

    @property
    def in_features(self) -> int:
        return self.ne0

    @property
    def out_features(self) -> int:
        return self.ne1

    @property
    def byte_len(self) -> int:
        return self.data.numel()

    def ptr(self) -> int:
        return self.data.data_ptr()


# ---------------------------------------------------------------------------
# backend
# ---------------------------------------------------------------------------

class HipKernelBackend:
    """The gfx950 backend object (KernelBackend, lib.rs:84-495)."""

    def __init__(self, ordinal: int = 0):
        _call("okq_init", int(ordinal))
        torch = _torch()
        self._ctx = KernelContext(Device.gpu(ordinal))
        self._device = torch.device("cuda", ordinal)

    # -- identity -------------------------------------------------------------
    def name(self) -> str:
        return okq.backend_name()

    def context(self) -> KernelContext:
        return self._ctx

    def _stream(self) -> int:
        return _torch().cuda.current_stream(self._device).cuda_stream

    # -- buffers --------------------------------------------------------------
    def upload(self, host) -> DeviceTensor:
        torch = _torch()
        arr = np.ascontiguousarray(host, dtype=np.float32).reshape(-1)
        return DeviceTensor(torch.from_numpy(arr).to(self._device))

    def alloc(self, length: int) -> DeviceTensor:
        return DeviceTensor(_torch().zeros(int(length), dtype=_torch().float32, device=self._device))

    def upload_quantized(self, tensor_type: int, ne0: int, ne1: int, blocks) -> QuantizedWeight:
        """Upload raw GGUF blocks of any block format (dequantize serves all of
        them; linear_d takes Q8_0 / Q4K / Q5K / Q6K); validates the byte length first."""
        torch = _torch()
        tt = int(tensor_type)
        if tt not in [int(t) for t in BLOCK_FORMATS]:
            raise UnsupportedError("quantized_tensor_type", str(tt), [t.name for t in BLOCK_FORMATS])
        want = tensor_byte_len(tt, [ne0, ne1])
        if isinstance(blocks, np.ndarray):
            b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
            if b.size != want:
                raise KernelError(BACKEND, f"quantized weight has {b.size} bytes, shape [{ne0}, {ne1}] needs {want}")
            data = torch.from_numpy(b).to(self._device)
        else:
            data = blocks.contiguous().view(-1)
            if data.numel() != want:
                raise KernelError(BACKEND, f"quantized weight has {data.numel()} bytes, shape [{ne0}, {ne1}] needs {want}")
        return QuantizedWeight(GgmlTensorType(tt), int(ne0), int(ne1), data)

    # -- compute ----------------------------------------------------------------
    def dequantize(self, weight: QuantizedWeight) -> DeviceTensor:
        n = weight.ne0 * weight.ne1
        out = _torch().empty(n, dtype=_torch().float32, device=self._device)
        _call("okq_dequantize", int(weight.tensor_type), weight.ptr(), n, out.data_ptr(), self._stream(),
              type_id=int(weight.tensor_type))
        return DeviceTensor(out)

    def linear_d(self, x: DeviceTensor, rows: int, in_features: int, weight: QuantizedWeight, out_features: int,
                 bias: Optional[DeviceTensor], out: DeviceTensor) -> None:
        """Device-resident linear (lib.rs:186-217); `out` caller-supplied."""
        if weight.ne0 != in_features or weight.ne1 != out_features:
            raise KernelError(BACKEND, f"linear_d weight shape [{weight.ne0}, {weight.ne1}] does not match "
                                       f"in_features={in_features} out_features={out_features}")
        if x.len() != rows * in_features:
            raise KernelError(BACKEND, f"linear_out_by_in x.len()={x.len()} does not match "
                                       f"rows*in_features={rows}*{in_features}={rows * in_features}")
        if bias is not None and bias.len() != out_features:
            raise KernelError(BACKEND, f"linear_out_by_in bias.len()={bias.len()} does not match "
                                       f"out_features={out_features}")
        if out.len() != rows * out_features:
            raise KernelError(BACKEND, f"linear_out_by_in out.len()={out.len()} does not match "
                                       f"rows*out_features={rows}*{out_features}={rows * out_features}")
        _call("okq_linear_out_by_in_q", x.ptr(), rows, in_features, int(weight.tensor_type), weight.ptr(),
              weight.byte_len, out_features, None if bias is None else bias.ptr(), out.ptr(), self._stream(),
              type_id=int(weight.tensor_type))

    def linear_out_by_in(self, x, rows: int, in_features: int, weight: QuantizedWeight, out_features: int,
                         bias, out: np.ndarray) -> None:
        """Host-slice linear (lib.rs:106-116): uploads x/bias, runs on the GPU,
        writes `out` in place (the trait default's host bounce, lib.rs:193-217)."""
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        if x.size != rows * in_features:
            raise KernelError(BACKEND, f"linear_out_by_in x.len()={x.size} does not match "
                                       f"rows*in_features={rows}*{in_features}={rows * in_features}")
        if out.size != rows * out_features:
            raise KernelError(BACKEND, f"linear_out_by_in out.len()={out.size} does not match "
                                       f"rows*out_features={rows}*{out_features}={rows * out_features}")
        xd = self.upload(x)
        bd = None if bias is None else self.upload(bias)
        od = self.alloc(rows * out_features)
        self.linear_d(xd, rows, in_features, weight, out_features, bd, od)
        out.reshape(-1)[:] = od.to_host_owned()
