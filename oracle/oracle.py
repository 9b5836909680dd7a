"""CPU oracle for the k-quant linear path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker or as the timed
CPU baseline.  The product (``ocelotl_amd``) never imports it.

Two independent restatements live here:

* :class:`Oracle` -- ctypes binding of ``liboracle.so`` (``kquant_oracle.c``):
  fp16/bf16 decode (``crates/loader/src/safetensors_values.rs:115-183``),
  block dequant, the build's quantizers, the seeded generator and the
  reference CPU linear path (``crates/kernels/src/lib.rs:1974-2123``,
  ``:2216-2239``, ``:2294-2390``; ``crates/kernels/src/cpu_avx2.rs:58-253``).
* ``np_dequant_*`` -- a second decoder written from the GGUF block spec with
  explicit per-bit field extraction in numpy (no table, no shared code with
  the C file).  Tests require both decoders to agree bit for bit.

Parity status of each oracle function (what pins it) is recorded in the test
modules ``tests/test_oracle_*.py``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

# GGML type ids (crates/loader/src/gguf_inspect.rs:170-206)
F32, F16, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 8, 12, 14, 30
# the other block formats GgmlTensorType names (gguf_inspect.rs:132-167) that
# the dequantize and row-gather entry points serve
Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q5_K = 2, 3, 6, 7, 10, 11, 13
LINEAR_TYPES = (Q8_0, Q4_K, Q5_K, Q6_K)
GATHER_TYPES = (Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K)
BLOCK_ELEMS = {Q4_0: 32, Q4_1: 32, Q5_0: 32, Q5_1: 32, Q8_0: 32,
               Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256}
BLOCK_BYTES = {Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24, Q8_0: 34,
               Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210}
# byte offsets of the f16 fields (d, and m / dmin where present) in a block
F16_FIELDS = {Q4_0: (0,), Q4_1: (0, 2), Q5_0: (0,), Q5_1: (0, 2), Q8_0: (0,),
              Q2_K: (80, 82), Q3_K: (108,), Q4_K: (0, 2), Q5_K: (0, 2), Q6_K: (208,)}
TYPE_NAMES = {Q4_0: "Q4_0", Q4_1: "Q4_1", Q5_0: "Q5_0", Q5_1: "Q5_1", Q8_0: "Q8_0",
              Q2_K: "Q2_K", Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K"}

MODE_SCALAR, MODE_OPTIMIZED, MODE_AVX2 = 0, 1, 2

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i64 = ctypes.c_int64


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE, "-B" if force else "all"], check=True)
    return LIB_PATH


def _ptr(a: np.ndarray, t):
    return a.ctypes.data_as(t)


class Oracle:
    """ctypes front-end of liboracle.so (numpy in, numpy out)."""

    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            build()
        lib = ctypes.CDLL(path)
        self.lib = lib
        lib.okr_f16_to_f32.restype = ctypes.c_float
        lib.okr_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.okr_bf16_to_f32.restype = ctypes.c_float
        lib.okr_bf16_to_f32.argtypes = [ctypes.c_uint16]
        lib.okr_f32_to_f16.restype = ctypes.c_uint16
        lib.okr_f32_to_f16.argtypes = [ctypes.c_float]
        lib.okr_f32_to_bf16.restype = ctypes.c_uint16
        lib.okr_f32_to_bf16.argtypes = [ctypes.c_float]
        for name, a, b in (("okr_f16_to_f32_array", _u16p, _f32p), ("okr_bf16_to_f32_array", _u16p, _f32p),
                           ("okr_f32_to_f16_array", _f32p, _u16p), ("okr_f32_to_bf16_array", _f32p, _u16p)):
            f = getattr(lib, name)
            f.restype = None
            f.argtypes = [a, _i64, b]
        lib.okr_dequantize.restype = ctypes.c_int
        lib.okr_dequantize.argtypes = [ctypes.c_int, _u8p, _i64, _f32p]
        lib.okr_quantize.restype = ctypes.c_int
        lib.okr_quantize.argtypes = [ctypes.c_int, _f32p, _i64, _u8p]
        lib.okr_fill_normal.restype = None
        lib.okr_fill_normal.argtypes = [ctypes.c_uint64, _i64, _i64, ctypes.c_float, _f32p]
        lib.okr_normal_at.restype = ctypes.c_float
        lib.okr_normal_at.argtypes = [ctypes.c_uint64, _i64, ctypes.c_float]
        lib.okr_linear_out_by_in.restype = ctypes.c_int
        lib.okr_linear_out_by_in.argtypes = [ctypes.c_int, ctypes.c_int, _f32p, _i64, _i64, _f32p, _i64, _f32p, _f32p]
        lib.okr_linear_q.restype = ctypes.c_int
        lib.okr_linear_q.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, _i64, _i64, _u8p, _i64,
                                     _f32p, _f32p]
        lib.okr_validate_linear.restype = ctypes.c_int
        lib.okr_validate_linear.argtypes = [_i64] * 7
        lib.okr_last_error.restype = ctypes.c_char_p
        lib.okr_has_avx2.restype = ctypes.c_int
        lib.okr_block_bytes.restype = _i64
        lib.okr_block_bytes.argtypes = [ctypes.c_int]
        lib.okr_block_elems.restype = _i64
        lib.okr_block_elems.argtypes = [ctypes.c_int]
        lib.okr_rmsnorm.restype = None
        lib.okr_rmsnorm.argtypes = [_f32p, _i64, _i64, _f32p, ctypes.c_float, _f32p]
        lib.okr_swiglu.restype = None
        lib.okr_swiglu.argtypes = [_f32p, _f32p, _i64, _f32p]

    # ---- scalar conversions -------------------------------------------------
    def f16_to_f32(self, bits: np.ndarray) -> np.ndarray:
        bits = np.ascontiguousarray(bits, dtype=np.uint16)
        out = np.empty(bits.shape, np.float32)
        self.lib.okr_f16_to_f32_array(_ptr(bits, _u16p), bits.size, _ptr(out, _f32p))
        return out

    def bf16_to_f32(self, bits: np.ndarray) -> np.ndarray:
        bits = np.ascontiguousarray(bits, dtype=np.uint16)
        out = np.empty(bits.shape, np.float32)
        self.lib.okr_bf16_to_f32_array(_ptr(bits, _u16p), bits.size, _ptr(out, _f32p))
        return out

    def f32_to_f16(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, np.uint16)
        self.lib.okr_f32_to_f16_array(_ptr(x, _f32p), x.size, _ptr(out, _u16p))
        return out

    def f32_to_bf16(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, np.uint16)
        self.lib.okr_f32_to_bf16_array(_ptr(x, _f32p), x.size, _ptr(out, _u16p))
        return out

    # ---- blocks -------------------------------------------------------------
    def dequantize(self, ggml_type: int, blocks: np.ndarray, n: int) -> np.ndarray:
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        assert blocks.size == n // BLOCK_ELEMS[ggml_type] * BLOCK_BYTES[ggml_type]
        out = np.empty(n, np.float32)
        rc = self.lib.okr_dequantize(ggml_type, _ptr(blocks, _u8p), n, _ptr(out, _f32p))
        if rc:
            raise ValueError(f"okr_dequantize rc={rc}")
        return out

    def quantize(self, ggml_type: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        nb = x.size // BLOCK_ELEMS[ggml_type]
        out = np.empty(nb * BLOCK_BYTES[ggml_type], np.uint8)
        rc = self.lib.okr_quantize(ggml_type, _ptr(x, _f32p), x.size, _ptr(out, _u8p))
        if rc:
            raise ValueError(f"okr_quantize rc={rc}")
        return out

    def normal(self, seed: int, n: int, sigma: float = 1.0, offset: int = 0) -> np.ndarray:
        out = np.empty(n, np.float32)
        self.lib.okr_fill_normal(seed, offset, n, sigma, _ptr(out, _f32p))
        return out

    # ---- reference CPU linear path -------------------------------------------
    def linear(self, x: np.ndarray, rows: int, in_f: int, w: np.ndarray, out_f: int, bias=None,
               mode: int = MODE_SCALAR, threads: int = 1) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        out = np.empty(rows * out_f, np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        rc = self.lib.okr_validate_linear(x.size, rows, in_f, w.size, out_f, -1 if b is None else b.size, out.size)
        if rc:
            raise ValueError(self.lib.okr_last_error().decode())
        rc = self.lib.okr_linear_out_by_in(mode, threads, _ptr(x, _f32p), rows, in_f, _ptr(w, _f32p), out_f,
                                           None if b is None else _ptr(b, _f32p), _ptr(out, _f32p))
        if rc:
            raise ValueError(self.lib.okr_last_error().decode())
        return out.reshape(rows, out_f)

    def linear_q(self, ggml_type: int, x: np.ndarray, rows: int, in_f: int, wq: np.ndarray, out_f: int,
                 bias=None, mode: int = MODE_SCALAR, threads: int = 1) -> np.ndarray:
        w = self.dequantize(ggml_type, wq, out_f * in_f)
        return self.linear(x, rows, in_f, w, out_f, bias, mode, threads)

    def rmsnorm(self, x: np.ndarray, rows: int, hidden: int, weight: np.ndarray, eps: float) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        w = np.ascontiguousarray(weight, np.float32).reshape(-1)
        assert x.size == rows * hidden and w.size == hidden
        out = np.empty(rows * hidden, np.float32)
        self.lib.okr_rmsnorm(_ptr(x, _f32p), rows, hidden, _ptr(w, _f32p), ctypes.c_float(eps),
                             _ptr(out, _f32p))
        return out

    def swiglu(self, gate: np.ndarray, up: np.ndarray) -> np.ndarray:
        g = np.ascontiguousarray(gate, np.float32).reshape(-1)
        u = np.ascontiguousarray(up, np.float32).reshape(-1)
        assert g.size == u.size
        out = np.empty(g.size, np.float32)
        self.lib.okr_swiglu(_ptr(g, _f32p), _ptr(u, _f32p), g.size, _ptr(out, _f32p))
        return out

    def validate(self, x_len, rows, in_f, w_len, out_f, bias_len, out_len):
        rc = self.lib.okr_validate_linear(x_len, rows, in_f, w_len, out_f, bias_len, out_len)
        return None if rc == 0 else self.lib.okr_last_error().decode()

    def has_avx2(self) -> bool:
        return bool(self.lib.okr_has_avx2())


# ----------------------------------------------------------------------------
# Independent numpy decoder (bit-field extraction straight from the spec)
# ----------------------------------------------------------------------------

def np_f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """IEEE half -> float via numpy's own float16 (independent of the C code)."""
    return np.ascontiguousarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def _bit(v, i):
    return (v >> i) & 1


def np_dequant_q8_0(blocks: np.ndarray) -> np.ndarray:
    b = np.asarray(blocks, np.uint8).reshape(-1, 34)
    d = np_f16_bits_to_f32(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (q * d[:, None]).astype(np.float32).reshape(-1)


def _q4k_field(scales: np.ndarray, j: int):
    """6-bit (scale, min) of sub-block j, assembled bit by bit."""
    sc = np.zeros(scales.shape[0], np.int64)
    mn = np.zeros(scales.shape[0], np.int64)
    s = scales.astype(np.int64)
    if j < 4:
        for i in range(6):
            sc |= _bit(s[:, j], i) << i
            mn |= _bit(s[:, j + 4], i) << i
    else:
        for i in range(4):
            sc |= _bit(s[:, j + 4], i) << i
            mn |= _bit(s[:, j + 4], 4 + i) << i
        for i in range(2):
            sc |= _bit(s[:, j - 4], 6 + i) << (4 + i)
            mn |= _bit(s[:, j], 6 + i) << (4 + i)
    return sc, mn


def np_dequant_q4_k(blocks: np.ndarray) -> np.ndarray:
    b = np.asarray(blocks, np.uint8).reshape(-1, 144)
    nb = b.shape[0]
    d = np_f16_bits_to_f32(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
    dmin = np_f16_bits_to_f32(b[:, 2].astype(np.uint16) | (b[:, 3].astype(np.uint16) << 8))
    scales = b[:, 4:16]
    qs = b[:, 16:144].astype(np.int64)
    y = np.empty((nb, 256), np.float32)
    for e in range(256):
        c, r = divmod(e, 64)          # 64-element chunk, position in chunk
        hi, l = divmod(r, 32)         # low or high nibble, byte within chunk
        j = 2 * c + hi                # sub-block
        q = (qs[:, 32 * c + l] >> (4 * hi)) & 15
        sc, mn = _q4k_field(scales, j)
        ds = (d * sc.astype(np.float32)).astype(np.float32)
        dm = (dmin * mn.astype(np.float32)).astype(np.float32)
        y[:, e] = (ds * q.astype(np.float32)).astype(np.float32) - dm
    return y.reshape(-1)


def np_dequant_q6_k(blocks: np.ndarray) -> np.ndarray:
    b = np.asarray(blocks, np.uint8).reshape(-1, 210)
    nb = b.shape[0]
    ql = b[:, 0:128].astype(np.int64)
    qh = b[:, 128:192].astype(np.int64)
    sc = b[:, 192:208].view(np.int8).astype(np.float32)
    d = np_f16_bits_to_f32(b[:, 208].astype(np.uint16) | (b[:, 209].astype(np.uint16) << 8))
    y = np.empty((nb, 256), np.float32)
    for e in range(256):
        h, r = divmod(e, 128)         # half
        quarter, l = divmod(r, 32)    # which of the four 32-runs, position
        # low 4 bits: ql byte (l or l+32) of this half, low nibble for runs 0/1, high for 2/3
        ql_byte = ql[:, 64 * h + l + (32 if quarter in (1, 3) else 0)]
        lo4 = (ql_byte >> (4 if quarter >= 2 else 0)) & 15
        hi2 = (qh[:, 32 * h + l] >> (2 * quarter)) & 3
        q = (lo4 | (hi2 << 4)) - 32
        s = sc[:, 8 * h + l // 16 + 2 * quarter]
        ds = (d * s).astype(np.float32)
        y[:, e] = (ds * q.astype(np.float32)).astype(np.float32)
    return y.reshape(-1)


def _f16_at(b: np.ndarray, off: int) -> np.ndarray:
    return np_f16_bits_to_f32(b[:, off].astype(np.uint16) | (b[:, off + 1].astype(np.uint16) << 8))


def _legacy32(blocks, nbytes, has_min, has_high):
    """Q4_0 / Q4_1 / Q5_0 / Q5_1: 32 elements; element e < 16 is the low nibble
    of qs[e], e >= 16 the high nibble of qs[e-16]; the Q5 formats add bit e of
    the 32-bit little-endian qh word as the fifth bit; the symmetric formats
    subtract 8 (Q4_0) or 16 (Q5_0) and have no min."""
    b = np.asarray(blocks, np.uint8).reshape(-1, nbytes)
    d = _f16_at(b, 0)
    off = 2
    m = None
    if has_min:
        m = _f16_at(b, 2)
        off = 4
    qh = None
    if has_high:
        qh = b[:, off:off + 4].astype(np.int64)
        off += 4
    qs = b[:, off:off + 16].astype(np.int64)
    y = np.empty((b.shape[0], 32), np.float32)
    for e in range(32):
        v = (qs[:, e % 16] >> (4 * (e // 16))) & 15
        if has_high:
            v = v | (((qh[:, e // 8] >> (e % 8)) & 1) << 4)
        if not has_min:
            v = v - (16 if has_high else 8)
        prod = (v.astype(np.float32) * d).astype(np.float32)
        y[:, e] = prod if m is None else (prod + m).astype(np.float32)
    return y.reshape(-1)


def np_dequant_q4_0(blocks):
    return _legacy32(blocks, 18, False, False)


def np_dequant_q4_1(blocks):
    return _legacy32(blocks, 20, True, False)


def np_dequant_q5_0(blocks):
    return _legacy32(blocks, 22, False, True)


def np_dequant_q5_1(blocks):
    return _legacy32(blocks, 24, True, True)


def np_dequant_q2_k(blocks: np.ndarray) -> np.ndarray:
    b = np.asarray(blocks, np.uint8).reshape(-1, 84)
    d, dmin = _f16_at(b, 80), _f16_at(b, 82)
    y = np.empty((b.shape[0], 256), np.float32)
    for e in range(256):
        h, r = divmod(e, 128)
        j, s = divmod(r, 32)
        byte = b[:, 16 + 32 * h + s].astype(np.int64)
        q = _bit(byte, 2 * j) | (_bit(byte, 2 * j + 1) << 1)
        sc = b[:, e // 16].astype(np.int64)
        dl = (d * (sc & 15).astype(np.float32)).astype(np.float32)
        ml = (dmin * (sc >> 4).astype(np.float32)).astype(np.float32)
        y[:, e] = ((dl * q.astype(np.float32)).astype(np.float32) - ml).astype(np.float32)
    return y.reshape(-1)


def _q3k_field(scales: np.ndarray, i: int) -> np.ndarray:
    """6-bit scale i of a Q3_K block, bit by bit: bits 0-3 from byte i (i < 8,
    low nibble) or byte i-8 (high nibble); bits 4-5 from byte 8 + i%4 at bit
    offset 2*(i//4)."""
    s = scales.astype(np.int64)
    v = np.zeros(s.shape[0], np.int64)
    src, base = (i, 0) if i < 8 else (i - 8, 4)
    for k in range(4):
        v |= _bit(s[:, src], base + k) << k
    for k in range(2):
        v |= _bit(s[:, 8 + i % 4], 2 * (i // 4) + k) << (4 + k)
    return v


def np_dequant_q3_k(blocks: np.ndarray) -> np.ndarray:
    b = np.asarray(blocks, np.uint8).reshape(-1, 110)
    d = _f16_at(b, 108)
    y = np.empty((b.shape[0], 256), np.float32)
    for e in range(256):
        h, r = divmod(e, 128)
        j, s = divmod(r, 32)
        byte = b[:, 32 + 32 * h + s].astype(np.int64)
        q = _bit(byte, 2 * j) | (_bit(byte, 2 * j + 1) << 1)
        q = q - 4 * (1 - _bit(b[:, s].astype(np.int64), 4 * h + j))
        sc = _q3k_field(b[:, 96:108], e // 16) - 32
        dl = (d * sc.astype(np.float32)).astype(np.float32)
        y[:, e] = (dl * q.astype(np.float32)).astype(np.float32)
    return y.reshape(-1)


def np_dequant_q5_k(blocks: np.ndarray) -> np.ndarray:
    b = np.asarray(blocks, np.uint8).reshape(-1, 176)
    d, dmin = _f16_at(b, 0), _f16_at(b, 2)
    scales = b[:, 4:16]
    y = np.empty((b.shape[0], 256), np.float32)
    for e in range(256):
        c, r = divmod(e, 64)
        hi, l = divmod(r, 32)
        q = (b[:, 48 + 32 * c + l].astype(np.int64) >> (4 * hi)) & 15
        q = q + 16 * _bit(b[:, 16 + l].astype(np.int64), 2 * c + hi)
        sc, mn = _q4k_field(scales, 2 * c + hi)
        ds = (d * sc.astype(np.float32)).astype(np.float32)
        dm = (dmin * mn.astype(np.float32)).astype(np.float32)
        y[:, e] = ((ds * q.astype(np.float32)).astype(np.float32) - dm).astype(np.float32)
    return y.reshape(-1)


NP_DEQUANT = {Q8_0: np_dequant_q8_0, Q4_K: np_dequant_q4_k, Q6_K: np_dequant_q6_k,
              Q4_0: np_dequant_q4_0, Q4_1: np_dequant_q4_1, Q5_0: np_dequant_q5_0, Q5_1: np_dequant_q5_1,
              Q2_K: np_dequant_q2_k, Q3_K: np_dequant_q3_k, Q5_K: np_dequant_q5_k}


def np_linear_sequential(x: np.ndarray, w: np.ndarray, bias=None) -> np.ndarray:
    """Naive sequential f32 loop (acc = bias; acc += x*w, each op rounded):
    the exact-equality check of lib.rs:2843-2889.  Small sizes only."""
    x = np.asarray(x, np.float32)
    w = np.asarray(w, np.float32)
    rows, in_f = x.shape
    out_f = w.shape[0]
    out = np.empty((rows, out_f), np.float32)
    for r in range(rows):
        prods = (x[r][None, :] * w).astype(np.float32)  # [out, in], each product rounded
        acc = np.zeros(out_f, np.float32) if bias is None else np.asarray(bias, np.float32).copy()
        for k in range(in_f):
            acc = (acc + prods[:, k]).astype(np.float32)
        out[r] = acc
    return out


def allclose_ref_rule(got: np.ndarray, want: np.ndarray, tol: float):
    """The reference's per-element rule abs <= tol || rel <= tol
    (crates/kernels/src/lib.rs:2995-3002, cubecl_backend.rs:2578-2585).
    Returns (ok, index_of_first_failure, max_abs, max_rel)."""
    got = np.asarray(got, np.float64).reshape(-1)
    want = np.asarray(want, np.float64).reshape(-1)
    diff = np.abs(got - want)
    rel = diff / np.maximum(np.abs(want), 1e-30)
    bad = ~((diff <= tol) | (rel <= tol))
    idx = int(np.argmax(bad)) if bad.any() else -1
    return (not bad.any()), idx, float(diff.max(initial=0.0)), float(np.where(diff > tol, rel, 0).max(initial=0.0))
