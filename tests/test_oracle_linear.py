"""Pins the oracle's restatement of the reference CPU linear path (CPU only).

Each test restates one of the reference's own tests in
crates/kernels/src/lib.rs with the same inputs and tolerance:
  :2809-2840  optimized vs scalar with bias, |d| <= 1e-6
  :2843-2889  scalar 4x4 tiles + row/output tails == naive loop, exact
  :2891-2943  threaded == serial bit for bit (rows >= 32 take the chunked path)
  :2946-3005  AVX2 vs scalar, abs <= 1e-4 || rel <= 1e-4
  :2514-2545  validation messages (validate_linear_out_by_in, :2443-2497)
plus the one-hot invariant of the quantized path: x = e_j reproduces the
dequantized column j exactly.
"""
import numpy as np
import pytest

from oracle import oracle as O


def test_optimized_matches_scalar_with_bias(orc):
    x = np.array([1.0, -2.0, 0.5, -0.25, 1.5, 2.0], np.float32)
    w = np.array([0.5, -1.0, 0.25, -0.75, 0.5, 1.25, 1.0, 1.5, -1.0, 0.0, -0.5, 0.75], np.float32)
    b = np.array([0.1, -0.2, 0.3, -0.4], np.float32)
    s = orc.linear(x, 2, 3, w, 4, b, O.MODE_SCALAR)
    o = orc.linear(x, 2, 3, w, 4, b, O.MODE_OPTIMIZED)
    assert np.abs(s - o).max() <= 1e-6


def test_scalar_tiles_and_tails_equal_naive_loop(orc):
    x = np.arange(1, 16, dtype=np.float32)
    w = np.array([0.5, 1.0, -0.5, -1.0, 0.25, 0.75, 1.5, -0.25, 0.0, 0.0, -0.5, 2.0, -0.75, 0.5, 1.25], np.float32)
    b = np.array([0.1, -0.2, 0.3, -0.4, 0.5], np.float32)
    got = orc.linear(x, 5, 3, w, 5, b)
    want = O.np_linear_sequential(x.reshape(5, 3), w.reshape(5, 3), b)
    assert (got == want).all()


@pytest.mark.parametrize("rows,in_f,out_f", [(1, 7, 9), (3, 33, 5), (4, 16, 4), (7, 17, 13), (9, 64, 11)])
def test_scalar_equals_sequential_on_trig_inputs(orc, rows, in_f, out_f):
    i = np.arange(rows * in_f, dtype=np.float32)
    x = np.sin(i * np.float32(0.013)).astype(np.float32)
    w = np.cos(np.arange(out_f * in_f, dtype=np.float32) * np.float32(0.019)).astype(np.float32)
    b = (np.arange(out_f, dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    got = orc.linear(x, rows, in_f, w, out_f, b)
    want = O.np_linear_sequential(x.reshape(rows, in_f), w.reshape(out_f, in_f), b)
    assert (got == want).all()


@pytest.mark.parametrize("mode", [O.MODE_SCALAR, O.MODE_OPTIMIZED, O.MODE_AVX2])
def test_threaded_matches_serial_bit_for_bit(orc, mode):
    if mode == O.MODE_AVX2 and not orc.has_avx2():
        pytest.skip("host lacks avx2+fma")
    rows, in_f, out_f = 64, 17, 13
    x = np.sin(np.arange(rows * in_f, dtype=np.float32) * np.float32(0.013)).astype(np.float32)
    w = np.cos(np.arange(out_f * in_f, dtype=np.float32) * np.float32(0.019)).astype(np.float32)
    b = (np.arange(out_f, dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    serial = orc.linear(x, rows, in_f, w, out_f, b, mode, threads=1)
    threaded = orc.linear(x, rows, in_f, w, out_f, b, mode, threads=4)
    assert (serial.view(np.uint32) == threaded.view(np.uint32)).all()


def test_avx2_matches_scalar_within_tolerance(orc):
    if not orc.has_avx2():
        pytest.skip("host lacks avx2+fma")
    rows, in_f, out_f = 64, 200, 33
    x = np.sin(np.arange(rows * in_f, dtype=np.float32) * np.float32(0.011)).astype(np.float32)
    w = np.cos(np.arange(out_f * in_f, dtype=np.float32) * np.float32(0.017)).astype(np.float32)
    b = (np.arange(out_f, dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    s = orc.linear(x, rows, in_f, w, out_f, b, O.MODE_SCALAR)
    a = orc.linear(x, rows, in_f, w, out_f, b, O.MODE_AVX2)
    ok, idx, _, _ = O.allclose_ref_rule(a, s, 1e-4)
    assert ok, idx


def test_validation_messages(orc):
    msg = orc.validate(5, 2, 3, 12, 4, -1, 8)
    assert "x.len()=5 does not match rows*in_features=2*3=6" in msg
    msg = orc.validate(6, 2, 3, 11, 4, -1, 8)
    assert "weight.len()=11 does not match out_features*in_features=4*3=12" in msg
    msg = orc.validate(6, 2, 3, 12, 4, 3, 8)
    assert "bias.len()=3 does not match out_features=4" in msg
    msg = orc.validate(6, 2, 3, 12, 4, -1, 7)
    assert "out.len()=7 does not match rows*out_features=2*4=8" in msg
    assert orc.validate(0, 0, 3, 12, 4, -1, 0) is None


@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_K, O.Q6_K])
def test_quantized_one_hot_column_is_exact(orc, t):
    in_f, out_f = 512, 24
    wq = orc.quantize(t, orc.normal(31 + t, in_f * out_f, 0.02))
    w = orc.dequantize(t, wq, in_f * out_f).reshape(out_f, in_f)
    for j in (0, 1, 255, 256, 511):
        x = np.zeros(in_f, np.float32)
        x[j] = 1.0
        y = orc.linear_q(t, x, 1, in_f, wq, out_f)
        assert (y[0] == w[:, j]).all()


def test_linear_q_is_linear_in_x(orc):
    in_f, out_f = 512, 16
    wq = orc.quantize(O.Q4_K, orc.normal(5, in_f * out_f, 0.02))
    a = orc.normal(6, in_f)
    b = orc.normal(7, in_f)
    ya = orc.linear_q(O.Q4_K, a, 1, in_f, wq, out_f)
    yb = orc.linear_q(O.Q4_K, b, 1, in_f, wq, out_f)
    yab = orc.linear_q(O.Q4_K, (a + b).astype(np.float32), 1, in_f, wq, out_f)
    ok, idx, _, _ = O.allclose_ref_rule(yab, ya + yb, 1e-4)
    assert ok, idx
