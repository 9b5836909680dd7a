"""GPU parity of libokq.so against the CPU oracle (needs an MI355X).

Bars: dequant/quantize/generator bit-exact; GEMV within the reference rule
abs <= 1e-3 || rel <= 1e-3 per element (crates/kernels/src/lib.rs:2995-3002,
BASELINE north_star tolerance), exact for the one-hot column probe.
All calls go through the C-ABI (ctypes), device memory from torch.
"""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3
TYPES = [O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K]


@pytest.fixture(scope="module")
def torch():
    import torch as _t
    if not _t.cuda.is_available():
        pytest.skip("no GPU")
    return _t


@pytest.fixture(scope="module")
def okq(torch):
    from ocelotl_amd import okq as _okq
    _okq.call("okq_init", 0)
    return _okq


def _stream(torch):
    return torch.cuda.current_stream().cuda_stream


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    return t.cpu().numpy()


def _same_bits(a, b):
    a = np.asarray(a, np.float32).reshape(-1)
    b = np.asarray(b, np.float32).reshape(-1)
    return (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))


def gpu_dequant(torch, okq, t, blocks, n):
    src = _dev(torch, blocks)
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    okq.call("okq_dequantize", t, src.data_ptr(), n, out.data_ptr(), _stream(torch))
    return _host(out)


def gpu_linear(torch, okq, t, x, rows, k, wq, n, bias=None, entry="okq_linear_out_by_in_q"):
    xd = _dev(torch, np.asarray(x, np.float32).reshape(-1))
    wd = _dev(torch, wq)
    bd = None if bias is None else _dev(torch, np.asarray(bias, np.float32))
    out = torch.full((rows * n,), float("nan"), dtype=torch.float32, device="cuda")
    okq.call(entry, xd.data_ptr(), rows, k, t, wd.data_ptr(), wq.size, n,
             None if bd is None else bd.data_ptr(), out.data_ptr(), _stream(torch))
    torch.cuda.synchronize()
    return _host(out).reshape(rows, n)


# ---------------------------------------------------------------------------
# bit-exact data-path kernels
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("t", O.GATHER_TYPES)
def test_dequant_bit_exact_on_random_bytes(torch, okq, orc, t):
    print(f"[gpu] dequant random bytes type={t}", flush=True)
    rng = np.random.default_rng(10 + t)
    nb = 8192
    blocks = rng.integers(0, 256, nb * O.BLOCK_BYTES[t], dtype=np.uint8)
    n = nb * O.BLOCK_ELEMS[t]
    got = gpu_dequant(torch, okq, t, blocks, n)
    want = orc.dequantize(t, blocks, n)
    same = _same_bits(got, want)
    assert same.all(), f"{(~same).sum()} mismatches, first at {np.argmax(~same)}"
    finite = np.isfinite(want)
    assert (got[finite].view(np.uint32) == want[finite].view(np.uint32)).all()


@pytest.mark.parametrize("t", TYPES)
def test_dequant_bit_exact_on_quantized_normal(torch, okq, orc, t):
    n = 4096 * 64
    wq = orc.quantize(t, orc.normal(20 + t, n, 0.02))
    got = gpu_dequant(torch, okq, t, wq, n)
    assert (got.view(np.uint32) == orc.dequantize(t, wq, n).view(np.uint32)).all()


@pytest.mark.parametrize("t", TYPES)
def test_gpu_quantizer_matches_oracle_bytes(torch, okq, orc, t):
    print(f"[gpu] quantize type={t}", flush=True)
    n = 256 * 2048
    x = orc.normal(40 + t, n, 0.02)
    # include exact zeros, a constant block and large values
    x[:256] = 0.0
    x[256:512] = 0.125
    x[512:768] *= 1000.0
    xd = _dev(torch, x)
    out = torch.zeros(n // O.BLOCK_ELEMS[t] * O.BLOCK_BYTES[t], dtype=torch.uint8, device="cuda")
    okq.call("okq_quantize", t, xd.data_ptr(), n, out.data_ptr(), _stream(torch))
    got = _host(out)
    want = orc.quantize(t, x)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} bytes differ, first block {bad[0] // O.BLOCK_BYTES[t]}"


def test_fill_normal_matches_oracle(torch, okq, orc):
    n = 1 << 20
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    okq.call("okq_fill_normal", 0x5EED, 12345, n, 0.02, out.data_ptr(), _stream(torch))
    assert (_host(out).view(np.uint32) == orc.normal(0x5EED, n, 0.02, offset=12345).view(np.uint32)).all()


def test_f32_to_bf16_matches_oracle(torch, okq, orc):
    x = orc.normal(3, 1 << 18, 1.0) * np.float32(7.0)
    xd = _dev(torch, x)
    out = torch.empty(x.size, dtype=torch.int16, device="cuda")
    okq.call("okq_f32_to_bf16", xd.data_ptr(), x.size, out.data_ptr(), _stream(torch))
    assert (_host(out).view(np.uint16) == orc.f32_to_bf16(x)).all()


# ---------------------------------------------------------------------------
# GEMV parity
# ---------------------------------------------------------------------------

GEMV_SHAPES = {
    # few rows with long K (teams of waves per row, x covered by extra teams) included;
    # (20000, 256) gives one wave per row and five steps per wave: rows past each
    # wave's first ones come from the workgroup's counter
    O.Q4_K: [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336), (17, 256), (3, 768), (64, 20480),
             (300, 14336), (17, 8192), (2, 16384), (20000, 256)],
    # Q6_K: a unit's scales (and d) come in one 16-byte window that may reach
    # 2 bytes into the next block, so the streaming kernel takes tensors whose
    # last block starts 2 bytes off a dword (size a multiple of 4): odd
    # super-block counts with an even row count (34 x 768) stream, with an
    # odd one (33 x 768, 35 x 1280) they take the generic kernel
    O.Q6_K: [(4096, 4096), (1024, 4096), (4096, 14336), (5, 512), (33, 768), (34, 768), (35, 1280), (64, 20480),
             (33, 12288), (20000, 256)],
    O.Q8_0: [(4096, 4096), (1024, 4096), (4096, 14336), (7, 64), (9, 800), (64, 20480), (5, 14336),
             (20000, 256)],
    # Q5_K streams like Q4_K (same units, one more 32-byte qh read per unit)
    O.Q5_K: [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336), (17, 256), (64, 20480), (300, 14336),
             (2, 16384), (20000, 256)],
}
CASES = [(t, n, k) for t in TYPES for (n, k) in GEMV_SHAPES[t]]


@pytest.mark.parametrize("t,n,k", CASES)
def test_gemv_matches_reference_cpu_path(torch, okq, orc, t, n, k):
    print(f"[gpu] gemv type={t} N={n} K={k}", flush=True)
    wq = orc.quantize(t, orc.normal(1000 * t + n + k, n * k, 0.02))
    x = orc.normal(7 * k + t, k, 1.0)
    bias = orc.normal(99, n, 0.1)
    got = gpu_linear(torch, okq, t, x, 1, k, wq, n, bias, entry="okq_gemv")
    want = orc.linear_q(t, x, 1, k, wq, n, bias)
    ok, idx, dmax, rmax = O.allclose_ref_rule(got, want, TOL)
    assert ok, f"idx={idx} got={got.reshape(-1)[idx]} want={want.reshape(-1)[idx]} max_abs={dmax}"


def test_q6k_head_gemv_matches_reference(torch, okq, orc):
    """C3: the 128256 x 4096 Q6_K output head at batch 1."""
    n, k = 128256, 4096
    print(f"[gpu] gemv head N={n} K={k}", flush=True)
    wq = orc.quantize(O.Q6_K, orc.normal(314, n * k, 0.02))
    x = orc.normal(315, k, 1.0)
    got = gpu_linear(torch, okq, O.Q6_K, x, 1, k, wq, n)
    want = orc.linear_q(O.Q6_K, x, 1, k, wq, n)
    ok, idx, dmax, _ = O.allclose_ref_rule(got, want, TOL)
    assert ok, f"idx={idx} max_abs={dmax}"


@pytest.mark.parametrize("t", TYPES)
def test_gemv_one_hot_reproduces_dequantized_column_exactly(torch, okq, orc, t):
    n, k = 96, 4096
    wq = orc.quantize(t, orc.normal(50 + t, n * k, 0.02))
    w = orc.dequantize(t, wq, n * k).reshape(n, k)
    for j in (0, 1, 31, 32, 255, 256, 4095):
        x = np.zeros(k, np.float32)
        x[j] = 1.0
        got = gpu_linear(torch, okq, t, x, 1, k, wq, n, entry="okq_gemv")[0]
        assert (got == w[:, j]).all(), (t, j)


@pytest.mark.parametrize("t", TYPES)
def test_gemv_edge_inputs(torch, okq, orc, t):
    n, k = 40, 1024
    wq = orc.quantize(t, orc.normal(60 + t, n * k, 0.02))
    bias = orc.normal(61, n, 1.0)
    # zero activations give exactly the bias
    got = gpu_linear(torch, okq, t, np.zeros(k, np.float32), 1, k, wq, n, bias)
    assert (got[0] == bias).all()
    x = orc.normal(62, k, 1.0)
    y = gpu_linear(torch, okq, t, x, 1, k, wq, n)
    # homogeneity under power-of-two scaling is exact: the activation runs'
    # power-of-two scales absorb the factor, the integer dots are unchanged
    for e in (13, -60):
        ys = gpu_linear(torch, okq, t, (x * np.float32(2.0 ** e)).astype(np.float32), 1, k, wq, n)
        assert (ys == (y * np.float32(2.0 ** e)).astype(np.float32)).all(), e
    # large and tiny magnitudes mixed in one vector (whole runs scaled, so every
    # run stays narrow and takes the two-limb 16-bit quantisation): the error
    # is bounded by |err| <= 2^-14 * sum_k max|x_run(k)| |w_k| (plus f32
    # rounding), not by an absolute 1e-3 -- outputs here are ~1e3 and some are
    # the small difference of sums of ~1e4 (intra-run outliers against the
    # rule itself: test_gpu_activation_domain.py)
    xm = x.copy()
    xm[:256] *= np.float32(1e4)
    xm[256:512] *= np.float32(1e-30)
    got = gpu_linear(torch, okq, t, xm, 1, k, wq, n)[0]
    want = orc.linear_q(t, xm, 1, k, wq, n)[0]
    w = orc.dequantize(t, wq, n * k).reshape(n, k)
    run_max = np.repeat(np.abs(xm).reshape(-1, 32).max(1), 32)
    bound = 2.0 ** -14 * (np.abs(w) * run_max[None, :]).sum(1) + 1e-6 * np.abs(want) + 1e-5
    assert (np.abs(got - want) <= bound).all()
    ok, idx, _, _ = O.allclose_ref_rule(got / 1e4, want / 1e4, TOL)
    assert ok, idx


@pytest.mark.parametrize("t", TYPES)
def test_small_batch_rows_and_determinism(torch, okq, orc, t):
    n, k, rows = 300, 2048, 3
    wq = orc.quantize(t, orc.normal(70 + t, n * k, 0.02))
    x = orc.normal(71, rows * k, 1.0)
    got = gpu_linear(torch, okq, t, x, rows, k, wq, n)
    want = orc.linear_q(t, x, rows, k, wq, n)
    ok, idx, _, _ = O.allclose_ref_rule(got, want, TOL)
    assert ok, idx
    again = gpu_linear(torch, okq, t, x, rows, k, wq, n)
    assert (got.view(np.uint32) == again.view(np.uint32)).all()


MULTIROW_CASES = [
    # (type, rows, n, k): every pass over the weights serves up to four rows
    (O.Q4_K, 2, 4096, 4096), (O.Q4_K, 3, 1024, 4096), (O.Q4_K, 4, 14336, 4096), (O.Q4_K, 4, 4096, 14336),
    (O.Q4_K, 8, 512, 14336), (O.Q4_K, 4, 33, 8192),
    (O.Q6_K, 2, 1024, 4096), (O.Q6_K, 4, 4096, 14336), (O.Q6_K, 7, 300, 12288),
    (O.Q8_0, 3, 4096, 4096), (O.Q8_0, 4, 17, 16384), (O.Q8_0, 5, 300, 96),
    (O.Q5_K, 2, 4096, 4096), (O.Q5_K, 4, 4096, 14336), (O.Q5_K, 3, 20000, 256),
    # dynamic rows in both the batched and the one-row launches
    (O.Q8_0, 2, 20000, 256), (O.Q6_K, 3, 20000, 512),
]


@pytest.mark.parametrize("t,rows,n,k", MULTIROW_CASES)
def test_multirow_gemv_equals_single_rows_bit_for_bit(torch, okq, orc, t, rows, n, k):
    """A launch over R activation rows does each row's arithmetic exactly as a
    one-row launch (same per-lane contraction, same reduction order), so the
    batched GEMV must equal row-by-row GEMVs bit for bit, and the reference
    CPU path within the rule."""
    print(f"[gpu] multirow gemv type={t} rows={rows} N={n} K={k}", flush=True)
    wq = orc.quantize(t, orc.normal(5000 + t + k, n * k, 0.02))
    bias = orc.normal(5001, n, 0.1)
    x = orc.normal(5002 + rows, rows * k, 1.0)
    got = gpu_linear(torch, okq, t, x, rows, k, wq, n, bias, entry="okq_gemv")
    for r in range(rows):
        one = gpu_linear(torch, okq, t, x[r * k:(r + 1) * k], 1, k, wq, n, bias, entry="okq_gemv")
        assert _same_bits(got[r], one[0]).all(), f"row {r}"
    want = orc.linear_q(t, x, rows, k, wq, n, bias)
    ok, idx, dmax, _ = O.allclose_ref_rule(got, want, TOL)
    assert ok, f"idx={idx} max_abs={dmax}"


def test_empty_inputs_are_noops(torch, okq):
    out = torch.full((4,), 7.0, device="cuda")
    okq.call("okq_linear_out_by_in_q", None, 0, 256, O.Q4_K, None, 144 * 4, 4, None, out.data_ptr(), None)
    torch.cuda.synchronize()
    assert (_host(out) == 7.0).all()


def test_python_mirror_linear_d_and_host_slices(torch, orc):
    from ocelotl_amd.backend import HipKernelBackend, GgmlTensorType, KernelError
    be = HipKernelBackend(0)
    assert be.name() == "hip-gfx950" and be.context().device.kind == "gpu"
    n, k = 128, 512
    wq = orc.quantize(O.Q4_K, orc.normal(80, n * k, 0.02))
    w = be.upload_quantized(GgmlTensorType.Q4K, k, n, wq)
    x = orc.normal(81, 2 * k)
    b = orc.normal(82, n)
    out = np.zeros(2 * n, np.float32)
    be.linear_out_by_in(x, 2, k, w, n, b, out)
    ok, idx, _, _ = O.allclose_ref_rule(out, orc.linear_q(O.Q4_K, x, 2, k, wq, n, b), TOL)
    assert ok, idx
    deq = be.dequantize(w).to_host_owned()
    assert (deq.view(np.uint32) == orc.dequantize(O.Q4_K, wq, n * k).view(np.uint32)).all()
    with pytest.raises(KernelError):
        be.linear_d(be.upload(x), 2, k, w, n, None, be.alloc(2 * n - 1))


@pytest.mark.parametrize("t,rows,n,k", [(O.Q6_K, 1, 1024, 4096), (O.Q6_K, 6, 300, 1024), (O.Q8_0, 1, 1024, 4096),
                                        (O.Q8_0, 5, 130, 800)])
def test_bf16_activations_on_the_gemv_path(torch, okq, orc, t, rows, n, k):
    """okq_linear_out_by_in_q_bf16 for formats without an MFMA path: the bf16
    activations are widened to f32 on the device (exactly, as
    safetensors_values.rs:115-123) and run through the GEMV."""
    print(f"[gpu] bf16 linear type={t} rows={rows} N={n} K={k}", flush=True)
    wq = orc.quantize(t, orc.normal(2000 + t + n, n * k, 0.02))
    xb = orc.f32_to_bf16(orc.normal(2001 + rows, rows * k, 1.0))
    x32 = orc.bf16_to_f32(xb)
    bias = orc.normal(2002, n, 0.1)
    xd = _dev(torch, xb.view(np.int16))
    wd = _dev(torch, wq)
    bd = _dev(torch, bias)
    out = torch.full((rows * n,), float("nan"), dtype=torch.float32, device="cuda")
    okq.call("okq_linear_out_by_in_q_bf16", xd.data_ptr(), rows, k, t, wd.data_ptr(), wq.size, n, bd.data_ptr(),
             out.data_ptr(), _stream(torch))
    torch.cuda.synchronize()
    got = _host(out).reshape(rows, n)
    # same result as the f32 entry point on the decoded activations, bit for bit
    ref32 = gpu_linear(torch, okq, t, x32, rows, k, wq, n, bias)
    assert _same_bits(got, ref32).all()
    want = orc.linear_q(t, x32, rows, k, wq, n, bias)
    ok, idx, dmax, _ = O.allclose_ref_rule(got, want, TOL)
    assert ok, f"idx={idx} got={got.reshape(-1)[idx]} want={want.reshape(-1)[idx]} max_abs={dmax}"


@pytest.mark.parametrize("t", TYPES)
def test_gemv_run_max_at_the_limb_boundary(torch, okq, orc, t):
    """Every activation run's maximum has mantissa 255/256 (1.9921875 * 2^j,
    exactly representable in bf16): the run's integer scale must leave the
    high int8 limb in range (q + 128) >> 8 <= 127, here and at the largest
    mantissa below 255/256."""
    n, k = 96, 1024
    wq = orc.quantize(t, orc.normal(3000 + t, n * k, 0.02))
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(k) * 0.3).astype(np.float32)
    run = 16 if t == O.Q6_K else 32
    edge = np.float32(1.9921875)
    below = np.nextafter(np.float32(0.99), np.float32(1)) * np.float32(2.0)
    for r in range(k // run):
        scale = np.float32(2.0 ** (r % 7 - 3))
        sign = np.float32(-1.0 if r % 2 else 1.0)
        x[r * run + (r % run)] = sign * (edge if r % 3 else below) * scale
    got = gpu_linear(torch, okq, t, x, 1, k, wq, n, entry="okq_gemv")
    want = orc.linear_q(t, x, 1, k, wq, n, None)
    ok, idx, dmax, _ = O.allclose_ref_rule(got, want, TOL)
    assert ok, f"idx={idx} got={got.reshape(-1)[idx]} want={want.reshape(-1)[idx]} max_abs={dmax}"


MULTI_CASES = [
    (O.Q4_K, 1, 4096, [4096, 1024, 1024]),   # q/k/v of a Llama-3-8B layer
    (O.Q4_K, 1, 4096, [14336, 14336]),       # gate/up: dynamic rows, the single launches are static
    (O.Q4_K, 3, 14336, [300, 17]),           # K > 4096: teams of waves
    (O.Q6_K, 2, 1024, [33, 300, 5, 64]),
    (O.Q8_0, 1, 4096, [1024, 4096]),
    (O.Q5_K, 1, 4096, [14336, 14336]),
    (O.Q5_K, 2, 14336, [300, 17, 64]),
]


@pytest.mark.parametrize("t,rows,k,ns", MULTI_CASES)
def test_gemv_multi_equals_single_gemvs_bit_for_bit(torch, okq, orc, t, rows, k, ns):
    """okq_gemv_multi streams several matrices sharing x in one launch; every
    output must equal okq_gemv on its matrix alone, bit for bit, and the
    reference CPU path within the rule."""
    import ctypes
    print(f"[gpu] gemv_multi type={t} rows={rows} K={k} N={ns}", flush=True)
    wqs = [orc.quantize(t, orc.normal(4000 + 17 * i + t, n * k, 0.02)) for i, n in enumerate(ns)]
    biases = [orc.normal(4100 + i, n, 0.1) if i % 2 == 0 else None for i, n in enumerate(ns)]
    x = orc.normal(4200 + rows, rows * k, 1.0)
    xd = _dev(torch, x)
    wds = [_dev(torch, wq) for wq in wqs]
    bds = [None if b is None else _dev(torch, b) for b in biases]
    outs = [torch.full((rows * n,), float("nan"), dtype=torch.float32, device="cuda") for n in ns]
    c = len(ns)
    arr = lambda ty, vals: (ty * c)(*vals)
    okq.call("okq_gemv_multi", xd.data_ptr(), rows, k, t, c,
             arr(ctypes.c_void_p, [w.data_ptr() for w in wds]),
             arr(ctypes.c_uint64, [wq.size for wq in wqs]),
             arr(ctypes.c_int64, ns),
             arr(ctypes.c_void_p, [None if b is None else b.data_ptr() for b in bds]),
             arr(ctypes.c_void_p, [o.data_ptr() for o in outs]), _stream(torch))
    torch.cuda.synchronize()
    for i, n in enumerate(ns):
        got = _host(outs[i]).reshape(rows, n)
        single = gpu_linear(torch, okq, t, x, rows, k, wqs[i], n, biases[i], entry="okq_gemv")
        assert _same_bits(got, single).all(), f"matrix {i}"
        want = orc.linear_q(t, x, rows, k, wqs[i], n, biases[i])
        ok, idx, dmax, _ = O.allclose_ref_rule(got, want, TOL)
        assert ok, f"matrix {i} idx={idx} max_abs={dmax}"


MULTI_BATCH_CASES = [
    # (type, rows, K, out_features, the MFMA matrices share one decode-batch launch)
    (O.Q4_K, 8, 4096, [14336, 14336], True),         # gate/up at 8 rows
    (O.Q4_K, 8, 4096, [4096, 1024, 14336], True),    # q, k (2.4 MB) and the large one share a decode-batch launch
    (O.Q4_K, 8, 4096, [1024, 512, 14336], True),     # 512 x 4096 (1.2 MB) on the GEMV, the other two share
    (O.Q4_K, 8, 4096, [256, 512, 14336], False),     # two under 2 MB on the GEMV, the large one alone
    (O.Q4_K, 5, 4096, [4096, 1024, 14336], True),    # 5 rows: k on the GEMV, q and the large one share
    (O.Q6_K, 24, 1024, [33, 300], True),             # above 8 rows: every Q6_K matrix on the MFMA path
    (O.Q4_K, 32, 1024, [17, 1000, 256, 40], True),   # four matrices, ragged tiles, two 16-row groups
    (O.Q8_0, 12, 1024, [100, 64], True),             # Q8_0 above 8 rows: the MFMA kernels too
    (O.Q4_K, 40, 1024, [300, 200], False),           # above 32 rows: each on the tiled GEMM
    (O.Q5_K, 8, 4096, [14336, 14336], True),         # a Q5_K gate/up pair at 8 rows
    (O.Q5_K, 24, 1024, [33, 300, 17], True),         # Q5_K above 8 rows: one decode-batch launch
]


@pytest.mark.parametrize("t,rows,k,ns,shared", MULTI_BATCH_CASES)
def test_gemv_multi_batches_route_like_the_linear_dispatch(torch, okq, orc, t, rows, k, ns, shared):
    """At decode-batch row counts okq_gemv_multi sends every matrix to the
    kernels okq_linear_out_by_in_q would pick for it: outputs equal that entry
    point's, matrix by matrix, bit for bit -- except where several matrices
    share one decode-batch launch (its K split follows the combined columns),
    which must match within the rule -- and the reference within the rule."""
    import ctypes
    print(f"[gpu] gemv_multi batch type={t} rows={rows} K={k} N={ns}", flush=True)
    wqs = [orc.quantize(t, orc.normal(4300 + 17 * i + t, n * k, 0.02)) for i, n in enumerate(ns)]
    biases = [orc.normal(4400 + i, n, 0.1) if i % 2 == 1 else None for i, n in enumerate(ns)]
    x = orc.normal(4500 + rows, rows * k, 1.0)
    xd = _dev(torch, x)
    wds = [_dev(torch, wq) for wq in wqs]
    bds = [None if b is None else _dev(torch, b) for b in biases]
    outs = [torch.full((rows * n,), float("nan"), dtype=torch.float32, device="cuda") for n in ns]
    c = len(ns)
    arr = lambda ty, vals: (ty * c)(*vals)
    okq.call("okq_gemv_multi", xd.data_ptr(), rows, k, t, c,
             arr(ctypes.c_void_p, [w.data_ptr() for w in wds]),
             arr(ctypes.c_uint64, [wq.size for wq in wqs]),
             arr(ctypes.c_int64, ns),
             arr(ctypes.c_void_p, [None if b is None else b.data_ptr() for b in bds]),
             arr(ctypes.c_void_p, [o.data_ptr() for o in outs]), _stream(torch))
    torch.cuda.synchronize()
    for i, n in enumerate(ns):
        got = _host(outs[i]).reshape(rows, n)
        single = gpu_linear(torch, okq, t, x, rows, k, wqs[i], n, biases[i])
        if shared:
            ok, idx, dmax, _ = O.allclose_ref_rule(got, single, TOL)
            assert ok, f"matrix {i} vs its own call: idx={idx} max_abs={dmax}"
        else:
            assert _same_bits(got, single).all(), f"matrix {i}"
        want = orc.linear_q(t, x, rows, k, wqs[i], n, biases[i])
        ok, idx, dmax, _ = O.allclose_ref_rule(got, want, TOL)
        assert ok, f"matrix {i} idx={idx} max_abs={dmax}"


def test_gemv_multi_validates_every_matrix_before_launch(torch, okq, orc):
    import ctypes
    k, ns = 256, [8, 8]
    wq = orc.quantize(O.Q4_K, orc.normal(4300, 8 * k, 0.02))
    wd = _dev(torch, wq)
    xd = _dev(torch, orc.normal(4301, k, 1.0))
    o0 = torch.full((8,), 7.0, device="cuda")
    o1 = torch.full((8,), 7.0, device="cuda")
    ptrs = (ctypes.c_void_p * 2)(wd.data_ptr(), wd.data_ptr())
    nn = (ctypes.c_int64 * 2)(*ns)
    outs = (ctypes.c_void_p * 2)(o0.data_ptr(), o1.data_ptr())
    with pytest.raises(okq.OkqStatusError) as e:
        okq.call("okq_gemv_multi", xd.data_ptr(), 1, k, O.Q4_K, 2, ptrs, (ctypes.c_uint64 * 2)(wq.size, wq.size - 1),
                 nn, None, outs, _stream(torch))
    assert e.value.status == okq.E_SHAPE and "matrix 1" in e.value.message
    with pytest.raises(okq.OkqStatusError) as e:
        okq.call("okq_gemv_multi", xd.data_ptr(), 1, k, O.Q4_K, 5, ptrs, (ctypes.c_uint64 * 2)(wq.size, wq.size),
                 nn, None, outs, _stream(torch))
    assert e.value.status == okq.E_ARG
    torch.cuda.synchronize()
    assert (o0.cpu().numpy() == 7.0).all() and (o1.cpu().numpy() == 7.0).all()
