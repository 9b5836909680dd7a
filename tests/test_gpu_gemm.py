"""GPU parity of the MFMA dequant-GEMM (prefill) against the CPU oracle.

Bar: the reference rule abs <= 1e-3 || rel <= 1e-3 per element against the
reference CPU path (oracle restatement of linear_out_by_in on the dequantized
weights, crates/kernels/src/lib.rs:1974-2123) on the same inputs; bf16
activations are decoded exactly for the CPU path (safetensors_values.rs:
115-123).  Exact for the one-hot column probe.  Large M are checked on a
sample of rows (rows are independent outputs).
"""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-3


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


def run(torch, okq, entry, t, x, rows, k, wq, n, bias=None):
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    wd = torch.from_numpy(wq).cuda()
    bd = None if bias is None else torch.from_numpy(np.asarray(bias, np.float32)).cuda()
    out = torch.full((rows * n,), float("nan"), dtype=torch.float32, device="cuda")
    okq.call(entry, xd.data_ptr(), rows, k, t, wd.data_ptr(), wq.size, n, None if bd is None else bd.data_ptr(),
             out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return out.cpu().numpy().reshape(rows, n)


def bf16_inputs(orc, seed, rows, k):
    xf = orc.normal(seed, rows * k, 1.0)
    xb = orc.f32_to_bf16(xf)
    return xb, orc.bf16_to_f32(xb)


def check_rows(orc, t, got, x32, rows, k, wq, n, bias, sample):
    idx = np.arange(rows) if sample is None else np.unique(np.r_[np.arange(min(sample, rows)),
                                                                  np.arange(max(0, rows - sample), rows)])
    want = orc.linear_q(t, x32.reshape(rows, k)[idx].reshape(-1), idx.size, k, wq, n, bias, O.MODE_SCALAR, 16)
    ok, i, dmax, _ = O.allclose_ref_rule(got[idx], want, TOL)
    assert ok, f"row {idx[i // n]} col {i % n}: got {got[idx].reshape(-1)[i]} want {want.reshape(-1)[i]} max_abs {dmax}"


GEMM_CASES = [
    # (rows, n, k)
    (5, 96, 256), (33, 130, 512), (128, 256, 1024), (130, 300, 2048), (200, 1000, 768),
    (128, 4096, 4096), (128, 1024, 4096), (128, 14336, 4096), (128, 4096, 14336),
]


@pytest.mark.parametrize("rows,n,k", GEMM_CASES)
def test_gemm_bf16_q4k_matches_reference(torch, okq, orc, rows, n, k):
    print(f"[gpu] gemm bf16 Q4_K M={rows} N={n} K={k}", flush=True)
    wq = orc.quantize(O.Q4_K, orc.normal(500 + n + k, n * k, 0.02))
    xb, x32 = bf16_inputs(orc, 600 + rows, rows, k)
    bias = orc.normal(601, n, 0.1)
    got = run(torch, okq, "okq_gemm_bf16", O.Q4_K, xb, rows, k, wq, n, bias)
    check_rows(orc, O.Q4_K, got, x32, rows, k, wq, n, bias, None)


@pytest.mark.parametrize("rows,n,k", [(512, 4096, 4096), (512, 14336, 4096), (512, 4096, 14336), (2048, 1024, 4096)])
def test_gemm_bf16_q4k_c4_shapes_sampled_rows(torch, okq, orc, rows, n, k):
    print(f"[gpu] gemm bf16 Q4_K M={rows} N={n} K={k} (sampled rows)", flush=True)
    wq = orc.quantize(O.Q4_K, orc.normal(700 + n + k, n * k, 0.02))
    xb, x32 = bf16_inputs(orc, 800 + rows, rows, k)
    got = run(torch, okq, "okq_gemm_bf16", O.Q4_K, xb, rows, k, wq, n)
    assert np.isfinite(got).all()
    check_rows(orc, O.Q4_K, got, x32, rows, k, wq, n, None, 24)


@pytest.mark.parametrize("rows,n,k", [(4, 64, 256), (8, 64, 256), (12, 300, 1024), (32, 520, 1024),
                                      (64, 4096, 4096)])
def test_gemm_f32_q4k_matches_reference(torch, okq, orc, rows, n, k):
    wq = orc.quantize(O.Q4_K, orc.normal(900 + n, n * k, 0.02))
    x = orc.normal(901 + rows, rows * k, 1.0)
    got = run(torch, okq, "okq_gemm", O.Q4_K, x, rows, k, wq, n)
    check_rows(orc, O.Q4_K, got, x, rows, k, wq, n, None, None)
    # the automatic path picks the MFMA path above 8 rows (the GEMV up to 8
    # for matrices this small) and agrees with the pinned path bit for bit
    auto = run(torch, okq, "okq_linear_out_by_in_q", O.Q4_K, x, rows, k, wq, n)
    pinned = got if rows > 8 else run(torch, okq, "okq_gemv", O.Q4_K, x, rows, k, wq, n)
    assert (auto.view(np.uint32) == pinned.view(np.uint32)).all()


def test_gemm_one_hot_columns_are_exact(torch, okq, orc):
    n, k = 160, 1024
    wq = orc.quantize(O.Q4_K, orc.normal(77, n * k, 0.02))
    w = orc.dequantize(O.Q4_K, wq, n * k).reshape(n, k)
    cols = np.array([0, 1, 31, 32, 255, 256, 700, 1023])
    x = np.zeros((cols.size, k), np.float32)
    x[np.arange(cols.size), cols] = 1.0
    got = run(torch, okq, "okq_gemm_bf16", O.Q4_K, orc.f32_to_bf16(x.reshape(-1)), cols.size, k, wq, n)
    assert (got == w[:, cols].T).all()
    got32 = run(torch, okq, "okq_gemm", O.Q4_K, x.reshape(-1), cols.size, k, wq, n)
    assert (got32 == w[:, cols].T).all()


def test_gemm_is_deterministic_and_row_independent(torch, okq, orc):
    """Same inputs, same bits; and a row's result does not depend on the
    other rows of its batch within a kernel family: the tiled kernel (more
    than 32 rows) and the decode-batch kernel (up to 32 rows) each sum a
    row's products in one fixed order (the two families' orders differ, so
    across the boundary results agree within the rule only)."""
    rows, n, k = 300, 384, 2048
    wq = orc.quantize(O.Q4_K, orc.normal(88, n * k, 0.02))
    xb, x32 = bf16_inputs(orc, 89, rows, k)
    a = run(torch, okq, "okq_gemm_bf16", O.Q4_K, xb, rows, k, wq, n)
    b = run(torch, okq, "okq_gemm_bf16", O.Q4_K, xb, rows, k, wq, n)
    assert (a.view(np.uint32) == b.view(np.uint32)).all()
    # tiled: rows 100..163 on their own equal the same rows of the big batch
    sub = run(torch, okq, "okq_gemm_bf16", O.Q4_K, xb.reshape(rows, k)[100:164].reshape(-1), 64, k, wq, n)
    assert (sub.view(np.uint32) == a[100:164].view(np.uint32)).all()
    # decode-batch kernel: a row alone equals the same row among 12
    few = run(torch, okq, "okq_gemm_bf16", O.Q4_K, xb.reshape(rows, k)[130:142].reshape(-1), 12, k, wq, n)
    one = run(torch, okq, "okq_gemm_bf16", O.Q4_K, xb.reshape(rows, k)[137:138].reshape(-1), 1, k, wq, n)
    assert (one[0].view(np.uint32) == few[7].view(np.uint32)).all()
    check_rows(orc, O.Q4_K, few, x32.reshape(rows, k)[130:142].reshape(-1), 12, k, wq, n, None, None)


# ---- decode batches (up to 32 rows: one or two 16-row MFMA tiles, weights
# dequantised into B fragments by the lanes that load them) ---------------------
DEC_CASES = [
    # (entry, rows, n, k): ragged N, every row count class, split and unsplit K
    ("okq_gemm", 1, 96, 256), ("okq_gemm", 2, 17, 512), ("okq_gemm", 5, 300, 1024),
    ("okq_gemm", 8, 4096, 4096), ("okq_gemm", 16, 1000, 768), ("okq_gemm", 13, 4096, 14336),
    # K unsplit across workgroups, 8 waves share each tile (2 tiles per workgroup)
    ("okq_gemm", 6, 8000, 4096),
    ("okq_gemm_bf16", 3, 14336, 4096), ("okq_gemm_bf16", 16, 520, 2048), ("okq_gemm_bf16", 7, 33, 256),
    # one super-block per row: K is never split, outputs and bias written directly
    ("okq_gemm", 3, 70001, 256), ("okq_gemm_bf16", 9, 65540, 256),
    # more column tiles than 256 CUs x 16 waves x 4 staged biases: more column groups keep every wave
    # within its staged bias tiles
    ("okq_gemm", 8, 270000, 256),
    # 17-32 rows: two 16-row MFMA groups share each B fragment
    ("okq_gemm", 17, 300, 1024), ("okq_gemm", 32, 4096, 4096), ("okq_gemm_bf16", 25, 1000, 768),
    ("okq_gemm", 32, 14336, 4096),
    # column groups x the LDS-bound K split exceed one round of 256 CUs: the
    # plan takes fewer column groups and waves take several tiles (ragged)
    ("okq_gemm", 32, 28672, 4096), ("okq_gemm_bf16", 32, 30000, 4096),
    # one real row in the second 16-row group, a single column, a few columns
    # at 32 rows, one super-block per row with more tiles than the staged
    # biases, and column blocks that do not divide evenly among the groups
    ("okq_gemm", 17, 1, 256), ("okq_gemm", 32, 5, 512), ("okq_gemm_bf16", 32, 70000, 256),
    ("okq_gemm", 29, 33000, 1024),
    # more than 16 K slices (32 rows stage 4 super-blocks a slice: 32 and 64
    # slices): the split-K reduction loads its slices in several batches of 16
    ("okq_gemm", 32, 300, 32768), ("okq_gemm_bf16", 32, 300, 65536),
]


DEC_Q6K_CASES = [
    ("okq_gemm", 1, 96, 256), ("okq_gemm", 4, 257, 768), ("okq_gemm", 8, 4096, 4096), ("okq_gemm", 16, 1024, 4096),
    ("okq_gemm", 11, 4096, 14336), ("okq_gemm_bf16", 6, 300, 1024), ("okq_gemm_bf16", 16, 4095, 512),
    # an odd super-block count per row: block starts alternate between the two 2-byte alignments.
    # Tensors of an odd block count (257 x 3, 333 x 5, 70003, 257 x 3 at 31 rows) end on a block
    # that starts on a dword and read d with a 2-byte load; the rest take it from the scale window.
    ("okq_gemm", 5, 333, 1280), ("okq_gemm", 2, 70003, 256),
    ("okq_gemm", 20, 1024, 4096), ("okq_gemm", 32, 4096, 14336), ("okq_gemm_bf16", 31, 257, 768),
    # more column groups x K slices than one round of CUs (waves take 1-2 tiles)
    ("okq_gemm", 24, 20000, 4096),
]


@pytest.mark.parametrize("entry,rows,n,k", DEC_CASES)
def test_gemm_decode_batch_q4k_matches_reference(torch, okq, orc, entry, rows, n, k):
    print(f"[gpu] gemm decode-batch {entry} Q4_K M={rows} N={n} K={k}", flush=True)
    wq = orc.quantize(O.Q4_K, orc.normal(1500 + n + k, n * k, 0.02))
    bias = orc.normal(1501 + rows, n, 0.1)
    if entry == "okq_gemm_bf16":
        xin, x32 = bf16_inputs(orc, 1502 + rows, rows, k)
    else:
        xin = x32 = orc.normal(1502 + rows, rows * k, 1.0)
    got = run(torch, okq, entry, O.Q4_K, xin, rows, k, wq, n, bias)
    assert np.isfinite(got).all()
    check_rows(orc, O.Q4_K, got, x32, rows, k, wq, n, bias, None if n * k <= 20_000_000 else 6)


@pytest.mark.parametrize("entry,rows,n,k", DEC_Q6K_CASES)
def test_gemm_decode_batch_q6k_matches_reference(torch, okq, orc, entry, rows, n, k):
    print(f"[gpu] gemm decode-batch {entry} Q6_K M={rows} N={n} K={k}", flush=True)
    wq = orc.quantize(O.Q6_K, orc.normal(1600 + n + k, n * k, 0.02))
    bias = orc.normal(1601 + rows, n, 0.1)
    if entry == "okq_gemm_bf16":
        xin, x32 = bf16_inputs(orc, 1602 + rows, rows, k)
    else:
        xin = x32 = orc.normal(1602 + rows, rows * k, 1.0)
    got = run(torch, okq, entry, O.Q6_K, xin, rows, k, wq, n, bias)
    assert np.isfinite(got).all()
    check_rows(orc, O.Q6_K, got, x32, rows, k, wq, n, bias, None if n * k <= 20_000_000 else 6)


def test_gemm_decode_batch_split_k_repeat(torch, okq, orc):
    """The decode-batch kernel either splits K across workgroups (partials in
    the stream's workspace, summed in slice order by the reduction) or, when the
    whole K fits one workgroup, splits it among the waves that share a tile
    (summed through LDS in wave order).  Many back-to-back launches on one
    stream, alternating between problems of both kinds and different column
    group and slice counts, must each give the same bits as the first launch
    of that problem, and match the reference."""
    cases = [(O.Q4_K, 8, 14336, 4096), (O.Q6_K, 5, 4096, 14336), (O.Q4_K, 24, 1000, 2048), (O.Q6_K, 2, 333, 1280)]
    stream = torch.cuda.current_stream().cuda_stream
    prepared = []
    for i, (t, rows, n, k) in enumerate(cases):
        print(f"[gpu] gemm decode-batch split-K repeat type={t} M={rows} N={n} K={k}", flush=True)
        wq = orc.quantize(t, orc.normal(1700 + i, n * k, 0.02))
        x = orc.normal(1710 + i, rows * k, 1.0)
        bias = orc.normal(1720 + i, n, 0.1)
        dev = [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (x, wq, bias)]
        prepared.append((t, rows, n, k, wq, x, bias, dev))
    outs = [[] for _ in cases]
    for rep in range(12):
        for i, (t, rows, n, k, wq, x, bias, (xd, wd, bd)) in enumerate(prepared):
            out = torch.full((rows * n,), float("nan"), dtype=torch.float32, device="cuda")
            okq.call("okq_gemm", xd.data_ptr(), rows, k, t, wd.data_ptr(), wq.size, n, bd.data_ptr(), out.data_ptr(),
                     stream)
            outs[i].append(out)
    torch.cuda.synchronize()
    for i, (t, rows, n, k, wq, x, bias, _) in enumerate(prepared):
        first = outs[i][0].cpu().numpy()
        for o in outs[i][1:]:
            assert (o.cpu().numpy().view(np.uint32) == first.view(np.uint32)).all()
        check_rows(orc, t, first.reshape(rows, n), x, rows, k, wq, n, bias, 4)


def q4k_parts(orc, wq, n, k):
    """|d*sc*q| and |dmin*m| per weight: dequantizing with every 4-bit quant
    zeroed leaves exactly -dmin*m (Q4_K qs are bytes 16..143 of a block)."""
    w = orc.dequantize(O.Q4_K, wq, n * k).reshape(n, k)
    z = wq.reshape(-1, 144).copy()
    z[:, 16:] = 0
    w0 = orc.dequantize(O.Q4_K, z.reshape(-1), n * k).reshape(n, k)
    return np.abs(w.astype(np.float64) - w0), np.abs(w0.astype(np.float64))


def test_gemm_wide_dynamic_range_rows(torch, okq, orc):
    """Activations far outside fp16's range: the pre-pass's per-row
    power-of-two scale keeps every operand finite.
      rows 0-2: N(0,1) plus outlier channels (a 32-run of 3000 summing to
                96000 > 65504, -2500 every 7th channel, a single 60000);
      rows 3-4: row 0 times 2^40 and 2^-60 -- outputs must equal row 0's times
                the same power of two, bit for bit (the scale is undone
                exactly);
      row 5:    zeros -> exactly zero;
      row 6:    N(0,1) times 1e6.
    Outliers make outputs the small difference of large sums, where any f32
    evaluation order (the reference's included) rounds at the scale of the
    sums; the GEMM contracts x with d*sc*q and with dmin*m separately, so rows
    0-2 and 6 are held to 1e-3 |want| + 2^-20 sum_k |x_k| (|d sc q_k| +
    |dmin m_k|) -- far below what a wrong term, index or scale produces."""
    rows, n, k = 7, 256, 1024
    wq = orc.quantize(O.Q4_K, orc.normal(91, n * k, 0.02))
    pa, pb = q4k_parts(orc, wq, n, k)
    x = orc.normal(92, rows * k, 1.0).reshape(rows, k)
    x[0, 64:96] = 3000.0
    x[1, ::7] = -2500.0
    x[2, 5] = 60000.0
    x[3] = x[0] * np.float32(2.0 ** 40)
    x[4] = x[0] * np.float32(2.0 ** -60)
    x[5] = 0.0
    x[6] *= np.float32(1e6)
    for entry, xin in (("okq_gemm_bf16", "bf16"), ("okq_gemm", "f32")):
        if xin == "bf16":
            xb = orc.f32_to_bf16(x.reshape(-1))
            x32 = orc.bf16_to_f32(xb).reshape(rows, k)
            got = run(torch, okq, entry, O.Q4_K, xb, rows, k, wq, n)
        else:
            x32 = x
            got = run(torch, okq, entry, O.Q4_K, x.reshape(-1), rows, k, wq, n)
        assert np.isfinite(got).all(), entry
        want = orc.linear_q(O.Q4_K, x32.reshape(-1), rows, k, wq, n, None, O.MODE_SCALAR, 1)
        for r in (0, 1, 2, 6):
            ax = np.abs(x32[r].astype(np.float64))
            bound = 1e-3 * np.abs(want[r]) + 2.0 ** -20 * (pa @ ax + pb @ ax)
            err = np.abs(got[r].astype(np.float64) - want[r])
            assert (err <= bound).all(), (entry, r, float((err / bound).max()))
        assert (got[3] == got[0] * np.float32(2.0 ** 40)).all(), entry
        assert (got[4] == got[0] * np.float32(2.0 ** -60)).all(), entry
        assert (got[5] == 0.0).all(), entry


def test_gemm_decode_batch_per_slice_scaling(torch, okq, orc):
    """The decode-batch kernel scales each 256-wide super-block of a row by its
    own power of two (and splits K 56 ways here).  Checked: halves 2^60 apart
    in one row, rows with all-zero super-blocks, exact power-of-two
    homogeneity, and non-finite activations -- an inf or a NaN makes its own
    row non-finite and leaves every other row bit-identical to a batch
    without it."""
    rows, n, k = 6, 1000, 14336  # K split across workgroups (a 4096-long row fits one workgroup's LDS)
    wq = orc.quantize(O.Q4_K, orc.normal(95, n * k, 0.02))
    pa, pb = q4k_parts(orc, wq, n, k)
    x = orc.normal(96, rows * k, 1.0).reshape(rows, k)
    x[1, : k // 2] *= np.float32(2.0 ** 30)
    x[1, k // 2:] *= np.float32(2.0 ** -30)
    for sl in range(0, k, 512):  # every other 256-wide slice of row 2 is zero
        x[2, sl:sl + 256] = 0.0
    x[5] = x[0] * np.float32(2.0 ** -100)
    clean = x.copy()
    x[3] = x[0]
    x[3, 100] = np.inf
    x[4] = x[0]
    x[4, 3000] = np.nan
    clean[3] = x[0]
    clean[4] = x[0]
    got = run(torch, okq, "okq_gemm", O.Q4_K, x.reshape(-1), rows, k, wq, n)
    ref = run(torch, okq, "okq_gemm", O.Q4_K, clean.reshape(-1), rows, k, wq, n)
    want = orc.linear_q(O.Q4_K, clean.reshape(-1), rows, k, wq, n, None, O.MODE_SCALAR, 1)
    for r in (0, 1, 2):
        ax = np.abs(clean[r].astype(np.float64))
        bound = 1e-3 * np.abs(want[r]) + 2.0 ** -20 * (pa @ ax + pb @ ax)
        err = np.abs(got[r].astype(np.float64) - want[r])
        assert (err <= bound).all(), (r, float((err / bound).max()))
    assert (got[5] == got[0] * np.float32(2.0 ** -100)).all()
    assert not np.isfinite(got[3]).any() and np.isnan(got[4]).all()
    for r in (0, 1, 2, 5):
        assert (got[r].view(np.uint32) == ref[r].view(np.uint32)).all(), r


# ---- Q6_K -----------------------------------------------------------------------
# B = sc * (q - 32) (|.| <= 4096) enters as two exact fp16 planes, fp16(v) and
# the remainder v - fp16(v) in {-1, 0, 1}: the products are exact as for Q4_K.

Q6K_CASES = [
    # (entry, rows, n, k)
    ("okq_gemm_bf16", 9, 96, 256), ("okq_gemm_bf16", 33, 300, 1024), ("okq_gemm_bf16", 130, 1024, 4096),
    ("okq_gemm_bf16", 128, 4096, 14336), ("okq_gemm", 32, 1024, 4096), ("okq_gemm", 32, 4096, 14336),
    ("okq_gemm", 100, 257, 768), ("okq_gemm", 5, 64, 512),
    # the last super-block of the last row ends 2 bytes past a dword (257 rows x 630 bytes)
    ("okq_gemm_bf16", 100, 257, 768), ("okq_gemm", 32, 257, 768),
]


@pytest.mark.parametrize("entry,rows,n,k", Q6K_CASES)
def test_gemm_q6k_matches_reference(torch, okq, orc, entry, rows, n, k):
    print(f"[gpu] gemm {entry} Q6_K M={rows} N={n} K={k}", flush=True)
    wq = orc.quantize(O.Q6_K, orc.normal(900 + n + k, n * k, 0.02))
    bias = orc.normal(901, n, 0.1)
    if entry == "okq_gemm_bf16":
        x, x32 = bf16_inputs(orc, 902 + rows, rows, k)
    else:
        x = x32 = orc.normal(903 + rows, rows * k, 1.0)
    got = run(torch, okq, entry, O.Q6_K, x, rows, k, wq, n, bias)
    check_rows(orc, O.Q6_K, got, x32, rows, k, wq, n, bias, None if rows <= 130 else 16)


def test_gemm_q6k_one_hot_columns_are_exact(torch, okq, orc):
    """x = e_j picks column j of every weight row: the GEMM returns d * (hi +
    lo) with hi + lo = sc * (q - 32) exactly, the dequantized value bit for
    bit (scales up to |sc| = 128 included)."""
    rows, n, k = 16, 64, 512
    wq = orc.quantize(O.Q6_K, orc.normal(910, n * k, 0.02))
    w = orc.dequantize(O.Q6_K, wq, n * k).reshape(n, k)
    blocks = np.frombuffer(wq.tobytes(), np.uint8).reshape(n, k // 256, 210)
    assert np.abs(blocks[:, :, 192:208].view(np.int8).astype(int)).max() > 64  # products above 2048 occur
    x = np.zeros((rows, k), np.float32)
    cols = np.arange(rows) * 31 % k
    x[np.arange(rows), cols] = 1.0
    for entry, xin in (("okq_gemm", x.reshape(-1)), ("okq_gemm_bf16", orc.f32_to_bf16(x.reshape(-1)))):
        got = run(torch, okq, entry, O.Q6_K, xin, rows, k, wq, n)
        # values, not bits: a zero product with a negative scale dequantizes to -0.0
        assert np.array_equal(got, w[:, cols].T), entry


# bf16 grids whose 128 x 256 tiles fill the CUs take gemm_wide_q6k_kernel (the
# weights as the same two exact planes, dequantised in registers): the C4
# down shape, ragged M and N split and unsplit, and rows of 630 / 1050 bytes
# (2-byte aligned super-blocks).
Q6K_WIDE_CASES = [(512, 4096, 14336), (500, 3900, 4096), (2048, 3000, 768), (1000, 3900, 1280)]


@pytest.mark.parametrize("rows,n,k", Q6K_WIDE_CASES)
def test_gemm_q6k_bf16_wide_rows_of_every_m_tile(torch, okq, orc, rows, n, k):
    print(f"[gpu] gemm Q6_K bf16 M={rows} N={n} K={k} (rows of every tile)", flush=True)
    wq = orc.quantize(O.Q6_K, orc.normal(960 + n + k, n * k, 0.02))
    xb, x32 = bf16_inputs(orc, 961 + rows, rows, k)
    bias = orc.normal(962, n, 0.1)
    got = run(torch, okq, "okq_gemm_bf16", O.Q6_K, xb, rows, k, wq, n, bias)
    assert np.isfinite(got).all()
    idx = np.unique(np.r_[np.arange(0, rows, 128) + 3, np.arange(0, rows, 128) + 126, rows - 1])
    idx = idx[idx < rows]
    want = orc.linear_q(O.Q6_K, x32.reshape(rows, k)[idx].reshape(-1), idx.size, k, wq, n, bias, O.MODE_SCALAR, 16)
    ok, i, dmax, _ = O.allclose_ref_rule(got[idx].reshape(-1), want, TOL)
    assert ok, f"row {idx[i // n]} col {i % n}: max_abs {dmax}"


def test_gemm_q6k_bf16_wide_one_hot_columns_are_exact(torch, okq, orc):
    """The wide Q6_K kernel on one-hot rows returns d * sc * (q - 32), the
    dequantized weights, for every weight row (scales beyond |sc| = 64, whose
    products exceed 2048, included); rows of 630 bytes."""
    rows, n, k = 2048, 3000, 768
    wq = orc.quantize(O.Q6_K, orc.normal(970, n * k, 0.02))
    w = orc.dequantize(O.Q6_K, wq, n * k).reshape(n, k)
    blocks = np.frombuffer(wq.tobytes(), np.uint8).reshape(n, k // 256, 210)
    assert np.abs(blocks[:, :, 192:208].view(np.int8).astype(int)).max() > 64
    x = np.zeros((rows, k), np.float32)
    cols = np.arange(rows) * 37 % k
    x[np.arange(rows), cols] = 1.0
    got = run(torch, okq, "okq_gemm_bf16", O.Q6_K, orc.f32_to_bf16(x.reshape(-1)), rows, k, wq, n)
    assert np.array_equal(got, w[:, cols].T)


def _dispatch_pairs(torch, okq, orc, t, n, k, seed, pairs):
    """okq_linear_out_by_in_q at each (rows, pinned entry): bit-identical to the
    pinned path (okq_gemv: the GEMV; okq_gemm: the MFMA kernels), and within
    the rule of the reference."""
    wq = orc.quantize(t, orc.normal(seed, n * k, 0.02))
    for rows, pinned in pairs:
        print(f"[gpu] dispatch type={t} rows={rows} N={n} K={k} -> {pinned}", flush=True)
        x = orc.normal(seed + 1 + rows, rows * k, 1.0)
        auto = run(torch, okq, "okq_linear_out_by_in_q", t, x, rows, k, wq, n)
        pin = run(torch, okq, pinned, t, x, rows, k, wq, n)
        assert np.array_equal(auto.view(np.uint32), pin.view(np.uint32)), rows
        check_rows(orc, t, auto, x, rows, k, wq, n, None, 2)
    return wq


@pytest.mark.parametrize("t", [O.Q4_K, O.Q6_K])
def test_linear_dispatch_large_matrices_take_the_decode_batch_kernel_from_5_rows(torch, okq, orc, t):
    """A matrix of 8 MB or more with K = 4096 (33-34 MB here): 4 rows run the
    GEMV, 5 rows the decode-batch kernel."""
    n, k = 14336 if t == O.Q4_K else 10240, 4096
    wq = _dispatch_pairs(torch, okq, orc, t, n, k, 930 + t, ((4, "okq_gemv"), (5, "okq_gemm")))
    assert wq.size >= 16 << 20


def test_linear_dispatch_long_rows_take_the_decode_batch_kernel_from_3_rows(torch, okq, orc):
    """A matrix of 16 MB or more with K >= 8192 (the Llama down projection,
    33 MB, K = 14336): 2 rows run the GEMV, 3 rows the decode-batch kernel."""
    wq = _dispatch_pairs(torch, okq, orc, O.Q4_K, 4096, 14336, 935, ((2, "okq_gemv"), (3, "okq_gemm")))
    assert wq.size >= 16 << 20


@pytest.mark.parametrize("n,edge", [(4096, 5), (1024, 6)])
def test_linear_dispatch_mid_size_matrices_take_the_decode_batch_kernel(torch, okq, orc, n, edge):
    """Q4_K with K = 4096: the 9.4 MB q/o projection runs the decode-batch
    kernel from 5 rows, the 2.4 MB k/v projection from 6 rows; one row fewer
    runs the GEMV."""
    wq = _dispatch_pairs(torch, okq, orc, O.Q4_K, n, 4096, 940 + edge, ((edge - 1, "okq_gemv"), (edge, "okq_gemm")))
    assert (8 << 20 <= wq.size < 16 << 20) if edge == 5 else (2 << 20 <= wq.size < 8 << 20)


def test_linear_dispatch_takes_the_q6k_gemm_above_eight_rows(torch, okq, orc):
    """okq_linear_out_by_in_q: 9+ rows of a Q6_K weight run the MFMA GEMM
    (bit-identical to okq_gemm), up to 8 rows the GEMV (bit-identical to
    okq_gemv)."""
    n, k = 256, 1024
    wq = orc.quantize(O.Q6_K, orc.normal(920, n * k, 0.02))
    for rows, pinned in ((8, "okq_gemv"), (9, "okq_gemm")):
        x = orc.normal(921 + rows, rows * k, 1.0)
        auto = run(torch, okq, "okq_linear_out_by_in_q", O.Q6_K, x, rows, k, wq, n)
        pin = run(torch, okq, pinned, O.Q6_K, x, rows, k, wq, n)
        assert np.array_equal(auto.view(np.uint32), pin.view(np.uint32)), rows


# ---- Q8_0 -----------------------------------------------------------------------
# f32 activations (tiled kernel): B = d * q (d the block's fp16 scale, q its
# int8 quant) enters as two exact fp16 planes, fp16(d * q) and the remainder
# d * q - fp16(d * q): the products are exact as for the K-quants, and no
# per-block scaling follows.  bf16 activations above 32 rows (gemm_q8_kernel):
# x and q enter bf16 MFMAs as they are (exact products), each block's f32 sum
# is scaled by d; ragged tiles, split and unsplit K, K of one stage pair.

Q80_CASES = [
    # decode batches (one or two 16-row MFMA groups, split and unsplit K)
    ("okq_gemm", 1, 96, 256), ("okq_gemm", 5, 300, 1024), ("okq_gemm", 8, 4096, 4096), ("okq_gemm", 16, 1000, 768),
    ("okq_gemm", 13, 4096, 14336), ("okq_gemm_bf16", 3, 14336, 4096), ("okq_gemm", 32, 4096, 4096),
    ("okq_gemm", 24, 20000, 4096), ("okq_gemm", 2, 70003, 256), ("okq_gemm_bf16", 31, 257, 768),
    # tiled GEMM (odd block counts per tile row: 2-byte aligned block starts alternate)
    ("okq_gemm_bf16", 33, 300, 1024), ("okq_gemm_bf16", 130, 1024, 4096), ("okq_gemm_bf16", 128, 4096, 14336),
    ("okq_gemm", 100, 257, 768), ("okq_gemm", 64, 4096, 4096), ("okq_gemm_bf16", 200, 1001, 256),
    ("okq_gemm_bf16", 200, 4096, 4096), ("okq_gemm_bf16", 130, 1000, 2048), ("okq_gemm_bf16", 64, 300, 256),
    ("okq_gemm_bf16", 384, 4352, 512), ("okq_gemm_bf16", 1000, 1000, 512),
    # an odd number of super-blocks, and slices of unequal stage counts (26
    # stages over 6 slices)
    ("okq_gemm_bf16", 130, 520, 768), ("okq_gemm_bf16", 40, 200, 3328),
]


@pytest.mark.parametrize("entry,rows,n,k", Q80_CASES)
def test_gemm_q8_0_matches_reference(torch, okq, orc, entry, rows, n, k):
    print(f"[gpu] gemm {entry} Q8_0 M={rows} N={n} K={k}", flush=True)
    wq = orc.quantize(O.Q8_0, orc.normal(1800 + n + k, n * k, 0.02))
    bias = orc.normal(1801 + rows, n, 0.1)
    if entry == "okq_gemm_bf16":
        xin, x32 = bf16_inputs(orc, 1802 + rows, rows, k)
    else:
        xin = x32 = orc.normal(1802 + rows, rows * k, 1.0)
    got = run(torch, okq, entry, O.Q8_0, xin, rows, k, wq, n, bias)
    assert np.isfinite(got).all()
    check_rows(orc, O.Q8_0, got, x32, rows, k, wq, n, bias, None if n * k * rows <= 2e9 else 8)


@pytest.mark.parametrize("rows", [128, 512, 2048])
def test_gemm_q8_0_prefill_4096_sampled_rows(torch, okq, orc, rows):
    """Q8_0 prefill at M in {128, 512, 2048} on 4096 x 4096 (bf16 activations)."""
    n = k = 4096
    print(f"[gpu] gemm Q8_0 prefill M={rows}", flush=True)
    wq = orc.quantize(O.Q8_0, orc.normal(1850, n * k, 0.02))
    xb, x32 = bf16_inputs(orc, 1851 + rows, rows, k)
    got = run(torch, okq, "okq_linear_out_by_in_q_bf16", O.Q8_0, xb, rows, k, wq, n)
    assert np.isfinite(got).all()
    check_rows(orc, O.Q8_0, got, x32, rows, k, wq, n, None, 16)


@pytest.mark.parametrize("rows,n,k", [(2048, 4096, 4096), (2000, 4000, 512), (1100, 7000, 1024)])
def test_gemm_q8_0_bf16_rows_of_every_m_tile(torch, okq, orc, rows, n, k):
    """bf16 Q8_0 prefill on grids that take the 8-wave 128 x 256 tiles (and
    ragged M and N tiles): two rows of every 128-row tile and the last row
    checked against the reference CPU path."""
    print(f"[gpu] gemm Q8_0 bf16 M={rows} N={n} K={k} (rows of every tile)", flush=True)
    wq = orc.quantize(O.Q8_0, orc.normal(1880 + n + k, n * k, 0.02))
    xb, x32 = bf16_inputs(orc, 1881 + rows, rows, k)
    bias = orc.normal(1882, n, 0.1)
    got = run(torch, okq, "okq_gemm_bf16", O.Q8_0, xb, rows, k, wq, n, bias)
    assert np.isfinite(got).all()
    idx = np.unique(np.r_[np.arange(0, rows, 128) + 3, np.arange(0, rows, 128) + 126, rows - 1])
    idx = idx[idx < rows]
    want = orc.linear_q(O.Q8_0, x32.reshape(rows, k)[idx].reshape(-1), idx.size, k, wq, n, bias, O.MODE_SCALAR, 16)
    ok, i, dmax, _ = O.allclose_ref_rule(got.reshape(rows, n)[idx].reshape(-1), want, TOL)
    assert ok, f"row {idx[i // n]} col {i % n}: max_abs {dmax}"


def test_gemm_q8_0_one_hot_columns_are_exact(torch, okq, orc):
    """x = e_j returns d * q of every weight row bit for bit (hi + lo = d * q
    exactly), on the decode-batch (16 rows) and tiled (40 rows) kernels, with
    scales up to d = 500 (|d * q| up to 63500) in some blocks."""
    n, k = 64, 512
    wq = orc.quantize(O.Q8_0, orc.normal(1860, n * k, 0.02))
    blocks = wq.reshape(-1, 34).copy()
    big = np.array([500.0, 3.0, 2.0 ** -20, 257.125], np.float16).view(np.uint16)
    blocks[::7, 0:2] = big[np.arange(blocks[::7].shape[0]) % 4].view(np.uint8).reshape(-1, 2)
    wq = blocks.reshape(-1)
    w = orc.dequantize(O.Q8_0, wq, n * k).reshape(n, k)
    assert np.abs(w).max() > 60000
    for rows in (16, 40):
        x = np.zeros((rows, k), np.float32)
        cols = (np.arange(rows) * 37) % k
        x[np.arange(rows), cols] = 1.0
        for entry, xin in (("okq_gemm", x.reshape(-1)), ("okq_gemm_bf16", orc.f32_to_bf16(x.reshape(-1)))):
            got = run(torch, okq, entry, O.Q8_0, xin, rows, k, wq, n)
            assert np.array_equal(got, w[:, cols].T), (entry, rows)


def test_linear_dispatch_takes_the_q8_0_gemm_above_eight_rows(torch, okq, orc):
    """okq_linear_out_by_in_q on a small Q8_0 weight: 9+ rows run the MFMA
    kernels (bit-identical to okq_gemm), up to 8 rows the GEMV; a 17.8 MB
    4096 x 4096 weight takes the decode-batch kernel from 5 rows."""
    for n, k, cases in ((256, 1024, ((8, "okq_gemv"), (9, "okq_gemm"), (40, "okq_gemm"))),
                        (4096, 4096, ((4, "okq_gemv"), (5, "okq_gemm")))):
        wq = orc.quantize(O.Q8_0, orc.normal(1870 + n, n * k, 0.02))
        for rows, pinned in cases:
            print(f"[gpu] dispatch Q8_0 rows={rows} N={n} K={k}", flush=True)
            x = orc.normal(1871 + rows, rows * k, 1.0)
            auto = run(torch, okq, "okq_linear_out_by_in_q", O.Q8_0, x, rows, k, wq, n)
            pin = run(torch, okq, pinned, O.Q8_0, x, rows, k, wq, n)
            assert np.array_equal(auto.view(np.uint32), pin.view(np.uint32)), (n, rows)
            check_rows(orc, O.Q8_0, auto, x, rows, k, wq, n, None, 2)


# ---- Q4_K prefill with bf16 activations: weights dequantised in registers --------
# gemm_wide_q4k_kernel: 128 x 256 tiles, each weight column owned by one wave,
# the min term contracted exactly (dmin * m as two fp16 planes), split-K when
# the tiles leave CUs idle.

WIDE_CASES = [
    # (rows, n, k): ragged M and N (partial tiles, columns past N), one
    # super-block, split K (few tiles), a long K, several M-tiles per N-tile
    (33, 257, 256), (129, 300, 1024), (100, 4096, 4096), (256, 1000, 14336), (300, 520, 2048),
    (512, 1024, 4096), (777, 2100, 768),
]


@pytest.mark.parametrize("rows,n,k", WIDE_CASES)
def test_gemm_wide_q4k_bf16_matches_reference(torch, okq, orc, rows, n, k):
    print(f"[gpu] gemm wide bf16 Q4_K M={rows} N={n} K={k}", flush=True)
    wq = orc.quantize(O.Q4_K, orc.normal(2100 + n + k, n * k, 0.02))
    xb, x32 = bf16_inputs(orc, 2101 + rows, rows, k)
    bias = orc.normal(2102, n, 0.1)
    got = run(torch, okq, "okq_gemm_bf16", O.Q4_K, xb, rows, k, wq, n, bias)
    assert np.isfinite(got).all()
    check_rows(orc, O.Q4_K, got, x32, rows, k, wq, n, bias, None if rows * n * k <= 4e8 else 16)


@pytest.mark.parametrize("t,rows,n,k", [(O.Q4_K, 129, 300, 1024), (O.Q4_K, 511, 4096, 4096),
                                         (O.Q8_0, 127, 4096, 4096), (O.Q6_K, 511, 4096, 14336)])
def test_splitk_reduction_paths_agree_bit_for_bit(torch, okq, orc, t, rows, n, k):
    """Split-K shapes with N a multiple of 4 and an odd row count: a 16-byte
    aligned output takes the reduction with four outputs and two rows per
    thread (the last row pair half empty), an output 4 bytes into its buffer
    the one-output-per-thread reduction.  Both sum the slices in the same
    order and scale and add the bias as one exact FMA: the same bits, and the
    reference rule on sampled rows."""
    print(f"[gpu] split-K reduction paths type {t} M={rows} N={n} K={k}", flush=True)
    wq = orc.quantize(t, orc.normal(2300 + n + k, n * k, 0.02))
    xb, x32 = bf16_inputs(orc, 2301 + rows, rows, k)
    bias = orc.normal(2302, n, 0.1)
    xd = torch.from_numpy(np.ascontiguousarray(xb)).cuda()
    wd = torch.from_numpy(wq).cuda()
    bd = torch.from_numpy(np.asarray(bias, np.float32)).cuda()
    buf = torch.full((rows * n + 4,), float("nan"), dtype=torch.float32, device="cuda")
    outs = []
    for off in (0, 1):  # element offset 0: 16-byte aligned; 1: 4 bytes in
        okq.call("okq_gemm_bf16", xd.data_ptr(), rows, k, t, wd.data_ptr(), wq.size, n, bd.data_ptr(),
                 buf.data_ptr() + 4 * off, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        outs.append(buf[off:off + rows * n].cpu().numpy().reshape(rows, n).copy())
        buf.fill_(float("nan"))
    assert buf.data_ptr() % 16 == 0
    assert np.isfinite(outs[0]).all()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    check_rows(orc, t, outs[0], x32, rows, k, wq, n, bias, 3)


def test_gemm_wide_one_hot_columns_are_exact(torch, okq, orc):
    """x = e_j (40 rows, bf16) returns the dequantised weights bit for bit:
    d * (sc * q) + (-(dmin * m))_hi + (-(dmin * m))_lo is the reference's
    d * sc * q - dmin * m when every product is exact, which the one-hot
    column makes the case (a single nonzero activation per row)."""
    n, k = 300, 1024
    wq = orc.quantize(O.Q4_K, orc.normal(2110, n * k, 0.02))
    w = orc.dequantize(O.Q4_K, wq, n * k).reshape(n, k)
    cols = np.array([0, 1, 7, 31, 32, 63, 64, 100, 127, 128, 200, 255, 256, 257, 300, 383, 384, 500, 511, 512,
                     600, 640, 700, 767, 768, 800, 900, 959, 960, 1000, 1010, 1015, 1016, 1017, 1020, 1021, 1022,
                     1023, 2, 3])
    x = np.zeros((cols.size, k), np.float32)
    x[np.arange(cols.size), cols] = 1.0
    got = run(torch, okq, "okq_gemm_bf16", O.Q4_K, orc.f32_to_bf16(x.reshape(-1)), cols.size, k, wq, n)
    assert np.array_equal(got, w[:, cols].T)


# ---- Q5_K ------------------------------------------------------------------------
# Q4_K with a fifth bit per weight (qh): B = sc * q with q <= 31, so sc * q <=
# 1953 stays an exact fp16 integer and every product is exact as for Q4_K.
# The decode-batch kernel (DecQ5K), the tiled kernel (f32 activations) and
# the register-dequant kernels (bf16 activations) take it.

Q5K_CASES = [
    # decode batches: one and two 16-row groups, split and unsplit K, ragged N
    ("okq_gemm", 1, 96, 256), ("okq_gemm", 5, 300, 1024), ("okq_gemm", 8, 4096, 4096), ("okq_gemm", 16, 1000, 768),
    ("okq_gemm", 13, 4096, 14336), ("okq_gemm_bf16", 3, 14336, 4096), ("okq_gemm", 6, 8000, 4096),
    ("okq_gemm", 17, 300, 1024), ("okq_gemm", 32, 4096, 4096), ("okq_gemm_bf16", 25, 1000, 768),
    ("okq_gemm", 2, 70001, 256), ("okq_gemm", 32, 300, 32768),
    # tiled GEMM: 128-row tiles (f32 with the lo plane, bf16) and 256-row tiles (bf16 above 128 rows)
    ("okq_gemm", 33, 300, 1024), ("okq_gemm", 100, 257, 768), ("okq_gemm_bf16", 40, 1000, 512),
    ("okq_gemm_bf16", 130, 1024, 4096), ("okq_gemm_bf16", 300, 4096, 14336), ("okq_gemm", 64, 4096, 4096),
]


@pytest.mark.parametrize("entry,rows,n,k", Q5K_CASES)
def test_gemm_q5k_matches_reference(torch, okq, orc, entry, rows, n, k):
    print(f"[gpu] gemm {entry} Q5_K M={rows} N={n} K={k}", flush=True)
    wq = orc.quantize(O.Q5_K, orc.normal(2100 + n + k, n * k, 0.02))
    bias = orc.normal(2101 + rows, n, 0.1)
    if entry == "okq_gemm_bf16":
        xin, x32 = bf16_inputs(orc, 2102 + rows, rows, k)
    else:
        xin = x32 = orc.normal(2102 + rows, rows * k, 1.0)
    got = run(torch, okq, entry, O.Q5_K, xin, rows, k, wq, n, bias)
    assert np.isfinite(got).all()
    check_rows(orc, O.Q5_K, got, x32, rows, k, wq, n, bias, None if n * k * rows <= 2e9 else 8)


@pytest.mark.parametrize("rows", [128, 512, 2048])
def test_gemm_q5k_prefill_c4_gate_sampled_rows(torch, okq, orc, rows):
    """Q5_K prefill at M in {128, 512, 2048} on the 14336 x 4096 gate shape
    (bf16 activations), rows from both ends of the batch."""
    n, k = 14336, 4096
    print(f"[gpu] gemm Q5_K prefill M={rows}", flush=True)
    wq = orc.quantize(O.Q5_K, orc.normal(2150, n * k, 0.02))
    xb, x32 = bf16_inputs(orc, 2151 + rows, rows, k)
    got = run(torch, okq, "okq_linear_out_by_in_q_bf16", O.Q5_K, xb, rows, k, wq, n)
    assert np.isfinite(got).all()
    check_rows(orc, O.Q5_K, got, x32, rows, k, wq, n, None, 8)


def test_gemm_q5k_one_hot_columns_are_exact(torch, okq, orc):
    """x = e_j picks column j of every weight row: every Q5_K path (GEMV, the
    decode-batch kernel at 16 rows, the tiled kernel at 40 rows, f32 and
    bf16) returns the dequantized value bit for bit, with the fifth bit set
    on part of the columns."""
    n, k = 64, 512
    wq = orc.quantize(O.Q5_K, orc.normal(2160, n * k, 0.02))
    w = orc.dequantize(O.Q5_K, wq, n * k).reshape(n, k)
    assert (wq.reshape(-1, 176)[:, 16:48] != 0).any()
    for rows in (1, 16, 40):
        x = np.zeros((rows, k), np.float32)
        cols = (np.arange(rows) * 37 + 5) % k
        x[np.arange(rows), cols] = 1.0
        entries = (("okq_gemv", x.reshape(-1)),) if rows == 1 else \
            (("okq_gemm", x.reshape(-1)), ("okq_gemm_bf16", orc.f32_to_bf16(x.reshape(-1))))
        for entry, xin in entries:
            got = run(torch, okq, entry, O.Q5_K, xin, rows, k, wq, n)
            assert np.array_equal(got, w[:, cols].T), (entry, rows)


def test_gemm_q5k_fifth_bit_probe(torch, okq, orc):
    """Blocks whose only non-zero quant bit is the fifth (qs = 0, one qh bit
    set, d = 1, sc = 1, dmin = 0): the value 16 must land at exactly the
    element the bit names, on the GEMV, the decode-batch kernel, the tiled
    kernel (f32) and the register-dequant kernels (bf16: the 4-wave pair
    kernel at 40 rows, the 8-wave wide kernel at 256), so that a misplaced
    bit plane or chunk shift moves or drops it."""
    k = 256
    blocks = []
    for p in range(k):
        b = np.zeros(176, np.uint8)
        b[0], b[1] = 0x00, 0x3C                  # d = 1.0
        b[4:8] = 1                                # sc of sub-blocks 0-3 = 1 (6-bit), mins 0
        b[12:16] = 0x01                           # sc of sub-blocks 4-7 = 1 (low nibble), mins 0
        c, hi, l = p // 64, (p // 32) % 2, p % 32
        b[16 + l] = 1 << (2 * c + hi)
        blocks.append(b)
    wq = np.concatenate(blocks)
    w = orc.dequantize(O.Q5_K, wq, k * k).reshape(k, k)
    assert (w == 16.0 * np.eye(k, dtype=np.float32)).all()
    x = np.eye(k, dtype=np.float32)
    for entry, rows in (("okq_gemv", 1), ("okq_gemm", 16), ("okq_gemm", 40), ("okq_gemm_bf16", 40),
                        ("okq_gemm_bf16", 256)):
        xin = x[:rows].reshape(-1)
        if entry == "okq_gemm_bf16":
            xin = orc.f32_to_bf16(xin)
        got = run(torch, okq, entry, O.Q5_K, xin, rows, k, wq, k)
        assert np.array_equal(got, w[:, :rows].T), (entry, rows)


def test_linear_dispatch_routes_q5k_like_q4k(torch, okq, orc):
    """okq_linear_out_by_in_q on Q5_K weights: up to 8 rows the GEMV (a
    36.7 MB 4096 x 14336 weight from 3 rows the decode-batch kernel), 9-32
    rows the decode-batch kernel, above 32 the tiled kernel; each bit for bit
    equal to the pinned entry point and within the rule of the reference."""
    _dispatch_pairs(torch, okq, orc, O.Q5_K, 256, 1024, 2170,
                    ((8, "okq_gemv"), (9, "okq_gemm"), (40, "okq_gemm")))
    _dispatch_pairs(torch, okq, orc, O.Q5_K, 4096, 14336, 2180, ((2, "okq_gemv"), (3, "okq_gemm")))
