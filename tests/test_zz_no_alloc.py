"""okq_linear_out_by_in_q_noalloc, the allocation-free variant of
okq_linear_out_by_in_q (needs an MI355X).

Same dispatch and kernels, scratch from a static device array instead of the
per-stream workspace: outputs must equal okq_linear_out_by_in_q's bit for
bit, on calls in a row that reuse the array (the second smaller than the
first, both with split-K partials in the scratch), under graph capture on a
stream that never ran a GEMM (where the allocating entry point would have to
allocate and fails), and a problem whose scratch exceeds the array must fail
before anything launches.
"""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


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


def _call(torch, okq, entry, t, xd, rows, k, wd, nbytes, n, bd):
    out = torch.full((rows * n,), float("nan"), dtype=torch.float32, device="cuda")
    okq.call(entry, xd.data_ptr(), rows, k, t, wd.data_ptr(), nbytes, n, None if bd is None else bd.data_ptr(),
             out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    return out


# pairs of calls in a row: a larger problem, then a smaller one (same kernel
# family), so the second call reuses scratch the first one filled.  At 256
# CUs the decode-batch plans of the first three pairs split K on both calls
# (16 and 16 slices; 16 and 16; 16 and 4), so partials of the first call sit
# in the scratch when the second one writes and reduces its own.
PAIRS = [
    # decode-batch kernel with split-K partials in the scratch
    [(O.Q4_K, 32, 4096, 14336), (O.Q4_K, 24, 1024, 4096)],
    [(O.Q6_K, 32, 4096, 14336), (O.Q6_K, 16, 4096, 4096)],
    [(O.Q8_0, 32, 4096, 4096), (O.Q8_0, 20, 14336, 4096)],
    # tiled GEMM: activation planes, sums, row scales and partials in the scratch
    [(O.Q4_K, 64, 4096, 4096), (O.Q4_K, 40, 300, 1024)],
    [(O.Q6_K, 130, 1024, 4096), (O.Q6_K, 33, 96, 256)],
    # the GEMV needs no scratch
    [(O.Q8_0, 4, 4096, 4096), (O.Q4_K, 1, 1024, 4096)],
]


@pytest.mark.parametrize("pair", PAIRS, ids=[f"{a[0]}-{a[1]}x{a[2]}x{a[3]}" for a, _ in PAIRS])
def test_noalloc_equals_linear_out_by_in_q_on_calls_in_a_row(torch, okq, orc, pair):
    prepared = []
    for i, (t, rows, n, k) in enumerate(pair):
        wq = orc.quantize(t, orc.normal(9900 + i + n, n * k, 0.02))
        x = orc.normal(9910 + i + rows, rows * k, 1.0)
        bias = orc.normal(9920 + i, n, 0.1) if i == 0 else None
        dev = [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (x, wq)]
        bd = None if bias is None else torch.from_numpy(bias).cuda()
        prepared.append((t, rows, n, k, wq, dev, bd))
    outs = []
    for t, rows, n, k, wq, (xd, wd), bd in prepared:
        print(f"[gpu] noalloc type={t} rows={rows} N={n} K={k}", flush=True)
        outs.append(_call(torch, okq, "okq_linear_out_by_in_q_noalloc", t, xd, rows, k, wd, wq.size, n, bd))
    torch.cuda.synchronize()
    for (t, rows, n, k, wq, (xd, wd), bd), got in zip(prepared, outs):
        want = _call(torch, okq, "okq_linear_out_by_in_q", t, xd, rows, k, wd, wq.size, n, bd)
        torch.cuda.synchronize()
        g, w = got.cpu().numpy(), want.cpu().numpy()
        assert np.isfinite(g).all()
        assert (g.view(np.uint32) == w.view(np.uint32)).all(), (t, rows, n, k)


def _gpu_quantized(torch, okq, t, n, k, seed):
    """Seeded N(0, 0.02) weights quantized on the GPU (large matrices)."""
    e, b = {O.Q4_K: (256, 144), O.Q6_K: (256, 210), O.Q8_0: (32, 34)}[t]
    s = torch.cuda.current_stream().cuda_stream
    w = torch.empty(n * k // e * b, dtype=torch.uint8, device="cuda")
    f = torch.empty(n * k, dtype=torch.float32, device="cuda")
    okq.call("okq_fill_normal", seed, 0, n * k, 0.02, f.data_ptr(), s)
    okq.call("okq_quantize", t, f.data_ptr(), n * k, w.data_ptr(), s)
    del f
    return w


def test_noalloc_output_head_at_32_rows(torch, okq):
    """The 128256 x 4096 Q6_K output head at 32 f32 rows splits K four ways
    (62.6 MiB of partials, within the 64 MiB array), then 20 rows of the
    14336 x 4096 gate reuse the array: both equal the allocating entry point
    bit for bit."""
    calls = []
    for i, (t, rows, n, k) in enumerate([(O.Q6_K, 32, 128256, 4096), (O.Q4_K, 20, 14336, 4096)]):
        wd = _gpu_quantized(torch, okq, t, n, k, 9950 + i)
        xd = torch.randn(rows * k, generator=torch.Generator().manual_seed(9960 + i)).cuda()
        calls.append((t, rows, n, k, xd, wd))
    outs = []
    for t, rows, n, k, xd, wd in calls:
        print(f"[gpu] noalloc type={t} rows={rows} N={n} K={k}", flush=True)
        outs.append(_call(torch, okq, "okq_linear_out_by_in_q_noalloc", t, xd, rows, k, wd, wd.numel(), n, None))
    torch.cuda.synchronize()
    for (t, rows, n, k, xd, wd), got in zip(calls, outs):
        want = _call(torch, okq, "okq_linear_out_by_in_q", t, xd, rows, k, wd, wd.numel(), n, None)
        torch.cuda.synchronize()
        g, w = got.cpu().numpy(), want.cpu().numpy()
        assert np.isfinite(g).all()
        assert (g.view(np.uint32) == w.view(np.uint32)).all(), (t, rows, n, k)


def test_noalloc_under_graph_capture_on_a_fresh_stream(torch, okq, orc):
    """A stream that never ran a GEMM has no workspace, so the allocating
    entry point cannot be captured on it (OKQ_E_ALLOC); the allocation-free
    one can.  The graph is replayed three times with eager work on another
    stream in between, each replay equal to the eager allocating call."""
    t, rows, n, k = O.Q4_K, 32, 4096, 14336
    wq = orc.quantize(t, orc.normal(9970, n * k, 0.02))
    xd = torch.from_numpy(orc.normal(9971, rows * k, 1.0)).cuda()
    wd = torch.from_numpy(wq).cuda()
    want = _call(torch, okq, "okq_linear_out_by_in_q", t, xd, rows, k, wd, wq.size, n, None)
    torch.cuda.synchronize()
    fresh = torch.cuda.Stream()
    out = torch.full((rows * n,), float("nan"), dtype=torch.float32, device="cuda")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=fresh):
        with pytest.raises(okq.OkqStatusError) as e:
            okq.call("okq_linear_out_by_in_q", xd.data_ptr(), rows, k, t, wd.data_ptr(), wq.size, n, None,
                     out.data_ptr(), fresh.cuda_stream)
        okq.call("okq_linear_out_by_in_q_noalloc", xd.data_ptr(), rows, k, t, wd.data_ptr(), wq.size, n, None,
                 out.data_ptr(), fresh.cuda_stream)
    assert e.value.status == okq.E_ALLOC
    w = want.cpu().numpy()
    for r in range(3):
        out.fill_(float("nan"))
        other = _call(torch, okq, "okq_linear_out_by_in_q", t, xd, 24, k, wd, wq.size, n, None)  # eager work between
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert (out.cpu().numpy().view(np.uint32) == w.view(np.uint32)).all(), f"replay {r}"
        del other
    del g


def test_noalloc_refuses_scratch_beyond_the_static_array(torch, okq, orc):
    """4096 f32 rows of 4096: the tiled GEMM's two fp16 planes alone are
    64 MiB, so with the sums and partials more than the array holds:
    OKQ_E_SHAPE, output untouched."""
    t, rows, n, k = O.Q4_K, 4096, 256, 4096
    wq = orc.quantize(t, orc.normal(9930, n * k, 0.02))
    xd = torch.zeros(rows * k, dtype=torch.float32, device="cuda")
    wd = torch.from_numpy(wq).cuda()
    out = torch.full((rows * n,), 7.0, dtype=torch.float32, device="cuda")
    with pytest.raises(okq.OkqStatusError) as e:
        okq.call("okq_linear_out_by_in_q_noalloc", xd.data_ptr(), rows, k, t, wd.data_ptr(), wq.size, n, None,
                 out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert e.value.status == okq.E_SHAPE and "scratch" in e.value.message
    torch.cuda.synchronize()
    assert (out.cpu().numpy() == 7.0).all()
