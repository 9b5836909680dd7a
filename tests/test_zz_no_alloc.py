"""okq_linear_out_by_in_q_noalloc, the allocation-free variant of
okq_linear_out_by_in_q (needs an MI355X).

Same dispatch and kernels, scratch from a static device array instead of the
per-stream workspace: outputs must equal okq_linear_out_by_in_q's bit for
bit, on calls in a row that reuse the array (the second smaller than the
first), and a problem whose scratch exceeds the array must fail before
anything launches.
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
# family), so the second call reuses scratch the first one filled
PAIRS = [
    # decode-batch kernel with split-K partials in the scratch
    [(O.Q4_K, 8, 14336, 4096), (O.Q4_K, 5, 1000, 2048)],
    [(O.Q6_K, 32, 4096, 14336), (O.Q6_K, 12, 300, 1024)],
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


def test_noalloc_refuses_scratch_beyond_the_static_array(torch, okq, orc):
    """2048 f32 rows of 4096: the tiled GEMM's two fp16 planes alone are
    32 MiB, more than the array holds: OKQ_E_SHAPE, output untouched."""
    t, rows, n, k = O.Q4_K, 2048, 256, 4096
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
