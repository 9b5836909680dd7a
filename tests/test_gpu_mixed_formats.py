"""GPU parity of okq_linear_multi_q: projections of different GGUF formats that
read the same activations (q/k in Q4_K and v in Q6_K in a Q4_K_M layer).

Bar: every output against the reference CPU path (oracle restatement of
linear_out_by_in on the dequantized weights, crates/kernels/src/lib.rs:
1974-2123) with the reference rule abs <= 1e-3 || rel <= 1e-3, and against
okq_linear_out_by_in_q on the same matrix: bit for bit where the matrix runs
alone or in a same-format group's GEMV launch, within the rule where it shares
the mixed decode-batch launch (the K split follows the combined columns).
"""
import ctypes

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


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _single(torch, okq, t, x, rows, k, wq, n, bias):
    xd = _dev(torch, x)
    wd = _dev(torch, wq)
    bd = None if bias is None else _dev(torch, bias)
    out = torch.full((rows * n,), float("nan"), dtype=torch.float32, device="cuda")
    okq.call("okq_linear_out_by_in_q", xd.data_ptr(), rows, k, t, wd.data_ptr(), wq.size, n,
             None if bd is None else bd.data_ptr(), out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return out.cpu().numpy().reshape(rows, n)


MIXED_CASES = [
    # (rows, k, [(type, n), ...], shared): shared = the Q4_K and Q6_K matrices
    # all take the one mixed decode-batch launch
    (1, 4096, [(O.Q4_K, 4096), (O.Q4_K, 1024), (O.Q6_K, 1024)], False),   # batch 1: a GEMV launch per format
    (8, 4096, [(O.Q4_K, 4096), (O.Q4_K, 1024), (O.Q6_K, 1024)], True),    # Llama q/k/v at 8 rows: K inside the workgroup
    (32, 4096, [(O.Q4_K, 4096), (O.Q4_K, 1024), (O.Q6_K, 1024)], True),   # 32 rows: split K, one reduction
    (16, 768, [(O.Q6_K, 257), (O.Q4_K, 300), (O.Q4_K, 40)], True),        # Q6_K listed first, ragged tiles
    (20, 1024, [(O.Q4_K, 1000), (O.Q6_K, 96), (O.Q6_K, 513), (O.Q4_K, 17)], True),
    (12, 14336, [(O.Q4_K, 1024), (O.Q6_K, 600)], True),                   # a long K
    (3, 1024, [(O.Q4_K, 256), (O.Q6_K, 256)], False),                     # small weights at 3 rows: GEMV
    (40, 1024, [(O.Q4_K, 300), (O.Q6_K, 200)], False),                    # above 32 rows: each on its GEMM
    # a Q5_K_M layer (q/k in Q5_K, v in Q6_K): grouped per format
    (1, 4096, [(O.Q5_K, 4096), (O.Q5_K, 1024), (O.Q6_K, 1024)], False),
    (8, 4096, [(O.Q5_K, 4096), (O.Q5_K, 1024), (O.Q6_K, 1024)], True),
]


@pytest.mark.parametrize("rows,k,mats,shared", MIXED_CASES)
def test_linear_multi_q_mixed_formats(torch, okq, orc, rows, k, mats, shared):
    print(f"[gpu] linear_multi_q rows={rows} K={k} mats={mats}", flush=True)
    wqs = [orc.quantize(t, orc.normal(5100 + 13 * i + t, n * k, 0.02)) for i, (t, n) in enumerate(mats)]
    biases = [orc.normal(5200 + i, n, 0.1) if i % 2 == 0 else None for i, (_, n) in enumerate(mats)]
    x = orc.normal(5300 + rows, rows * k, 1.0)
    xd = _dev(torch, x)
    wds = [_dev(torch, wq) for wq in wqs]
    bds = [None if b is None else _dev(torch, b) for b in biases]
    outs = [torch.full((rows * n,), float("nan"), dtype=torch.float32, device="cuda") for _, n in mats]
    c = len(mats)
    arr = lambda ty, vals: (ty * c)(*vals)
    okq.call("okq_linear_multi_q", xd.data_ptr(), rows, k, c, arr(ctypes.c_uint32, [t for t, _ in mats]),
             arr(ctypes.c_void_p, [w.data_ptr() for w in wds]), arr(ctypes.c_uint64, [wq.size for wq in wqs]),
             arr(ctypes.c_int64, [n for _, n in mats]),
             arr(ctypes.c_void_p, [None if b is None else b.data_ptr() for b in bds]),
             arr(ctypes.c_void_p, [o.data_ptr() for o in outs]), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for i, (t, n) in enumerate(mats):
        got = outs[i].cpu().numpy().reshape(rows, n)
        single = _single(torch, okq, t, x, rows, k, wqs[i], n, biases[i])
        if shared:
            ok, idx, dmax, _ = O.allclose_ref_rule(got, single, TOL)
            assert ok, f"matrix {i} vs its own call: idx={idx} max_abs={dmax}"
        else:
            assert (got.view(np.uint32) == single.view(np.uint32)).all(), f"matrix {i}"
        want = orc.linear_q(t, x, rows, k, wqs[i], n, biases[i])
        ok, idx, dmax, _ = O.allclose_ref_rule(got, want, TOL)
        assert ok, f"matrix {i} (type {t}) idx={idx} max_abs={dmax}"


def test_linear_multi_q_repeats_bit_for_bit(torch, okq, orc):
    """The mixed launch sums every output in a fixed order: two calls on the
    same inputs give the same bits."""
    rows, k, mats = 24, 2048, [(O.Q4_K, 2048), (O.Q6_K, 512)]
    wqs = [orc.quantize(t, orc.normal(5400 + i, n * k, 0.02)) for i, (t, n) in enumerate(mats)]
    xd = _dev(torch, orc.normal(5401, rows * k, 1.0))
    wds = [_dev(torch, wq) for wq in wqs]
    runs = []
    for _ in range(2):
        outs = [torch.empty(rows * n, dtype=torch.float32, device="cuda") for _, n in mats]
        okq.call("okq_linear_multi_q", xd.data_ptr(), rows, k, 2, (ctypes.c_uint32 * 2)(*[t for t, _ in mats]),
                 (ctypes.c_void_p * 2)(*[w.data_ptr() for w in wds]), (ctypes.c_uint64 * 2)(*[w.size for w in wqs]),
                 (ctypes.c_int64 * 2)(*[n for _, n in mats]), None,
                 (ctypes.c_void_p * 2)(*[o.data_ptr() for o in outs]), torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        runs.append([o.cpu().numpy() for o in outs])
    for a, b in zip(*runs):
        assert (a.view(np.uint32) == b.view(np.uint32)).all()
