"""GPU parity at the benchmark configurations' exact shapes (needs an MI355X).

Every shape the bench times is checked here against the reference CPU path
(the oracle's restatement of linear_out_by_in, crates/kernels/src/lib.rs:
1974-2123, on the dequantized weights) with the reference rule abs <= 1e-3 ||
rel <= 1e-3 per element (lib.rs:2995-3002).  The C4 prefill calls are checked
on every output (the 16-thread scalar oracle takes about 1.4 s for the largest,
M=2048 gate); the C5 problems on a sample of rows (every output row is an
independent dot product, so a wrong tile, split or index shows up in any row
it touches; the samples cover the first and last rows and rows inside).

  C4  Q4_K prefill GEMM, bf16 activations, M in {128, 512, 2048} at the four
      Llama-3-8B projection shapes (q/o 4096x4096, k/v 1024x4096, gate/up
      14336x4096, down 4096x14336)
  C5  the Q6_K head 128256x4096 at batch 8 and 32, and one Q4_K_M layer
      (Q4_K q, k, o, gate, up; Q6_K v, down) through the grouped calls an
      engine issues, at batch 1, 8 and 32
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


def _stream(torch):
    return torch.cuda.current_stream().cuda_stream


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def sample_rows(rows, k_first=4, k_mid=4):
    """First and last rows plus a few inside (deterministic)."""
    rng = np.random.default_rng(rows)
    mid = rng.choice(np.arange(k_first, max(k_first + 1, rows - k_first)), size=min(k_mid, max(0, rows - 2 * k_first)),
                     replace=False) if rows > 2 * k_first else np.array([], int)
    return np.unique(np.r_[np.arange(min(k_first, rows)), np.arange(max(0, rows - k_first), rows), mid]).astype(int)


def check(orc, t, got, x32, rows, k, wq, n, bias, idx, label):
    xs = x32.reshape(rows, k)[idx].reshape(-1)
    want = orc.linear_q(t, xs, idx.size, k, wq, n, bias, O.MODE_SCALAR, 16)
    ok, i, dmax, _ = O.allclose_ref_rule(got.reshape(rows, n)[idx], want, TOL)
    assert ok, (f"{label}: row {idx[i // n]} col {i % n}: got {got.reshape(rows, n)[idx].reshape(-1)[i]} "
                f"want {want.reshape(-1)[i]} max_abs {dmax}")


C2_SHAPES = {"q": (4096, 4096), "k": (1024, 4096), "gate": (14336, 4096), "down": (4096, 14336)}


@pytest.fixture(scope="module")
def c4_weights(orc):
    return {name: orc.quantize(O.Q4_K, orc.normal(7700 + i, n * k, 0.02))
            for i, (name, (n, k)) in enumerate(C2_SHAPES.items())}


@pytest.mark.parametrize("m,name", [(m, name) for m in (128, 512, 2048) for name in C2_SHAPES])
def test_c4_gemm_at_every_bench_shape(torch, okq, orc, c4_weights, m, name):
    """C4: okq_gemm_bf16 (the dispatch the bench times) at every M and
    projection shape, every output against the oracle: every 128-row tile,
    column tile and K slice of whichever kernel the plan picks."""
    n, k = C2_SHAPES[name]
    print(f"[gpu] C4 M={m} {name} N={n} K={k}", flush=True)
    wq = c4_weights[name]
    xb = orc.f32_to_bf16(orc.normal(7800 + m + k, m * k, 1.0))
    x32 = orc.bf16_to_f32(xb)
    bias = orc.normal(7801, n, 0.1)
    xd, wd, bd = _dev(torch, xb.view(np.int16)), _dev(torch, wq), _dev(torch, bias)
    out = torch.full((m * n,), float("nan"), dtype=torch.float32, device="cuda")
    okq.call("okq_gemm_bf16", xd.data_ptr(), m, k, O.Q4_K, wd.data_ptr(), wq.size, n, bd.data_ptr(), out.data_ptr(),
             _stream(torch))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    check(orc, O.Q4_K, got, x32, m, k, wq, n, bias, np.arange(m), f"C4 M={m} {name}")


@pytest.fixture(scope="module")
def head(orc):
    n, k = 128256, 4096
    return n, k, orc.quantize(O.Q6_K, orc.normal(7900, n * k, 0.02))


@pytest.mark.parametrize("rows", [8, 32])
def test_c5_head_at_decode_batches(torch, okq, orc, head, rows):
    """C5: the Q6_K output head at batch 8 and 32 through
    okq_linear_out_by_in_q (the decode-batch MFMA kernel: the widest problem
    it serves, several column tiles per wave)."""
    n, k, wq = head
    print(f"[gpu] C5 head rows={rows} N={n} K={k}", flush=True)
    x = orc.normal(7901 + rows, rows * k, 1.0)
    xd, wd = _dev(torch, x), _dev(torch, wq)
    out = torch.full((rows * n,), float("nan"), dtype=torch.float32, device="cuda")
    okq.call("okq_linear_out_by_in_q", xd.data_ptr(), rows, k, O.Q6_K, wd.data_ptr(), wq.size, n, None,
             out.data_ptr(), _stream(torch))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    check(orc, O.Q6_K, got, x, rows, k, wq, n, None, sample_rows(rows, 3, 2), f"C5 head rows={rows}")


C5_LAYER = [("q", O.Q4_K, 4096, 4096), ("k", O.Q4_K, 1024, 4096), ("v", O.Q6_K, 1024, 4096),
            ("o", O.Q4_K, 4096, 4096), ("gate", O.Q4_K, 14336, 4096), ("up", O.Q4_K, 14336, 4096),
            ("down", O.Q6_K, 4096, 14336)]


@pytest.fixture(scope="module")
def c5_layer(orc):
    return {name: (t, n, k, orc.quantize(t, orc.normal(8000 + i, n * k, 0.02)))
            for i, (name, t, n, k) in enumerate(C5_LAYER)}


@pytest.mark.parametrize("rows", [1, 8, 32])
def test_c5_layer_through_the_grouped_calls(torch, okq, orc, c5_layer, rows):
    """C5: one Llama-3-8B layer in the Q4_K_M mix, issued as the bench's
    `grouped` step issues it -- q+k+v through okq_linear_multi_q (Q4_K q/k and
    Q6_K v: GEMV launches at batch 1, one mixed-format decode-batch launch at 8
    and 32), gate+up through okq_gemv_multi, o and down through
    okq_linear_out_by_in_q -- every output against the reference."""
    s = _stream(torch)
    x4 = orc.normal(8100 + rows, rows * 4096, 1.0)
    x14 = orc.normal(8101 + rows, rows * 14336, 1.0)
    xd4, xd14 = _dev(torch, x4), _dev(torch, x14)
    wd = {name: _dev(torch, v[3]) for name, v in c5_layer.items()}
    outs = {name: torch.full((rows * v[1],), float("nan"), dtype=torch.float32, device="cuda")
            for name, v in c5_layer.items()}

    def group(names):
        t, _, k, _ = c5_layer[names[0]]
        c = len(names)
        okq.call("okq_gemv_multi", xd4.data_ptr(), rows, k, t, c,
                 (ctypes.c_void_p * c)(*[wd[m].data_ptr() for m in names]),
                 (ctypes.c_uint64 * c)(*[c5_layer[m][3].size for m in names]),
                 (ctypes.c_int64 * c)(*[c5_layer[m][1] for m in names]), None,
                 (ctypes.c_void_p * c)(*[outs[m].data_ptr() for m in names]), s)

    def multi(names):
        c = len(names)
        okq.call("okq_linear_multi_q", xd4.data_ptr(), rows, 4096, c,
                 (ctypes.c_uint32 * c)(*[c5_layer[m][0] for m in names]),
                 (ctypes.c_void_p * c)(*[wd[m].data_ptr() for m in names]),
                 (ctypes.c_uint64 * c)(*[c5_layer[m][3].size for m in names]),
                 (ctypes.c_int64 * c)(*[c5_layer[m][1] for m in names]), None,
                 (ctypes.c_void_p * c)(*[outs[m].data_ptr() for m in names]), s)

    def one(name):
        t, n, k, wq = c5_layer[name]
        xd = xd14 if k == 14336 else xd4
        okq.call("okq_linear_out_by_in_q", xd.data_ptr(), rows, k, t, wd[name].data_ptr(), wq.size, n, None,
                 outs[name].data_ptr(), s)

    print(f"[gpu] C5 layer rows={rows}", flush=True)
    multi(["q", "k", "v"])
    one("o")
    group(["gate", "up"])
    one("down")
    torch.cuda.synchronize()
    idx = sample_rows(rows, 3, 2)
    for name, (t, n, k, wq) in c5_layer.items():
        got = outs[name].cpu().numpy()
        assert np.isfinite(got).all(), name
        check(orc, t, got, x14 if k == 14336 else x4, rows, k, wq, n, None, idx, f"C5 rows={rows} {name}")
