"""GPU parity of the path's neighbours (needs an MI355X): the quantized
embedding row gather, and the projections fused with the RMSNorm before them
and the gated-SiLU activation after them.

Bars: gathered rows bit-exact against the oracle's dequantization; fused
projections within the reference rule abs <= 1e-3 || rel <= 1e-3 against the
reference order of operations (rmsnorm, crates/kernels/src/rmsnorm.rs:73-128;
mlp_gated_silu, crates/kernels/src/mlp.rs:139-250) evaluated on the CPU.
All calls go through the C-ABI (ctypes), device memory from torch.
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3
TYPES = [O.Q8_0, O.Q4_K, O.Q6_K]


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


@pytest.fixture(scope="module")
def orc():
    return O.Oracle()


def _stream(torch):
    return torch.cuda.current_stream().cuda_stream


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _same_bits(a, b):
    a = np.asarray(a, np.float32).reshape(-1)
    b = np.asarray(b, np.float32).reshape(-1)
    return (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))


# ---- quantized embedding gather ------------------------------------------------

def _get_rows(torch, okq, t, wq, ne0, ne1, ids):
    wd = _dev(torch, wq)
    n = len(ids)
    out = torch.full((max(n, 1) * ne0,), float("nan"), dtype=torch.float32, device="cuda")
    idarr = (ctypes.c_uint32 * max(n, 1))(*ids)
    okq.call("okq_get_rows_q", t, wd.data_ptr(), wq.size, ne0, ne1, idarr, n, out.data_ptr(), _stream(torch))
    torch.cuda.synchronize()
    return out.cpu().numpy()[: n * ne0].reshape(n, ne0)


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("ne0,ne1,n", [(256, 7, 5), (2560, 64, 33), (4096, 300, 1000)])
def test_get_rows_bit_exact(torch, okq, orc, t, ne0, ne1, n):
    """Every gathered row equals the oracle's dequantization of that row bit
    for bit, for repeated, first, last and out-of-order ids and for more ids
    than one launch carries (1000 > 480)."""
    print(f"[gpu] get_rows type={t} ne0={ne0} ne1={ne1} n={n}", flush=True)
    wq = orc.quantize(t, orc.normal(7000 + t + ne0, ne0 * ne1, 0.02))
    table = orc.dequantize(t, wq, ne0 * ne1).reshape(ne1, ne0)
    rng = np.random.default_rng(ne0 + n)
    ids = list(rng.integers(0, ne1, n))
    ids[0], ids[-1] = ne1 - 1, 0
    got = _get_rows(torch, okq, t, wq, ne0, ne1, ids)
    assert _same_bits(got, table[np.asarray(ids)]).all()


@pytest.mark.parametrize("t", [t for t in O.GATHER_TYPES if t not in TYPES])
@pytest.mark.parametrize("ne0,ne1,n", [(256, 5, 4), (2560, 48, 97)])
def test_get_rows_other_block_formats_bit_exact(torch, okq, orc, t, ne0, ne1, n):
    """The dequantize-only formats (Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q5_K)
    gather bit-exactly too.  The oracle has no quantizer for them, so the table
    is random block bytes with every f16 field forced finite (exponent < 31)."""
    print(f"[gpu] get_rows other type={t} ne0={ne0} ne1={ne1} n={n}", flush=True)
    rng = np.random.default_rng(7200 + t + ne0)
    nb = ne0 * ne1 // O.BLOCK_ELEMS[t]
    wq = rng.integers(0, 256, nb * O.BLOCK_BYTES[t], dtype=np.uint8).reshape(nb, O.BLOCK_BYTES[t])
    for off in O.F16_FIELDS[t]:
        wq[:, off + 1] &= 0x7B  # clear one exponent bit: finite halves only
    wq = wq.reshape(-1)
    table = orc.dequantize(t, wq, ne0 * ne1).reshape(ne1, ne0)
    assert np.isfinite(table).all()
    ids = list(rng.integers(0, ne1, n))
    ids[0], ids[-1] = ne1 - 1, 0
    got = _get_rows(torch, okq, t, wq, ne0, ne1, ids)
    assert _same_bits(got, table[np.asarray(ids)]).all()


def test_get_rows_rejects_out_of_range_ids_before_launch(torch, okq, orc):
    ne0, ne1 = 256, 4
    wq = orc.quantize(O.Q4_K, orc.normal(7100, ne0 * ne1, 0.02))
    wd = _dev(torch, wq)
    out = torch.full((2 * ne0,), 7.0, device="cuda")
    ids = (ctypes.c_uint32 * 2)(1, 4)
    with pytest.raises(okq.OkqStatusError) as e:
        okq.call("okq_get_rows_q", O.Q4_K, wd.data_ptr(), wq.size, ne0, ne1, ids, 2, out.data_ptr(), _stream(torch))
    assert e.value.status == okq.E_ARG
    assert "token id 4 is out of range for vocab_size 4" in e.value.message
    torch.cuda.synchronize()
    assert (out.cpu().numpy() == 7.0).all()  # nothing launched
    # byte length and unsupported types are refused too; zero ids is a no-op
    with pytest.raises(okq.OkqStatusError) as e:
        okq.call("okq_get_rows_q", O.Q4_K, wd.data_ptr(), wq.size - 1, ne0, ne1, ids, 1, out.data_ptr(),
                 _stream(torch))
    assert e.value.status == okq.E_SHAPE
    with pytest.raises(okq.OkqStatusError) as e:
        okq.call("okq_get_rows_q", 0, wd.data_ptr(), wq.size, ne0, ne1, ids, 1, out.data_ptr(), _stream(torch))
    assert e.value.status == okq.E_TYPE
    okq.call("okq_get_rows_q", O.Q4_K, wd.data_ptr(), wq.size, ne0, ne1, None, 0, None, _stream(torch))


# ---- RMSNorm, alone and folded into the projections --------------------------

def _rule(got, want, tol=TOL):
    ok, idx, dmax, _ = O.allclose_ref_rule(np.asarray(got, np.float32).reshape(-1),
                                           np.asarray(want, np.float32).reshape(-1), tol)
    return ok, (idx, dmax)


@pytest.mark.parametrize("rows,hidden", [(1, 3), (2, 3), (5, 4096), (3, 14336)])
def test_rmsnorm_matches_oracle(torch, okq, orc, rows, hidden):
    print(f"[gpu] rmsnorm rows={rows} hidden={hidden}", flush=True)
    x = orc.normal(7200 + hidden, rows * hidden, 2.0)
    w = orc.normal(7201 + hidden, hidden, 1.0)
    out = torch.full((rows * hidden,), float("nan"), device="cuda")
    xd, wd = _dev(torch, x), _dev(torch, w)  # named: a temporary's memory would be reused by the next one
    okq.call("okq_rmsnorm", xd.data_ptr(), rows, hidden, wd.data_ptr(), 1e-5, out.data_ptr(), _stream(torch))
    torch.cuda.synchronize()
    ok, info = _rule(out.cpu().numpy(), orc.rmsnorm(x, rows, hidden, w, 1e-5), 1e-5)
    assert ok, info


def test_rmsnorm_reference_kats_on_gpu(torch, okq):
    import json
    import os
    kats = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))["rmsnorm"]
    for k in kats:
        out = torch.full((len(k["x"]),), 42.0, device="cuda")
        xd, wd = _dev(torch, np.array(k["x"], np.float32)), _dev(torch, np.array(k["w"], np.float32))
        okq.call("okq_rmsnorm", xd.data_ptr(), k["rows"], k["hidden"], wd.data_ptr(), k["eps"], out.data_ptr(),
                 _stream(torch))
        torch.cuda.synchronize()
        assert np.all(np.abs(out.cpu().numpy() - np.array(k["want"], np.float32)) <= k["tol"]), k


def test_rmsnorm_rejects_bad_epsilon(torch, okq):
    x = torch.ones(8, device="cuda")
    with pytest.raises(okq.OkqStatusError) as e:
        okq.call("okq_rmsnorm", x.data_ptr(), 1, 8, x.data_ptr(), -1.0, x.data_ptr(), _stream(torch))
    assert "epsilon must be finite and non-negative" in e.value.message
    with pytest.raises(okq.OkqStatusError) as e:
        okq.call("okq_rmsnorm", x.data_ptr(), 1, 0, x.data_ptr(), 1e-6, x.data_ptr(), _stream(torch))
    assert "hidden dimension must be non-zero" in e.value.message


RMS_LINEAR_CASES = [
    # (type, rows, hidden, out_features per matrix)
    (O.Q4_K, 1, 4096, [4096, 1024]),         # q, k of an attention block: fused prologue
    (O.Q4_K, 3, 4096, [512, 256, 256]),      # decode batch, three matrices
    (O.Q6_K, 1, 4096, [1024]),               # v in Q6_K
    (O.Q8_0, 2, 2048, [300]),
    (O.Q4_K, 9, 2048, [512, 128]),           # batch: normalise, then the MFMA GEMM
    (O.Q6_K, 6, 1024, [64]),                 # batch on the per-row GEMV
    (O.Q8_0, 1, 96, [40]),                   # odd Q8_0 block count: generic GEMV after a normalised copy
    (O.Q4_K, 12, 2048, [512, 256, 256]),     # batch above 8 rows: q/k/v in one decode-batch launch
    (O.Q4_K, 1, 4096, [14336, 14336]),       # fused prologue with dynamic rows (gate/up shape)
    (O.Q6_K, 1, 256, [20000]),
]


@pytest.mark.parametrize("t,rows,hidden,ns", RMS_LINEAR_CASES)
def test_rmsnorm_linear_multi_matches_reference_order(torch, okq, orc, t, rows, hidden, ns):
    print(f"[gpu] rmsnorm_linear type={t} rows={rows} hidden={hidden} N={ns}", flush=True)
    x = orc.normal(7300 + rows + hidden, rows * hidden, 1.5)
    g = orc.normal(7301 + hidden, hidden, 1.0)
    wqs = [orc.quantize(t, orc.normal(7310 + 7 * i + t, n * hidden, 0.02)) for i, n in enumerate(ns)]
    biases = [orc.normal(7320 + i, n, 0.1) if i == 0 else None for i, n in enumerate(ns)]
    wds = [_dev(torch, w) for w in wqs]
    bds = [None if b is None else _dev(torch, b) for b in biases]
    outs = [torch.full((rows * n,), float("nan"), device="cuda") for n in ns]
    c = len(ns)
    arr = lambda ty, vals: (ty * c)(*vals)
    xd, gd = _dev(torch, x), _dev(torch, g)
    okq.call("okq_rmsnorm_linear_q_multi", xd.data_ptr(), rows, hidden, gd.data_ptr(), 1e-6,
             t, c, arr(ctypes.c_void_p, [w.data_ptr() for w in wds]), arr(ctypes.c_uint64, [w.size for w in wqs]),
             arr(ctypes.c_int64, ns), arr(ctypes.c_void_p, [None if b is None else b.data_ptr() for b in bds]),
             arr(ctypes.c_void_p, [o.data_ptr() for o in outs]), _stream(torch))
    torch.cuda.synchronize()
    xn = orc.rmsnorm(x, rows, hidden, g, 1e-6)
    for i, n in enumerate(ns):
        want = orc.linear_q(t, xn, rows, hidden, wqs[i], n, biases[i])
        ok, info = _rule(outs[i].cpu().numpy(), want)
        assert ok, (i, info)


# ---- gated-SiLU MLP -------------------------------------------------------------

MLP_CASES = [
    # (gate, up, down types, rows, hidden, intermediate)
    (O.Q4_K, O.Q4_K, O.Q6_K, 1, 4096, 14336),   # Llama-3-8B decode, Q4_K_M mix: grouped gate+up, fused down
    (O.Q4_K, O.Q4_K, O.Q4_K, 2, 1024, 2816),
    (O.Q4_K, O.Q8_0, O.Q6_K, 1, 1024, 2816),   # gate and up in different formats: two passes
    (O.Q4_K, O.Q4_K, O.Q6_K, 7, 1024, 2816),   # batch: GEMM gate/up, materialised SiLU, per-row Q6_K down
    (O.Q8_0, O.Q8_0, O.Q8_0, 3, 512, 1024),
    (O.Q4_K, O.Q4_K, O.Q6_K, 8, 4096, 14336),   # Llama-3-8B batch of 8: gate+up in one decode-batch launch
    (O.Q4_K, O.Q4_K, O.Q6_K, 24, 1024, 256),    # few tiles: gate+up split K, the SiLU in their reduction
    (O.Q6_K, O.Q6_K, O.Q4_K, 20, 1024, 512),    # the same with Q6_K gate/up
]


@pytest.mark.parametrize("tg,tu,td,rows,hidden,inter", MLP_CASES)
def test_mlp_gated_silu_q_matches_reference_order(torch, okq, orc, tg, tu, td, rows, hidden, inter):
    print(f"[gpu] mlp types={tg},{tu},{td} rows={rows} hidden={hidden} inter={inter}", flush=True)
    x = orc.normal(7400 + rows, rows * hidden, 1.0)
    gq = orc.quantize(tg, orc.normal(7401, inter * hidden, 0.02))
    uq = orc.quantize(tu, orc.normal(7402, inter * hidden, 0.02))
    dq = orc.quantize(td, orc.normal(7403, hidden * inter, 0.02))
    gb = torch.full((rows * inter,), float("nan"), device="cuda")
    ub = torch.full((rows * inter,), float("nan"), device="cuda")
    out = torch.full((rows * hidden,), float("nan"), device="cuda")
    gd, ud, dd, xd = _dev(torch, gq), _dev(torch, uq), _dev(torch, dq), _dev(torch, x)
    okq.call("okq_mlp_gated_silu_q", xd.data_ptr(), rows, hidden, inter, tg, gd.data_ptr(), gq.size,
             tu, ud.data_ptr(), uq.size, td, dd.data_ptr(), dq.size, gb.data_ptr(), ub.data_ptr(), out.data_ptr(),
             _stream(torch))
    torch.cuda.synchronize()
    got, g_buf, u_buf = out.cpu().numpy(), gb.cpu().numpy(), ub.cpu().numpy()
    gate = orc.linear_q(tg, x, rows, hidden, gq, inter)
    up = orc.linear_q(tu, x, rows, hidden, uq, inter)
    # Each of the three projections meets the per-output rule on its own
    # inputs.  A single row leaves gate(x) in gate_buf (the SiLU is folded
    # into the down GEMV's prologue; every down weight here streams); more
    # rows leave silu(gate(x)) * up(x) there, as the reference does.
    fused = rows == 1
    ok, info = _rule(u_buf, up)
    assert ok, ("up", info)
    ok, info = _rule(g_buf, gate if fused else orc.swiglu(gate, up))
    assert ok, ("gate", info)
    h = orc.swiglu(g_buf, u_buf) if fused else g_buf
    ok, info = _rule(got, orc.linear_q(td, h, rows, inter, dq, hidden))
    assert ok, ("down", info)
    # End to end against the reference chain, normwise: silu(gate) * up has
    # heavy tails (|h| reaches ~70 std here), so gate/up differences of
    # ~1e-5 reach the output amplified; per element the chain is not bound by
    # the single-projection rule.
    want = orc.linear_q(td, orc.swiglu(gate, up), rows, inter, dq, hidden).reshape(-1)
    assert np.abs(got - want).max() <= 1e-3 * np.abs(want).max()


MLP_SPLIT_CASES = [
    # (gate/up type, down type, rows, hidden, intermediate): gate and up share
    # one decode-batch launch that splits K over workgroups: above 16 rows
    # (up to 16 rows keep K inside the workgroup when it fits), for the LDS
    # (4 super-blocks of 32 rows) or to fill the CUs with few tiles
    (O.Q4_K, O.Q6_K, 32, 4096, 14336),   # Llama-3-8B batch of 32
    (O.Q4_K, O.Q4_K, 24, 1024, 256),
    (O.Q6_K, O.Q4_K, 20, 1024, 512),
    (O.Q8_0, O.Q8_0, 17, 1024, 224),     # down on the GEMV (K = 224 is not whole super-blocks)
]


@pytest.mark.parametrize("tgu,td,rows,hidden,inter", MLP_SPLIT_CASES)
def test_mlp_gated_silu_q_split_reduction_applies_silu(torch, okq, orc, tgu, td, rows, hidden, inter):
    """Where gate+up split K, their reduction leaves up(x) and silu(gate(x)) *
    up(x) itself: up_buf equals okq_gemv_multi's up output bit for bit (the
    same launch plan and slice-order sums), gate_buf equals silu(g) * u of
    okq_gemv_multi's outputs up to the rounding of exp (so each output pairs
    the right gate and up columns), and out is the down projection of
    gate_buf (bit for bit against okq_linear_out_by_in_q on it)."""
    print(f"[gpu] mlp split reduction types={tgu},{td} rows={rows} hidden={hidden} inter={inter}", flush=True)
    x = orc.normal(7500 + rows, rows * hidden, 1.0)
    gq = orc.quantize(tgu, orc.normal(7501, inter * hidden, 0.02))
    uq = orc.quantize(tgu, orc.normal(7502, inter * hidden, 0.02))
    dq = orc.quantize(td, orc.normal(7503, hidden * inter, 0.02))
    gd, ud, dd, xd = _dev(torch, gq), _dev(torch, uq), _dev(torch, dq), _dev(torch, x)
    gb = torch.full((rows * inter,), float("nan"), device="cuda")
    ub = torch.full((rows * inter,), float("nan"), device="cuda")
    out = torch.full((rows * hidden,), float("nan"), device="cuda")
    okq.call("okq_mlp_gated_silu_q", xd.data_ptr(), rows, hidden, inter, tgu, gd.data_ptr(), gq.size,
             tgu, ud.data_ptr(), uq.size, td, dd.data_ptr(), dq.size, gb.data_ptr(), ub.data_ptr(), out.data_ptr(),
             _stream(torch))
    g2 = torch.full((rows * inter,), float("nan"), device="cuda")
    u2 = torch.full((rows * inter,), float("nan"), device="cuda")
    okq.call("okq_gemv_multi", xd.data_ptr(), rows, hidden, tgu, 2, (ctypes.c_void_p * 2)(gd.data_ptr(), ud.data_ptr()),
             (ctypes.c_uint64 * 2)(gq.size, uq.size), (ctypes.c_int64 * 2)(inter, inter), None,
             (ctypes.c_void_p * 2)(g2.data_ptr(), u2.data_ptr()), _stream(torch))
    torch.cuda.synchronize()
    u_buf, g_buf = ub.cpu().numpy(), gb.cpu().numpy()
    g, u = g2.cpu().numpy(), u2.cpu().numpy()
    assert (u_buf.view(np.uint32) == u.view(np.uint32)).all()
    want = (g * (np.float32(1.0) / (np.float32(1.0) + np.exp(-g)))) * u
    assert np.all(np.isfinite(g_buf))
    assert np.abs(g_buf - want).max() <= 4e-7 * np.abs(want).max() + 1e-30
    assert np.all(np.abs(g_buf - want) <= 8 * np.spacing(np.abs(want)))
    out2 = torch.full((rows * hidden,), float("nan"), device="cuda")
    okq.call("okq_linear_out_by_in_q", gb.data_ptr(), rows, inter, td, dd.data_ptr(), dq.size, hidden, None,
             out2.data_ptr(), _stream(torch))
    torch.cuda.synchronize()
    assert (out.cpu().numpy().view(np.uint32) == out2.cpu().numpy().view(np.uint32)).all()


def test_mlp_gated_silu_q_validates_before_launch(torch, okq, orc):
    hidden, inter = 256, 512
    gq = orc.quantize(O.Q4_K, orc.normal(7500, inter * hidden, 0.02))
    dq = orc.quantize(O.Q4_K, orc.normal(7501, hidden * inter, 0.02))
    gd, dd = _dev(torch, gq), _dev(torch, dq)
    x = _dev(torch, orc.normal(7502, hidden, 1.0))
    gb = torch.zeros(inter, device="cuda")
    ub = torch.zeros(inter, device="cuda")
    out = torch.full((hidden,), 7.0, device="cuda")
    args = lambda rows, dbytes: (x.data_ptr(), rows, hidden, inter, O.Q4_K, gd.data_ptr(), gq.size, O.Q4_K,
                                 gd.data_ptr(), gq.size, O.Q4_K, dd.data_ptr(), dbytes, gb.data_ptr(), ub.data_ptr(),
                                 out.data_ptr(), _stream(torch))
    with pytest.raises(okq.OkqStatusError) as e:
        okq.call("okq_mlp_gated_silu_q", *args(0, dq.size))
    assert "seq_len must be non-zero" in e.value.message
    with pytest.raises(okq.OkqStatusError) as e:
        okq.call("okq_mlp_gated_silu_q", *args(1, dq.size - 2))
    assert e.value.status == okq.E_SHAPE and "down projection" in e.value.message
    torch.cuda.synchronize()
    assert (out.cpu().numpy() == 7.0).all()
