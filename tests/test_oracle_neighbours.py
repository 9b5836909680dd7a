"""The oracle's restatement of the projections' neighbours (rmsnorm, gated
SiLU) pinned against the reference's own hand-checked values
(crates/kernels/src/rmsnorm.rs:150-258, crates/kernels/src/mlp.rs:260-440,
copied as data into tests/golden/reference_kats.json) and against float64
closed forms.  CPU only."""
import json
import os

import numpy as np
import pytest

from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))


@pytest.fixture(scope="module")
def orc():
    return O.Oracle()


@pytest.mark.parametrize("case", range(len(KATS["rmsnorm"])))
def test_rmsnorm_reference_kats(orc, case):
    k = KATS["rmsnorm"][case]
    got = orc.rmsnorm(np.array(k["x"], np.float32), k["rows"], k["hidden"], np.array(k["w"], np.float32), k["eps"])
    want = np.array(k["want"], np.float32)
    assert np.all(np.abs(got - want) <= k["tol"]), (got, want)


def test_rmsnorm_matches_float64_closed_form(orc):
    rng = np.random.default_rng(11)
    rows, hidden = 3, 4096
    x = rng.standard_normal(rows * hidden).astype(np.float32) * 3
    w = rng.standard_normal(hidden).astype(np.float32)
    got = orc.rmsnorm(x, rows, hidden, w, 1e-5).reshape(rows, hidden)
    xd = x.astype(np.float64).reshape(rows, hidden)
    want = xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + 1e-5) * w
    assert np.allclose(got, want, rtol=2e-5, atol=1e-6)
    # a weight of e_j selects column j only: the weight is applied per feature
    e = np.zeros(hidden, np.float32)
    e[17] = 1.0
    sel = orc.rmsnorm(x, rows, hidden, e, 1e-5).reshape(rows, hidden)
    assert np.count_nonzero(sel[:, np.arange(hidden) != 17]) == 0


def test_silu_reference_kats(orc):
    k = KATS["silu"]
    got = orc.swiglu(np.array(k["x"], np.float32), np.ones(len(k["x"]), np.float32))
    assert np.all(np.abs(got - np.array(k["want"], np.float32)) <= k["tol"])
    a = k["asymptotes"]
    got = orc.swiglu(np.array(a["x"], np.float32), np.ones(2, np.float32))
    assert np.all(np.isfinite(got))
    assert np.all(np.abs(got - np.array(a["want"], np.float32)) <= np.array(a["tol"]))


def test_swiglu_matches_float64_and_multiplies_by_up(orc):
    rng = np.random.default_rng(12)
    g = (rng.standard_normal(10000) * 6).astype(np.float32)
    u = rng.standard_normal(10000).astype(np.float32)
    got = orc.swiglu(g, u)
    gd = g.astype(np.float64)
    want = gd / (1.0 + np.exp(-gd)) * u
    assert np.allclose(got, want, rtol=1e-5, atol=1e-7)
    assert np.all(orc.swiglu(g, np.zeros_like(u)) == 0)


def test_mlp_tiny_fixture_through_the_oracle(orc):
    """The reference's hand-computed gated MLP, composed from the oracle's
    reference linear (f32 weights, [out, in]) and its gated SiLU."""
    k = KATS["mlp_gated_silu"]
    rows, h, i = k["rows"], k["hidden"], k["intermediate"]
    x = np.array(k["x"], np.float32)
    # the fixture's weights are [in, out]; linear_out_by_in takes [out, in]
    gate_w = np.array(k["gate_w"], np.float32).reshape(h, i).T.copy()
    up_w = np.array(k["up_w"], np.float32).reshape(h, i).T.copy()
    down_w = np.array(k["down_w"], np.float32).reshape(i, h).T.copy()
    gate = orc.linear(x, rows, h, gate_w.reshape(-1), i)
    up = orc.linear(x, rows, h, up_w.reshape(-1), i)
    out = orc.linear(orc.swiglu(gate, up), rows, i, down_w.reshape(-1), h)
    assert np.all(np.abs(out.reshape(-1) - np.array(k["want"], np.float32)) <= k["tol"]), out
