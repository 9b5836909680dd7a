"""Pins the CPU oracle's format functions (CPU only).

What pins each oracle function:
  okr_f16_to_f32    reference KATs (safetensors_values.rs:316-351) + all 65536
                    halves against numpy.float16
  okr_bf16_to_f32   reference KATs (safetensors_values.rs:295-313) + exhaustive
                    against torch.bfloat16
  okr_f32_to_f16    1e6 floats incl. ties/subnormals/overflow against numpy
  okr_f32_to_bf16   1e6 floats against torch's RNE conversion
  okr_dequant_*     independent numpy bit-field decoder on random bytes,
                    closed forms, element-order probes, exhaustive Q4_K
                    scale/min unpack (all 2^12 byte combinations per case)
  okr_quantize_*    the build's own algorithm: structural invariants (valid
                    ranges, half-step error bounds where they hold, exact
                    round-trip on representable inputs)
  okr_normal_at     committed first values + moments
"""
import json
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _same_bits(a, b):
    a = np.asarray(a, np.float32).reshape(-1)
    b = np.asarray(b, np.float32).reshape(-1)
    return (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))


@pytest.fixture(scope="module")
def kats():
    with open(os.path.join(GOLDEN, "reference_kats.json")) as f:
        return json.load(f)


def test_f16_reference_kats(orc, kats):
    bits = np.array([b for b, _ in kats["f16"]], np.uint16)
    want = np.array([w for _, w in kats["f16"]], np.uint32)
    assert (orc.f16_to_f32(bits).view(np.uint32) == want).all()
    assert np.isnan(orc.f16_to_f32(np.array(kats["f16_nan"], np.uint16))).all()


def test_f16_exhaustive_matches_numpy(orc):
    bits = np.arange(65536, dtype=np.uint16)
    assert _same_bits(orc.f16_to_f32(bits), O.np_f16_bits_to_f32(bits)).all()
    # NaN payloads are carried as the reference does (frac << 13)
    nan = bits[(bits & 0x7C00) == 0x7C00]
    got = orc.f16_to_f32(nan).view(np.uint32)
    want = ((nan.astype(np.uint32) & 0x8000) << 16) | 0x7F800000 | ((nan.astype(np.uint32) & 0x3FF) << 13)
    assert (got == want).all()


def test_bf16_reference_kats_and_exhaustive(orc, kats):
    bits = np.array([b for b, _ in kats["bf16"]], np.uint16)
    want = np.array([w for _, w in kats["bf16"]], np.uint32)
    assert (orc.bf16_to_f32(bits).view(np.uint32) == want).all()
    allbits = np.arange(65536, dtype=np.uint16)
    assert (orc.bf16_to_f32(allbits).view(np.uint32) == (allbits.astype(np.uint32) << 16)).all()


def _float_sweep(n=1_000_000, seed=7):
    rng = np.random.default_rng(seed)
    mant = rng.standard_normal(n).astype(np.float32)
    exps = rng.integers(-30, 20, n).astype(np.float32)
    x = (mant * np.float32(2.0) ** exps).astype(np.float32)
    # exact halfway cases for f16 (bit 12 set, rest zero) and bf16
    ties = (rng.integers(0, 2**31, 4096, dtype=np.uint32) & ~np.uint32(0x1FFF)) | np.uint32(0x1000)
    ties16 = (rng.integers(0, 2**31, 4096, dtype=np.uint32) & ~np.uint32(0xFFFF)) | np.uint32(0x8000)
    special = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 5.96e-8, 2.98e-8, 2.99e-8,
                        6.1e-5, np.inf, -np.inf], np.float32)
    return np.concatenate([x, ties.view(np.float32), ties16.view(np.float32), special])


def test_f32_to_f16_matches_numpy(orc):
    x = _float_sweep()
    x = x[np.isfinite(x)]
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert (orc.f32_to_f16(x) == want).all()


def test_f32_to_bf16_matches_torch(orc):
    torch = pytest.importorskip("torch")
    x = _float_sweep()
    x = x[np.isfinite(x)]
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert (orc.f32_to_bf16(x) == want).all()


def test_type_ids_block_sizes_and_row_bytes(kats):
    ids = kats["type_ids"]
    assert (ids["Q8_0"], ids["Q4K"], ids["Q6K"]) == (O.Q8_0, O.Q4_K, O.Q6_K)
    assert {t: O.BLOCK_BYTES[t] for t in O.LINEAR_TYPES} == {O.Q8_0: 34, O.Q4_K: 144, O.Q5_K: 176, O.Q6_K: 210}
    assert {t: O.BLOCK_ELEMS[t] for t in O.LINEAR_TYPES} == {O.Q8_0: 32, O.Q4_K: 256, O.Q5_K: 256, O.Q6_K: 256}
    row = lambda t, k: k // O.BLOCK_ELEMS[t] * O.BLOCK_BYTES[t]  # noqa: E731
    assert (row(O.Q8_0, 4096), row(O.Q4_K, 4096), row(O.Q6_K, 4096)) == (4352, 2304, 3360)
    assert (row(O.Q4_K, 14336), row(O.Q6_K, 14336)) == (8064, 11760)
    # GGUF ne order: shape [in, out]; the fixture's token_embd is [2560, 262144] q4_k
    fx = kats["gguf_fixture_token_embd"]
    assert fx["shape"][0] % 256 == 0 and row(O.Q4_K, fx["shape"][0]) == 1440


@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_K, O.Q6_K])
def test_dequant_c_matches_numpy_on_random_bytes(orc, t):
    rng = np.random.default_rng(100 + t)
    nb = 3000
    blocks = rng.integers(0, 256, nb * O.BLOCK_BYTES[t], dtype=np.uint8)
    n = nb * O.BLOCK_ELEMS[t]
    with np.errstate(all="ignore"):
        assert _same_bits(orc.dequantize(t, blocks, n), O.NP_DEQUANT[t](blocks)).all()


def _f16(v):
    return int(np.float16(v).view(np.uint16))


def test_q8_0_closed_forms(orc):
    q = np.arange(-127, 128, dtype=np.int64)[:32 * 7].reshape(7, 32)
    for e in (0, -7, 3):
        blocks = np.zeros((7, 34), np.uint8)
        d = _f16(2.0 ** e)
        blocks[:, 0], blocks[:, 1] = d & 0xFF, d >> 8
        blocks[:, 2:] = q.astype(np.int8).view(np.uint8)
        y = orc.dequantize(O.Q8_0, blocks, 7 * 32)
        assert (y == (q.reshape(-1) * 2.0 ** e).astype(np.float32)).all()


def _q4k_pack_scales(sc, m):
    s = np.zeros(12, np.uint8)
    for j in range(8):
        if j < 4:
            s[j] |= sc[j] & 63
            s[j + 4] |= m[j] & 63
        else:
            s[j + 4] = (sc[j] & 15) | ((m[j] & 15) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (m[j] >> 4) << 6
    return s


def _q4k_block(d, dmin, sc, m, q):
    b = np.zeros(144, np.uint8)
    b[0], b[1] = d & 0xFF, d >> 8
    b[2], b[3] = dmin & 0xFF, dmin >> 8
    b[4:16] = _q4k_pack_scales(sc, m)
    for c in range(4):
        for l in range(32):
            b[16 + 32 * c + l] = q[64 * c + l] | (q[64 * c + 32 + l] << 4)
    return b


def test_q4_k_closed_forms(orc):
    rng = np.random.default_rng(3)
    q = rng.integers(0, 16, 256)
    # dmin = 0 and every sc = 1: y = d * q
    for dv in (1.0, 0.5, 2.0 ** -10):
        b = _q4k_block(_f16(dv), 0, [1] * 8, [0] * 8, q)
        assert (orc.dequantize(O.Q4_K, b, 256) == (q * dv).astype(np.float32)).all()
    # d = dmin = 1, sc = 1: y = q - m (per sub-block)
    m = rng.integers(0, 64, 8)
    b = _q4k_block(_f16(1.0), _f16(1.0), [1] * 8, m, q)
    want = (q - np.repeat(m, 32)).astype(np.float32)
    assert (orc.dequantize(O.Q4_K, b, 256) == want).all()


def test_q4_k_scale_min_unpack_exhaustive(orc):
    """Every combination of the bytes that feed one sub-block's 6-bit scale and
    min, decoded by the C oracle (d=1, dmin=0 -> y = sc*q; d=0, dmin=1 -> -m)
    and checked against the bit-by-bit numpy field extractor."""
    q = np.ones(256, np.int64)
    for j in range(8):
        combos = []
        for lo in range(256):          # the byte carrying the low bits
            for hi2 in range(4):       # top two bits of the second byte
                for hi2b in range(4):  # top two bits of the third byte
                    combos.append((lo, hi2, hi2b))
        blocks_sc = []
        blocks_m = []
        for lo, a, b2 in combos:
            s = np.zeros(12, np.uint8)
            if j < 4:
                s[j] = (lo & 63) | (a << 6)
                s[j + 4] = (lo & 63) | (b2 << 6)
            else:
                s[j + 4] = lo
                s[j - 4] = a << 6
                s[j] = b2 << 6
            base = np.zeros(144, np.uint8)
            base[4:16] = s
            for c in range(4):
                base[16 + 32 * c:16 + 32 * c + 32] = 0x11
            bsc = base.copy()
            bsc[0], bsc[1] = _f16(1.0) & 0xFF, _f16(1.0) >> 8
            bm = base.copy()
            bm[2], bm[3] = _f16(1.0) & 0xFF, _f16(1.0) >> 8
            blocks_sc.append(bsc)
            blocks_m.append(bm)
        blocks_sc = np.stack(blocks_sc)
        blocks_m = np.stack(blocks_m)
        y_sc = orc.dequantize(O.Q4_K, blocks_sc, 256 * len(combos)).reshape(-1, 256)[:, 32 * j]
        y_m = orc.dequantize(O.Q4_K, blocks_m, 256 * len(combos)).reshape(-1, 256)[:, 32 * j]
        sc_np, m_np = O._q4k_field(blocks_sc[:, 4:16], j)
        assert (y_sc == sc_np.astype(np.float32)).all(), j
        assert (y_m == -m_np.astype(np.float32)).all(), j
        assert q is not None


def _q6k_block(d, sc, L):
    b = np.zeros(210, np.uint8)
    for h in range(2):
        Lh = L[128 * h:128 * h + 128]
        for l in range(32):
            b[64 * h + l] = (Lh[l] & 15) | ((Lh[64 + l] & 15) << 4)
            b[64 * h + 32 + l] = (Lh[32 + l] & 15) | ((Lh[96 + l] & 15) << 4)
            b[128 + 32 * h + l] = ((Lh[l] >> 4) | ((Lh[32 + l] >> 4) << 2) | ((Lh[64 + l] >> 4) << 4)
                                   | ((Lh[96 + l] >> 4) << 6))
    b[192:208] = np.asarray(sc, np.int8).view(np.uint8)
    b[208], b[209] = d & 0xFF, d >> 8
    return b


def test_q6_k_closed_forms(orc):
    rng = np.random.default_rng(4)
    L = rng.integers(0, 64, 256)
    b = _q6k_block(_f16(1.0), [1] * 16, L)
    assert (orc.dequantize(O.Q6_K, b, 256) == (L - 32).astype(np.float32)).all()
    sc = rng.integers(-128, 128, 16)
    b = _q6k_block(_f16(0.25), sc, L)
    assert (orc.dequantize(O.Q6_K, b, 256) == ((L - 32) * np.repeat(sc, 16) * 0.25).astype(np.float32)).all()


@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_K, O.Q6_K])
def test_element_order_probe(orc, t):
    """A single non-zero quant at position p must land at y[p] and nowhere else."""
    n = O.BLOCK_ELEMS[t]
    blocks = []
    for p in range(n):
        if t == O.Q8_0:
            b = np.zeros(34, np.uint8)
            b[0], b[1] = _f16(1.0) & 0xFF, _f16(1.0) >> 8
            b[2 + p] = 1
        elif t == O.Q4_K:
            q = np.zeros(256, np.int64)
            q[p] = 1
            b = _q4k_block(_f16(1.0), 0, [1] * 8, [0] * 8, q)
        else:
            L = np.full(256, 32, np.int64)
            L[p] = 33
            b = _q6k_block(_f16(1.0), [1] * 16, L)
        blocks.append(b)
    y = orc.dequantize(t, np.stack(blocks), n * n).reshape(n, n)
    assert (y == np.eye(n, dtype=np.float32)).all()


@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K])
def test_quantizer_invariants(orc, t):
    x = orc.normal(77 + t, 256 * 64, 0.02)
    q = orc.quantize(t, x)
    y = orc.dequantize(t, q, x.size)
    err = np.abs(y - x)
    if t == O.Q8_0:
        b = q.reshape(-1, 34)
        d16 = O.np_f16_bits_to_f32(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
        amax = np.abs(x.reshape(-1, 32)).max(1)
        # q = rint(x*127/amax) with the f32 d; dequant uses fp16(d): half a step
        # plus 127 * |d - fp16(d)| <= 127 * d * 2^-11
        bound = 0.5 * d16 + 127 * (amax / 127) * 2.0 ** -11 + 1e-9
        assert (err.reshape(-1, 32) <= bound[:, None] * (1 + 1e-5)).all()
        assert (np.abs(b[:, 2:].view(np.int8).astype(int)) <= 127).all()
    elif t == O.Q6_K:
        b = q.reshape(-1, 210)
        d16 = O.np_f16_bits_to_f32(b[:, 208].astype(np.uint16) | (b[:, 209].astype(np.uint16) << 8))
        sc = b[:, 192:208].view(np.int8).astype(np.float32)
        de = np.abs(d16[:, None] * sc)                      # [nb, 16] step per sub-block
        step = np.repeat(de, 16, axis=1).reshape(-1)
        # no clipping happens for sub-blocks whose 6-bit scale was not clamped
        assert (err <= 0.5 * step * (1 + 1e-5) + np.abs(x) * 2.0 ** -6 + 1e-9).mean() > 0.99
    elif t in (O.Q4_K, O.Q5_K):
        # the dequantized values of a sub-block lie on one grid k * de - me
        # (k = 0..levels); every input lies within half a grid step of its
        # value unless the 6-bit rounding of the scale clamped it at the top
        # level.  The smallest gap between distinct values of a sub-block is a
        # multiple of de, so half of it bounds the error of unclamped values.
        ys, xs = y.reshape(-1, 32), x.reshape(-1, 32)
        gaps = np.array([np.diff(np.unique(r)).min() if np.unique(r).size > 1 else np.inf for r in ys])
        ok = np.abs(ys - xs) <= 0.5 * gaps[:, None] * (1 + 1e-4) + 1e-9
        assert ok.mean() > 0.99, ok.mean()
        # the finer grid of Q5_K: twice the levels over the same range
        levels = 31 if t == O.Q5_K else 15
        span = xs.max(1) - np.minimum(xs.min(1), 0)
        assert np.median(gaps[np.isfinite(gaps)] / (span[np.isfinite(gaps)] / levels)) < 1.1
    # reconstruction error relative to the weight scale
    rel = np.sqrt(np.mean(err.astype(np.float64) ** 2)) / x.std()
    assert rel < {O.Q8_0: 0.01, O.Q4_K: 0.12, O.Q5_K: 0.06, O.Q6_K: 0.04}[t], rel


def test_q5_k_quantizer_is_q4_k_with_a_fifth_bit(orc):
    """The Q5_K quantizer's fifth bit: qs holds the low four bits of each
    index and qh bit 2c (low nibble) / 2c + 1 (high nibble) of byte l the
    fifth; decoding the indices from the bytes and re-applying the block's
    scales reproduces the oracle's dequantisation, and the indices use the
    whole 0..31 range (the top half occurs, so the fifth bit is exercised)."""
    x = orc.normal(4321, 256 * 32, 0.02)
    q = orc.quantize(O.Q5_K, x).reshape(-1, 176)
    qs, qh = q[:, 48:].astype(np.int64), q[:, 16:48].astype(np.int64)
    idx = np.zeros((q.shape[0], 256), np.int64)
    for c in range(4):
        for l in range(32):
            idx[:, 64 * c + l] = (qs[:, 32 * c + l] & 15) | (((qh[:, l] >> (2 * c)) & 1) << 4)
            idx[:, 64 * c + 32 + l] = (qs[:, 32 * c + l] >> 4) | (((qh[:, l] >> (2 * c + 1)) & 1) << 4)
    assert idx.max() == 31 and (idx >= 16).mean() > 0.2
    # the same block with the fifth bits cleared and the nibbles kept is a
    # valid Q4_K block (same header): Q5_K = Q4_K's value + 16 * d * sc
    q4 = np.concatenate([q[:, :16], q[:, 48:]], axis=1).reshape(-1)
    y5 = orc.dequantize(O.Q5_K, q.reshape(-1), x.size).reshape(-1, 256)
    y4 = orc.dequantize(O.Q4_K, q4, x.size).reshape(-1, 256)
    q0 = q.copy()
    q0[:, 16:48] = 0
    y50 = orc.dequantize(O.Q5_K, q0.reshape(-1), x.size).reshape(-1, 256)
    assert (y50 == y4).all()
    assert ((y5 != y4) == (idx >= 16)).all()


@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K])
def test_quantize_roundtrip_on_representable_values(orc, t):
    """Inputs that are exactly a block's dequantized values of a canonical
    block re-quantize to themselves (values stay representable)."""
    x = orc.normal(500 + t, 256 * 32, 0.02)
    y = orc.dequantize(t, orc.quantize(t, x), x.size)
    y2 = orc.dequantize(t, orc.quantize(t, y), x.size)
    y3 = orc.dequantize(t, orc.quantize(t, y2), x.size)
    # the fixed point is reached after at most one extra pass on >= 95% of values
    assert np.mean(y3 == y2) > 0.95


def test_oracle_regression_vectors(orc):
    import hashlib
    with open(os.path.join(GOLDEN, "oracle_vectors.json")) as f:
        g = json.load(f)
    for seed, vals in g["normal_first16"].items():
        assert (orc.normal(int(seed), 16, 1.0) == np.array(vals, np.float32)).all()
    for name, t in (("Q8_0", O.Q8_0), ("Q4_K", O.Q4_K), ("Q6_K", O.Q6_K)):
        e = g["blocks"][name]
        x = orc.normal(e["seed"], e["n"], e["sigma"])
        q = orc.quantize(t, x)
        assert q.tobytes().hex() == e["blocks_hex"]
        y = orc.dequantize(t, q, e["n"])
        assert (y.view(np.uint32) == np.array(e["dequant_f32_bits"], np.uint32)).all()
        big = orc.quantize(t, orc.normal(e["sha256_4096x16_seed"], 4096 * 16, 0.02))
        assert hashlib.sha256(big.tobytes()).hexdigest() == e["sha256_4096x16"]


def test_normal_generator_moments(orc):
    z = orc.normal(123, 1 << 20, 1.0)
    assert abs(z.mean()) < 5e-3
    assert abs(z.std() - 1.0) < 5e-3
    assert np.abs(z).max() <= 6.0
    assert (orc.normal(123, 10, 0.02) == (orc.normal(123, 10, 1.0) * np.float32(0.02)).astype(np.float32)).all()
    # offset addressing: sample i of the stream is the same wherever it is drawn
    assert (orc.normal(9, 100)[37:] == orc.normal(9, 63, 1.0, offset=37)).all()
