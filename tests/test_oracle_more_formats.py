"""Pins the CPU oracle's decoders for the block formats served by dequantize
and the quantized row gather only (CPU only): Q4_0, Q4_1, Q5_0, Q5_1, Q2_K,
Q3_K and Q5_K (type ids 2, 3, 6, 7, 10, 11, 13 of GgmlTensorType::from_raw,
crates/loader/src/gguf_inspect.rs:170-206).

The reference holds no value of any of these formats, so, as for Q8_0 / Q4_K /
Q6_K, the pins are:
  * agreement bit for bit with the independent numpy bit-field decoder on
    random bytes;
  * closed forms built from the spec's field positions (unit scales give the
    raw quant, a zero scale isolates the min, offsets -8 / -16 / -32 / -4);
  * element-order probes through every bit plane (low bits, the Q5 formats'
    32-bit high word, Q3_K's hmask, Q5_K's qh) -- a single set bit at position
    p must land at y[p] and nowhere else;
  * the Q3_K 6-bit scale unpack exhaustively over both bytes feeding each of
    the 16 scales;
  * committed regression vectors (tests/golden/oracle_vectors.json).
A misreading of the spec shared by the C decoder, the numpy decoder and these
builders would not be caught: parity with ggml itself is unpinned (no ggml
code or GGUF payload is available here).
"""
import json
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
NEW = (O.Q4_0, O.Q4_1, O.Q5_0, O.Q5_1, O.Q2_K, O.Q3_K, O.Q5_K)


def _f16(v):
    return int(np.float16(v).view(np.uint16))


def _put16(b, off, bits):
    b[off], b[off + 1] = bits & 0xFF, bits >> 8


def _bits_same(a, b):
    a = np.asarray(a, np.float32).reshape(-1)
    b = np.asarray(b, np.float32).reshape(-1)
    return (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))


# ---- block builders from the spec's field positions ---------------------------

def legacy_block(t, d, v, m=0):
    """Q4_0/Q4_1/Q5_0/Q5_1 block with stored quants v[0..31] (4 or 5 bits,
    before any offset), f16 bits d (and m for the _1 formats)."""
    v = np.asarray(v, np.int64)
    b = np.zeros(O.BLOCK_BYTES[t], np.uint8)
    _put16(b, 0, d)
    off = 2
    if t in (O.Q4_1, O.Q5_1):
        _put16(b, 2, m)
        off = 4
    if t in (O.Q5_0, O.Q5_1):
        qh = 0
        for e in range(32):
            qh |= int((v[e] >> 4) & 1) << e
        b[off:off + 4] = np.frombuffer(qh.to_bytes(4, "little"), np.uint8)
        off += 4
    for j in range(16):
        b[off + j] = (v[j] & 15) | ((v[j + 16] & 15) << 4)
    return b


def q2k_block(d, dmin, sc, q):
    """sc: 16 scale bytes (low nibble scale, high nibble min); q: 256 2-bit."""
    b = np.zeros(84, np.uint8)
    b[0:16] = np.asarray(sc, np.uint8)
    for e in range(256):
        h, r = divmod(e, 128)
        j, s = divmod(r, 32)
        b[16 + 32 * h + s] |= (int(q[e]) & 3) << (2 * j)
    _put16(b, 80, d)
    _put16(b, 82, dmin)
    return b


def q3k_pack_scales(sc6):
    s = np.zeros(12, np.uint8)
    for i in range(16):
        v = int(sc6[i]) & 63
        if i < 8:
            s[i] |= v & 15
        else:
            s[i - 8] |= (v & 15) << 4
        s[8 + i % 4] |= (v >> 4) << (2 * (i // 4))
    return s


def q3k_block(d, sc6, q2, hbit):
    """sc6: 16 stored 6-bit scales (value - 32 is used); q2: 256 low 2-bit
    quants; hbit: 256 hmask bits (a clear bit subtracts 4)."""
    b = np.zeros(110, np.uint8)
    for e in range(256):
        h, r = divmod(e, 128)
        j, s = divmod(r, 32)
        b[32 + 32 * h + s] |= (int(q2[e]) & 3) << (2 * j)
        b[s] |= (int(hbit[e]) & 1) << (4 * h + j)
    b[96:108] = q3k_pack_scales(sc6)
    _put16(b, 108, d)
    return b


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


def q5k_block(d, dmin, sc, m, v):
    """v: 256 stored 5-bit quants."""
    b = np.zeros(176, np.uint8)
    _put16(b, 0, d)
    _put16(b, 2, dmin)
    b[4:16] = _q4k_pack_scales(sc, m)
    for e in range(256):
        c, r = divmod(e, 64)
        hi, l = divmod(r, 32)
        b[48 + 32 * c + l] |= (int(v[e]) & 15) << (4 * hi)
        b[16 + l] |= ((int(v[e]) >> 4) & 1) << (2 * c + hi)
    return b


# ---- tests ---------------------------------------------------------------------

def test_type_ids_and_block_sizes_of_the_other_formats():
    with open(os.path.join(GOLDEN, "reference_kats.json")) as f:
        ids = json.load(f)["type_ids"]
    assert (ids["Q4_0"], ids["Q4_1"], ids["Q5_0"], ids["Q5_1"], ids["Q2K"], ids["Q3K"], ids["Q5K"]) == NEW
    # block bytes from the field lists of the spec: f16 fields + quant bytes
    assert O.BLOCK_BYTES[O.Q4_0] == 2 + 32 // 2
    assert O.BLOCK_BYTES[O.Q4_1] == 2 + 2 + 32 // 2
    assert O.BLOCK_BYTES[O.Q5_0] == 2 + 4 + 32 // 2
    assert O.BLOCK_BYTES[O.Q5_1] == 2 + 2 + 4 + 32 // 2
    assert O.BLOCK_BYTES[O.Q2_K] == 16 + 256 // 4 + 2 + 2
    assert O.BLOCK_BYTES[O.Q3_K] == 256 // 8 + 256 // 4 + 12 + 2
    assert O.BLOCK_BYTES[O.Q5_K] == 2 + 2 + 12 + 256 // 8 + 256 // 2
    assert all(O.BLOCK_ELEMS[t] == (32 if t in (O.Q4_0, O.Q4_1, O.Q5_0, O.Q5_1) else 256) for t in NEW)


@pytest.mark.parametrize("t", NEW, ids=[O.TYPE_NAMES[t] for t in NEW])
def test_dequant_c_matches_numpy_on_random_bytes(orc, t):
    rng = np.random.default_rng(200 + t)
    nb = 2000
    blocks = rng.integers(0, 256, nb * O.BLOCK_BYTES[t], dtype=np.uint8)
    with np.errstate(all="ignore"):
        assert _bits_same(orc.dequantize(t, blocks, nb * O.BLOCK_ELEMS[t]), O.NP_DEQUANT[t](blocks)).all()


def test_legacy_closed_forms(orc):
    rng = np.random.default_rng(7)
    v4 = rng.integers(0, 16, 32)
    v5 = rng.integers(0, 32, 32)
    for e in (0, -3, 4):
        d = _f16(2.0 ** e)
        y = orc.dequantize(O.Q4_0, legacy_block(O.Q4_0, d, v4), 32)
        assert (y == ((v4 - 8) * 2.0 ** e).astype(np.float32)).all()
        y = orc.dequantize(O.Q5_0, legacy_block(O.Q5_0, d, v5), 32)
        assert (y == ((v5 - 16) * 2.0 ** e).astype(np.float32)).all()
    # _1 formats: y = v*d + m, exact for these d and m
    for dv, mv in ((1.0, 0.0), (0.25, 0.5), (1.0, -8.0)):
        y = orc.dequantize(O.Q4_1, legacy_block(O.Q4_1, _f16(dv), v4, _f16(mv)), 32)
        assert (y == (v4 * dv + mv).astype(np.float32)).all()
        y = orc.dequantize(O.Q5_1, legacy_block(O.Q5_1, _f16(dv), v5, _f16(mv)), 32)
        assert (y == (v5 * dv + mv).astype(np.float32)).all()


def test_q2_k_closed_forms(orc):
    rng = np.random.default_rng(8)
    q = rng.integers(0, 4, 256)
    # scale 1, min 0: y = q
    b = q2k_block(_f16(1.0), 0, [0x01] * 16, q)
    assert (orc.dequantize(O.Q2_K, b, 256) == q.astype(np.float32)).all()
    # arbitrary scale bytes, d = dmin = 1: y = (sc & 15) * q - (sc >> 4), per 16-element group
    sc = rng.integers(0, 256, 16)
    b = q2k_block(_f16(1.0), _f16(1.0), sc, q)
    want = (np.repeat(sc & 15, 16) * q - np.repeat(sc >> 4, 16)).astype(np.float32)
    assert (orc.dequantize(O.Q2_K, b, 256) == want).all()
    # d = 0 isolates the min term; dmin = 2^-3 scales it
    b = q2k_block(0, _f16(0.125), sc, q)
    assert (orc.dequantize(O.Q2_K, b, 256) == (-np.repeat(sc >> 4, 16) * 0.125).astype(np.float32)).all()


def test_q3_k_closed_forms(orc):
    rng = np.random.default_rng(9)
    q2 = rng.integers(0, 4, 256)
    hb = rng.integers(0, 2, 256)
    # stored scale 33 (= +1), d = 1: y = q2 - 4 * (1 - hbit)
    b = q3k_block(_f16(1.0), [33] * 16, q2, hb)
    assert (orc.dequantize(O.Q3_K, b, 256) == (q2 - 4 * (1 - hb)).astype(np.float32)).all()
    # arbitrary 6-bit scales, d = 2^-2: y = (sc - 32) * 0.25 * q
    sc = rng.integers(0, 64, 16)
    b = q3k_block(_f16(0.25), sc, q2, hb)
    want = (np.repeat(sc - 32, 16) * 0.25 * (q2 - 4 * (1 - hb))).astype(np.float32)
    assert (orc.dequantize(O.Q3_K, b, 256) == want).all()


def test_q5_k_closed_forms(orc):
    rng = np.random.default_rng(10)
    v = rng.integers(0, 32, 256)
    b = q5k_block(_f16(1.0), 0, [1] * 8, [0] * 8, v)
    assert (orc.dequantize(O.Q5_K, b, 256) == v.astype(np.float32)).all()
    m = rng.integers(0, 64, 8)
    sc = rng.integers(0, 64, 8)
    b = q5k_block(_f16(1.0), _f16(1.0), sc, m, v)
    want = (np.repeat(sc, 32) * v - np.repeat(m, 32)).astype(np.float32)
    assert (orc.dequantize(O.Q5_K, b, 256) == want).all()


def _probe_blocks(t, p, plane):
    """Block of type t whose element p alone is non-zero.  plane 0 sets p's
    lowest quant bit; plane 1 its high bit (Q5 qh word, Q3_K hmask, Q5_K qh)."""
    n = O.BLOCK_ELEMS[t]
    one = _f16(1.0)
    if t in (O.Q4_0, O.Q4_1, O.Q5_0, O.Q5_1):
        zero = {O.Q4_0: 8, O.Q4_1: 0, O.Q5_0: 16, O.Q5_1: 0}[t]
        v = np.full(n, zero, np.int64)
        v[p] = zero + (1 if plane == 0 else 16) if t != O.Q5_0 else (17 if plane == 0 else 0)
        return legacy_block(t, one, v)
    if t == O.Q2_K:
        q = np.zeros(n, np.int64)
        q[p] = 1 if plane == 0 else 2
        return q2k_block(one, 0, [1] * 16, q)
    if t == O.Q3_K:
        q2 = np.zeros(n, np.int64)
        hb = np.ones(n, np.int64)
        if plane == 0:
            q2[p] = 1
        else:
            hb[p] = 0
        return q3k_block(one, [33] * 16, q2, hb)
    v = np.zeros(n, np.int64)
    v[p] = 1 if plane == 0 else 16
    return q5k_block(one, 0, [1] * 8, [0] * 8, v)


@pytest.mark.parametrize("t", NEW, ids=[O.TYPE_NAMES[t] for t in NEW])
def test_element_order_probe(orc, t):
    n = O.BLOCK_ELEMS[t]
    has_high = t in (O.Q5_0, O.Q5_1, O.Q2_K, O.Q3_K, O.Q5_K)
    for plane in ((0, 1) if has_high else (0,)):
        blocks = np.stack([_probe_blocks(t, p, plane) for p in range(n)])
        y = orc.dequantize(t, blocks, n * n).reshape(n, n)
        val = {0: 1.0, 1: {O.Q5_0: -16.0, O.Q5_1: 16.0, O.Q2_K: 2.0, O.Q3_K: -4.0, O.Q5_K: 16.0}.get(t)}[plane]
        assert (y == np.eye(n, dtype=np.float32) * np.float32(val)).all(), (O.TYPE_NAMES[t], plane)
        assert _bits_same(y, O.NP_DEQUANT[t](blocks)).all()


def test_q3_k_scale_unpack_exhaustive(orc):
    """Every value of the two bytes feeding each of the 16 six-bit scales;
    every quant is +1 (q2 = 1, hmask set), d = 1, so y[16i] = scale_i - 32.
    Checked against the bit-by-bit numpy field extractor and the packer."""
    base = np.zeros(110, np.uint8)
    base[0:32] = 0xFF                   # hmask: every bit set
    base[32:96] = 0x55                  # every 2-bit quant = 1
    _put16(base, 108, _f16(1.0))
    combos = np.arange(1 << 16)
    for i in range(16):
        lo_byte = i if i < 8 else i - 8
        blocks = np.tile(base, (combos.size, 1))
        blocks[:, 96 + lo_byte] = combos & 0xFF
        blocks[:, 96 + 8 + i % 4] = combos >> 8
        y = orc.dequantize(O.Q3_K, blocks.reshape(-1), combos.size * 256).reshape(-1, 256)[:, 16 * i]
        field = O._q3k_field(blocks[:, 96:108], i)
        assert (y == (field - 32).astype(np.float32)).all(), i
        nib = (combos & 0xFF) >> (0 if i < 8 else 4) & 15
        top = (combos >> 8) >> (2 * (i // 4)) & 3
        assert (field == (nib | (top << 4))).all(), i
    # the packer used by the closed forms is the inverse of the unpack
    rng = np.random.default_rng(11)
    for _ in range(100):
        sc = rng.integers(0, 64, 16)
        s = q3k_pack_scales(sc)
        assert [int(O._q3k_field(s[None, :], i)[0]) for i in range(16)] == list(sc)


def test_regression_vectors_of_the_other_formats(orc):
    with open(os.path.join(GOLDEN, "oracle_vectors.json")) as f:
        raw = json.load(f)["raw_blocks"]
    assert sorted(raw) == sorted(O.TYPE_NAMES[t] for t in NEW)
    for name, e in raw.items():
        t = e["type"]
        b = np.frombuffer(bytes.fromhex(e["blocks_hex"]), np.uint8)
        n = b.size // O.BLOCK_BYTES[t] * O.BLOCK_ELEMS[t]
        y = orc.dequantize(t, b, n)
        assert (y.view(np.uint32) == np.array(e["dequant_f32_bits"], np.uint32)).all(), name
        assert np.isfinite(y).all()
