"""Writes the golden fixtures under tests/golden/.

* reference_kats.json -- known-answer vectors copied as data from the
  reference's own tests: fp16 -> f32 (crates/loader/src/safetensors_values.rs:
  316-351), bf16 -> f32 (:295-313), GGML type ids (gguf_inspect.rs:178-185)
  the GGUF fixture's ne-order shape and q4_k tag
  (fixtures/metadata/gemma4_e4b_it_q4_k_m_gguf_metadata.json), and the
  hand-checked rmsnorm / silu / gated-MLP values (crates/kernels/src/
  rmsnorm.rs:150-258, crates/kernels/src/mlp.rs:260-440).
* oracle_vectors.json -- regression vectors produced by the CPU oracle:
  the first values of the seeded generator and small quantized blocks with
  their dequantized values.  These pin the oracle against later edits; the
  oracle itself is pinned by the independent checks in tests/test_oracle_*.py.

Run from the repo root: python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import oracle as O  # noqa: E402


def reference_kats():
    return {
        "source": {
            "f16": "crates/loader/src/safetensors_values.rs:316-351",
            "bf16": "crates/loader/src/safetensors_values.rs:295-313",
            "type_ids": "crates/loader/src/gguf_inspect.rs:170-206",
            "gguf_fixture": "fixtures/metadata/gemma4_e4b_it_q4_k_m_gguf_metadata.json",
            "rmsnorm": "crates/kernels/src/rmsnorm.rs:150-258",
            "silu": "crates/kernels/src/mlp.rs:260-290",
            "mlp_gated_silu": "crates/kernels/src/mlp.rs:300-440",
        },
        # (bits, expected f32 bit pattern); 0x7e00 decodes to a NaN
        "f16": [[0x3C00, 0x3F800000], [0xC100, 0xC0200000], [0x0000, 0x00000000], [0x0400, 0x38800000],
                [0x0001, 0x33800000], [0x7C00, 0x7F800000]],
        "f16_nan": [0x7E00],
        "bf16": [[0x3F80, 0x3F800000], [0xC020, 0xC0200000], [0x0000, 0x00000000], [0x7F80, 0x7F800000]],
        "type_ids": {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8, "Q2K": 10,
                     "Q3K": 11, "Q4K": 12, "Q5K": 13, "Q6K": 14, "BF16": 30},
        "gguf_fixture_token_embd": {"name": "token_embd.weight", "shape": [2560, 262144], "tensor_type": "q4_k"},
        # rows x hidden input, weight, epsilon, expected output, absolute tolerance
        "rmsnorm": [
            {"x": [1, 2, 3], "rows": 1, "hidden": 3, "w": [1, 1, 1], "eps": 1e-6,
             "want": [0.46291006, 0.9258201, 1.3887302], "tol": 1e-6},
            {"x": [1, 2, 3], "rows": 1, "hidden": 3, "w": [2, 0.5, 1], "eps": 1e-6,
             "want": [0.9258201, 0.46291006, 1.3887302], "tol": 1e-6},
            {"x": [0, 0, 0, 0], "rows": 1, "hidden": 4, "w": [1.5, 2.5, 3.5, 4.5], "eps": 1e-6,
             "want": [0, 0, 0, 0], "tol": 0.0},
            {"x": [5], "rows": 1, "hidden": 1, "w": [1], "eps": 0.0, "want": [1.0], "tol": 1e-6},
            {"x": [1, 2, 3, 2, 4, 6], "rows": 2, "hidden": 3, "w": [1, 1, 1], "eps": 1e-6,
             "want": [0.46291006, 0.9258201, 1.3887302, 0.46291006, 0.9258201, 1.3887302], "tol": 1e-6},
        ],
        "silu": {"x": [0, 1, -1, 2, 3], "want": [0, 0.7310586, -0.26894143, 1.7615942, 2.8577223], "tol": 1e-6,
                 "asymptotes": {"x": [-30, 30], "want": [0, 30], "tol": [1e-6, 1e-3]}},
        # weights in the reference's [in, out] layout (mlp.rs:22-25), flattened row-major
        "mlp_gated_silu": {"x": [1, 2, 0, 0], "rows": 2, "hidden": 2, "intermediate": 4,
                           "gate_w": [1, 0, 1, -1, 0, 1, 1, 0], "up_w": [1, 1, 0, 2, 1, -1, 1, 0],
                           "down_w": [1, 0, 0, 1, 1, 0, 0, 1],
                           "want": [7.9086204, -2.299477, 0, 0], "tol": 1e-5},
    }


def oracle_vectors(o):
    seeds = [0, 1, 0x5EED, 2**63 + 12345]
    rng = {str(s): [float(v) for v in o.normal(s, 16, 1.0)] for s in seeds}
    blocks = {}
    for t, name in ((O.Q8_0, "Q8_0"), (O.Q4_K, "Q4_K"), (O.Q6_K, "Q6_K")):
        x = o.normal(1000 + t, 512, 0.02)
        q = o.quantize(t, x)
        y = o.dequantize(t, q, 512)
        big = o.quantize(t, o.normal(2000 + t, 4096 * 16, 0.02))
        blocks[name] = {
            "seed": 1000 + t, "n": 512, "sigma": 0.02,
            "blocks_hex": q.tobytes().hex(),
            "dequant_f32_bits": [int(v) for v in y.view(np.uint32)],
            "sha256_4096x16_seed": 2000 + t,
            "sha256_4096x16": hashlib.sha256(big.tobytes()).hexdigest(),
        }
    # the block formats without a quantizer here: seeded random bytes (f16
    # fields kept finite) and their dequantized values
    raw = {}
    for t in (O.Q4_0, O.Q4_1, O.Q5_0, O.Q5_1, O.Q2_K, O.Q3_K, O.Q5_K):
        nb = 4 if O.BLOCK_ELEMS[t] == 256 else 16
        b = finite_random_blocks(t, nb, 3000 + t)
        y = o.dequantize(t, b, nb * O.BLOCK_ELEMS[t])
        raw[O.TYPE_NAMES[t]] = {"type": t, "blocks_hex": b.tobytes().hex(),
                                "dequant_f32_bits": [int(v) for v in y.view(np.uint32)]}
    return {"generator": "SplitMix64 + Irwin-Hall(12), okr_normal_at", "normal_first16": rng, "blocks": blocks,
            "raw_blocks": raw}


# byte offsets of the f16 fields (d, and dmin or m) in each block format
F16_FIELDS = {O.Q4_0: (0,), O.Q4_1: (0, 2), O.Q5_0: (0,), O.Q5_1: (0, 2), O.Q8_0: (0,), O.Q2_K: (80, 82),
              O.Q3_K: (108,), O.Q4_K: (0, 2), O.Q5_K: (0, 2), O.Q6_K: (208,)}


def finite_random_blocks(t, nb, seed):
    """nb random blocks of type t whose f16 fields are finite values of
    moderate size (exponent field 1..20), so every element is finite."""
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (nb, O.BLOCK_BYTES[t]), dtype=np.uint8)
    for off in F16_FIELDS[t]:
        h = rng.integers(0, 1 << 16, nb).astype(np.uint16)
        h = (h & 0x83FF) | (rng.integers(1, 21, nb).astype(np.uint16) << 10)
        b[:, off] = h & 0xFF
        b[:, off + 1] = h >> 8
    return b.reshape(-1)


if __name__ == "__main__":
    O.build()
    o = O.Oracle()
    with open(os.path.join(HERE, "reference_kats.json"), "w") as f:
        json.dump(reference_kats(), f, indent=1)
    with open(os.path.join(HERE, "oracle_vectors.json"), "w") as f:
        json.dump(oracle_vectors(o), f, indent=1)
    print("wrote", os.listdir(HERE))
