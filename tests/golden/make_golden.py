"""Writes tests/golden/paged_decode_golden.json (run: python tests/golden/make_golden.py).

Contents are data only:
  * the reference's known-answer tests for this path, restated as inputs and
    expected values: crates/loom-kernels/src/tests/attention_tests.rs:4-118
    (closed-form expectation (1 + 10e + 20e^2) / (1 + e + e^2); single token
    returns V exactly; metadata errors leave the output untouched) and the
    FP8 E4M3FN table of crates/loom-kernels/src/tests/norm_tests.rs:119-139;
  * the two closed-form-input GPU-vs-oracle cases of
    crates/loom-cuda/src/attention_dispatch.rs:486-606, with expected outputs
    from the independent numpy dense restatement in tests/brute.py (F64).
Nothing here imports or runs the reference.
"""

from __future__ import annotations

import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from brute import paged_attention  # noqa: E402


def affine_values(n, mod, center, step):
    """F32 values (i % mod - center) * step of the flat index i (mod None: i - center)."""
    idx = np.arange(n, dtype=np.float32)
    if mod is not None:
        idx = idx % np.float32(mod)
    return ((idx - np.float32(center)) * np.float32(step)).astype(np.float32)


def main():
    e = math.e
    golden = {
        "attention_kat": [
            {
                "name": "block_indirection_and_gqa_mapping",
                "source": "crates/loom-kernels/src/tests/attention_tests.rs:4-30",
                "spec": [1, 2, 1, 1, 1, 2, 2, 2, 4, 1.0, "f32"],
                "query": [1.0, 1.0],
                "key_cache": [2.0, 99.0, 0.0, 1.0],
                "value_cache": [20.0, 99.0, 1.0, 10.0],
                "block_tables": [1, 0],
                "sequence_lengths": [3],
                "expected": [(1 + 10 * e + 20 * e * e) / (1 + e + e * e)] * 2,
                "tolerance": 1e-6,
            },
            {
                "name": "low_precision_and_distinct_value_width",
                "source": "crates/loom-kernels/src/tests/attention_tests.rs:32-56",
                "spec": [1, 1, 1, 2, 3, 1, 1, 1, 1, 0.5, "bf16"],
                "query": [2.0, -1.0],
                "key_cache": [4.0, 3.0],
                "value_cache": [1.25, -2.5, 7.0],
                "block_tables": [0],
                "sequence_lengths": [1],
                "expected": [1.25, -2.5, 7.0],
                "tolerance": 0.0,
            },
        ],
        "attention_errors": {
            "source": "crates/loom-kernels/src/tests/attention_tests.rs:58-118",
            "spec_errors": [
                {"spec": [1, 3, 2, 4, 4, 1, 16, 1, 16, 0.5, "f16"], "kind": "HeadCountNotDivisible",
                 "fields": {"query_heads": 3, "kv_heads": 2}},
                {"spec": [1, 2, 1, 4, 4, 1, 16, 1, 16, 0.0, "f16"], "kind": "InvalidScale",
                 "fields": {"scale": 0.0}},
            ],
            "buffer_spec": [2, 1, 1, 1, 1, 2, 2, 2, 4, 1.0, "f32"],
            "query": [1.0, 1.0],
            "key_cache": [1.0] * 4,
            "value_cache": [2.0] * 4,
            "sentinel": -7.0,
            "cases": [
                {"block_tables": [0, 1, 1, -1], "sequence_lengths": [3, 5],
                 "kind": "SequenceLengthOutOfBounds", "fields": {"sequence": 1, "length": 5, "capacity": 4}},
                {"block_tables": [0, 2, 1, -1], "sequence_lengths": [3, 1],
                 "kind": "BlockIdOutOfBounds",
                 "fields": {"sequence": 0, "logical_block": 1, "block_id": 2, "num_blocks": 2}},
            ],
        },
        "fp8_kat": {
            "source": "crates/loom-kernels/src/tests/norm_tests.rs:119-139",
            "encode": [[0.0, 0x00], [-0.0, 0x80], [1.0, 0x38], [-1.0, 0xB8], [448.0, 0x7E],
                       [500.0, 0x7E], [2.0 ** -9, 0x01], [1.0625, 0x38], [1.1875, 0x3A]],
            "encode_nan": 0x7F,
            "decode": [[0x38, 1.0], [0x7E, 448.0]],
        },
        "affine_cases": [],
    }

    # attention_dispatch.rs:486-606: inputs are affine functions of the flat
    # element index, value(i) = (i % mod - center) * step in F32 (mod = None:
    # no modulus); only their parameters and the expected outputs are stored.
    for name, spec, qg, kg, vg, tables, lens in [
        ("safe_rust_wrapper_matches_the_cpu_oracle", (2, 4, 2, 4, 3, 4, 2, 2, 4, 0.5),
         (None, 9.0, 0.07), (13, 6.0, 0.11), (17, 8.0, 0.09), [2, 0, 1, 3], [3, 2]),
        ("caller_owned_split_k_workspace_matches_the_cpu_oracle", (1, 4, 1, 128, 128, 8, 16, 8, 128, 0.125),
         (29, 14.0, 0.013), (37, 18.0, 0.011), (41, 20.0, 0.009), list(range(8)), [128]),
    ]:
        B, Hq, Hkv, D, Dv, NB, bs, maxb, maxlen, scale = spec
        q = affine_values(B * Hq * D, *qg).reshape(B, Hq, D)
        k = affine_values(NB * bs * Hkv * D, *kg).reshape(NB, bs, Hkv, D)
        v = affine_values(NB * bs * Hkv * Dv, *vg).reshape(NB, bs, Hkv, Dv)
        t = np.array(tables, dtype=np.int64).reshape(B, maxb)
        out, lse = paged_attention(q, k, v, t, lens, np.float32(scale), bs)
        golden["affine_cases"].append({
            "name": name,
            "source": "crates/loom-cuda/src/attention_dispatch.rs:486-606",
            "spec": [B, Hq, Hkv, D, Dv, NB, bs, maxb, maxlen, scale],
            "query_affine": list(qg),
            "key_affine": list(kg),
            "value_affine": list(vg),
            "block_tables": tables,
            "sequence_lengths": lens,
            "expected": out.ravel().tolist(),
            "expected_lse": lse.ravel().tolist(),
        })

    path = os.path.join(HERE, "paged_decode_golden.json")
    with open(path, "w") as f:
        json.dump(golden, f)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
