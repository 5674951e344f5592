"""Writes reference_kats.json: the known-answer inputs and asserted outputs
held by the reference's own tests (literal values from
/root/reference/src/metal_runtime.rs and src/paged_kv.rs, cited per entry).
The reference is Rust + Metal and cannot run here, so these asserted values
and tolerances are the fixtures; nothing is computed by this script.

Usage: python tests/golden/make_reference_kats.py
"""
import json
from pathlib import Path

KATS = {
    "q4_k128_n5": {
        "source": "metal_runtime.rs:9332-9362 (q4_affine_matvec_matches_cpu_reference)",
        "K": 128, "N": 5,
        "input": "x[i] = ((i % 17) - 8) * 0.125",
        "nibbles": "q[i] = (i * 7 + 3) % 16 over the row-major N*K values",
        "scales_cycle": [0.125, -0.0625, 0.25, 0.03125, -0.125, 0.0625],
        "biases_cycle": [0.03125, -0.015625, 0.0625, 0.125, -0.03125, 0.0],
        "abs_tolerance": 1e-3,
    },
    "q8_attention_single_token": {
        "source": "metal_runtime.rs:11587-11605 (q8_gqa_attention_keeps_kv_on_the_gpu)",
        "kv_heads": 1, "head_dim": 2, "num_heads": 1,
        "query": [1.0, 0.0], "gate": [0.0, 0.0], "key": [1.0, 0.0], "value": [2.0, -1.0],
        "expected": [1.0, -0.503937], "tolerance": [0.001, 0.005],
        "expected_value_q8": [127, -64], "expected_value_scale": "2/127",
    },
    "q8_prefill_matches_steps": {
        "source": "metal_runtime.rs:11608-11682",
        "kv_heads": 1, "head_dim": 2, "num_heads": 2, "rows": 3,
        "queries": [1.0, 0.0, 0.25, -0.5, 0.5, 0.5, -0.75, 0.25, -0.2, 0.8, 0.6, -0.4],
        "gates": [0.0, 0.0, 0.1, -0.1, -0.2, 0.2, 0.0, 0.0, 0.3, -0.3, 0.15, 0.05],
        "keys": [1.0, 0.0, 0.4, 0.9, -0.7, 0.2],
        "values": [2.0, -1.0, 0.75, 1.25, -0.5, 0.4],
        "next_query": [0.9, -0.1, -0.3, 0.7], "next_gate": [0.05, -0.05, 0.2, -0.2],
        "next_key": [0.2, -0.6], "next_value": [1.1, -0.8],
        "tolerance": 0.005,
    },
    "deltanet_scalar_recurrence": {
        "source": "metal_runtime.rs:10913-10944",
        "config": [1, 1, 2, 2, 1],
        "qkv": [-0.5, 0.25, 0.75, -1.0, 0.2, -0.4], "z": [0.1, -0.2], "b": [0.3], "a": [-0.1],
        "a_log": [0.2], "dt_bias": [-0.3], "norm": [1.1, 0.9], "epsilon": 1e-6, "conv_weight": "all 1.0",
        "tolerance": 0.001,
    },
    "deltanet_prefill_matches_steps": {
        "source": "metal_runtime.rs:11202-11300",
        "config": [1, 1, 2, 2, 2],
        "qkv": [-0.5, 0.25, 0.75, -1.0, 0.2, -0.4, 0.1, -0.7, -0.2, 0.6, 0.9, 0.3,
                0.8, -0.1, 0.4, -0.5, -0.6, 0.7],
        "z": [0.1, -0.2, -0.3, 0.4, 0.5, -0.6], "b": [0.3, -0.4, 0.2], "a": [-0.1, 0.25, -0.35],
        "conv_weight": [0.2, 0.8, -0.1, 0.7, 0.3, 0.6, -0.2, 0.9, 0.15, 0.85, -0.25, 0.75],
        "a_log": [0.2], "dt_bias": [-0.3], "norm": [1.1, 0.9], "epsilon": 1e-6,
        "next_qkv": [-0.35, 0.45, 0.55, -0.15, 0.25, 0.65], "next_z": [0.2, -0.45],
        "next_b": [0.15], "next_a": [-0.05],
        "tolerance": 0.001,
    },
    "page_table": {
        "source": "paged_kv.rs:136-163",
        "page_tokens": 16,
        "cases": "append(n) materialises pages first..last of [start, start+n) with sequential ids; "
                 "page_for_token(t) is None at or beyond the length; ZeroCapacity, EmptyAppend, "
                 "CapacityExceeded errors",
    },
}

if __name__ == "__main__":
    out = Path(__file__).with_name("reference_kats.json")
    out.write_text(json.dumps(KATS, indent=1) + "\n")
    print(out)
