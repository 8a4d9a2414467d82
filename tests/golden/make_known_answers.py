"""Writes known_answers.json: the literal known answers that bitnet-tt's own
tests and hardware scripts state for the BitLinear path.

Every entry is data copied by value from the cited reference test (inputs and
the expected result the test asserts or prints); nothing here runs reference
code.  Paths are relative to the bitnet-tt repository root.

    python tests/golden/make_known_answers.py
"""

import json
import os

KNOWN = {
    "encode_values": {
        "src": "tests/test_ternary_kernel.py:31-34",
        "values": [-1, 0, 1, 0],
        "codes": [0b10, 0b00, 0b01, 0b00],
    },
    "decode_values": {
        "src": "tests/test_ternary_kernel.py:36-39",
        "codes": [0b10, 0b00, 0b01, 0b00],
        "values": [-1, 0, 1, 0],
    },
    "pack_roundtrip_two_bytes": {
        "src": "tests/test_ternary_kernel.py:51-56",
        "codes": [0b01, 0b10, 0b00, 0b01, 0b10, 0b00, 0b01, 0b10],
        "n_bytes": 2,
    },
    "pack_single_byte": {
        "src": "tests/test_ternary_kernel.py:58-62",
        "codes": [0b10, 0b01, 0b00, 0b10],
        "byte": 0b10_01_00_10,
    },
    "face_ordering": {
        "src": "tests/test_ternary_kernel.py:84-95",
        # (row, col, value) set in a zero 32x32 tile -> (face-flat index, value)
        "marks": [[0, 0, 1], [0, 16, 2], [16, 0, 3], [16, 16, 4]],
        "expect": [[0, 1], [256, 2], [512, 3], [768, 4]],
    },
    "all_zeros_tile": {
        "src": "tests/test_ternary_kernel.py:136-140",
        "out_features": 32, "in_features": 64, "scale": 0.5, "expect": 0.0,
    },
    "all_ones_tile": {
        "src": "tests/test_ternary_kernel.py:142-147",
        "out_features": 32, "in_features": 32, "scale": 0.25, "expect": 0.25,
    },
    "tile_counts": {
        "src": "tests/test_ternary_kernel.py:153-170",
        # [in_features, out_features, tiles]
        "cases": [[2560, 2560, 6400], [2560, 6912, 17280], [128, 64, 8]],
        "bf16_over_packed_min_ratio": 7.5,
    },
    "seeded_roundtrips": {
        "src": "tests/test_ternary_kernel.py:41-45, 64-72, 101-134",
        "encode_seed": 42, "tile_seed": 123, "matrix_seed": 7, "matrix_shape": [64, 128],
        "nonaligned_seed": 99, "nonaligned_shape": [50, 100],
    },
    "weight_sign": {
        "src": "tests/test_model.py:79-89",
        "weight": [[1.0, -1.0], [0.1, -0.1]],
        "q00": 1, "q01": -1,
    },
    "act_scale_known": {
        "src": "tests/test_model.py:91-102",
        "shape": [1, 1, 10], "x000": 127.0, "scale": 1.0, "atol": 0.01,
    },
    "act_range": {
        "src": "tests/test_bitlinear.py:70-97",
        "shape": [2, 16, 256], "qmin": -128, "qmax": 127,
    },
    "generic_op_all_plus_one": {
        "src": "test_generic_op_ternary.py:24-40",
        "M": 32, "K": 32, "N": 32, "act": 0.5, "weight": 1, "expect": 16.0,
    },
    "matmul_ones": {
        "src": "test_matmul_only.py:12-19",
        "M": 32, "K": 32, "N": 32, "act": 1.0, "weight": 1, "expect": 32.0,
    },
    "identity_readback": {
        "src": "test_ternary_bias_diag.py:101-119",
        "M": 32, "K": 32, "N": 32, "seed": 42,
    },
    "ffn_shapes": {
        "src": "test_ternary_bias_diag.py:279-309",
        "cases": [[32, 2560, 6912], [32, 6912, 2560]], "seed": 2024,
    },
    "fused_gate_up_builder": {
        "src": "tests/test_ffn_fused.py:11-49",
        "gate": [[1.2, -0.8, 0.1], [-0.7, 0.4, 0.0]],
        "up": [[0.5, -1.5, 0.25], [2.0, -0.1, -0.3], [0.0, 0.8, -0.9]],
        "fused_shape": [3, 5],
    },
    "fused_qkv_builder": {
        "src": "tests/test_projection_fusion.py:11-43",
        "q": [[1.0, -0.5, 0.25], [0.0, 2.0, -1.0]],
        "k": [[-1.25, 0.1, 0.7]],
        "v": [[0.6, -0.2, 0.4]],
        "fused_shape": [3, 4],
    },
    "bitnet_2b_dims": {
        "src": "src/bitnet_tt/config.py:13-48, 150-172",
        "hidden_size": 2560, "num_layers": 30, "num_attention_heads": 20, "num_key_value_heads": 5,
        "intermediate_size": 6912, "rms_norm_eps": 1e-5, "rope_theta": 500000.0, "head_dim": 128,
    },
}

if __name__ == "__main__":
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "known_answers.json")
    with open(out, "w") as f:
        json.dump(KNOWN, f, indent=1, sort_keys=True)
    print(out)
