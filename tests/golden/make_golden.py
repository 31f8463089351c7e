"""Write tests/golden/reference_known_answers.json.

Every vector here is transcribed from a test in the aiqubits/quantinfer
source tree (cited per entry); nothing is imported or run from it. The
fixture is data: inputs, blocks and the expected result or bound that the
reference test asserts.

Run: python tests/golden/make_golden.py
"""
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))


def known_answers():
    cases = []
    # backends/cpu/src/tests.rs:8-15 (F32 matmul)
    cases.append({
        "name": "f32_matrix_product", "source": "backends/cpu/src/tests.rs:8-15",
        "op": "matmul_f32", "lhs_shape": [2, 3], "lhs": [1.0, 2.0, 3.0, 4.0, 5.0, 6.0],
        "rhs_shape": [3, 2], "rhs": [1.0, 2.0, 3.0, 4.0, 5.0, 6.0],
        "expect": "equal", "expected": [22.0, 28.0, 49.0, 64.0]})
    # backends/cpu/src/tests.rs:17-27
    cases.append({
        "name": "q8_0_ones_scale_two", "source": "backends/cpu/src/tests.rs:17-27",
        "op": "matmul_row_major", "qtype": "q8_0", "lhs_shape": [1, 32], "lhs_fill": 1.0,
        "rhs_shape": [32, 1], "blocks": [{"scale": 2.0, "values": [1] * 32}],
        "expect": "equal", "expected": [64.0]})
    # backends/cpu/src/tests.rs:29-43
    cases.append({
        "name": "q4_0_code_eight_is_zero", "source": "backends/cpu/src/tests.rs:29-43",
        "op": "matmul_row_major", "qtype": "q4_0", "lhs_shape": [1, 32], "lhs_fill": 1.0,
        "rhs_shape": [32, 1], "blocks": [{"scale": 1.0, "values": [8] * 32}],
        "expect": "equal", "expected": [0.0]})
    # backends/cpu/src/tests.rs:45-61
    cases.append({
        "name": "q4_k_0x99", "source": "backends/cpu/src/tests.rs:45-61",
        "op": "matmul_row_major", "qtype": "q4_k", "lhs_shape": [1, 256], "lhs_fill": 1.0,
        "rhs_shape": [256, 1],
        "blocks": [{"scale": 0.1, "min_scale": 0.0, "scales": [63] * 12, "values": [0x99] * 128}],
        "expect": "greater", "bound": 200.0})
    # backends/cpu/src/tests.rs:116-133
    cases.append({
        "name": "q5_k_0x99", "source": "backends/cpu/src/tests.rs:116-133",
        "op": "matmul_row_major", "qtype": "q5_k", "lhs_shape": [1, 256], "lhs_fill": 1.0,
        "rhs_shape": [256, 1],
        "blocks": [{"scale": 0.1, "min_scale": 0.0, "scales": [63] * 12, "high_bits": [0] * 32,
                    "values": [0x99] * 128}],
        "expect": "greater", "bound": 200.0})
    # backends/cpu/src/tests.rs:63-114: output rows bit-equal to row major
    cases.append({
        "name": "k_quant_output_rows_equal_row_major", "source": "backends/cpu/src/tests.rs:63-114",
        "op": "output_rows_equals_row_major", "lhs_shape": [1, 256], "lhs_fill": 1.0,
        "rhs_shape": [256, 1],
        "variants": [
            {"qtype": "q4_k", "blocks": [{"scale": 0.1, "min_scale": 0.0, "scales": [63] * 12,
                                          "values": [0x11] * 128}]},
            {"qtype": "q5_k", "blocks": [{"scale": 0.1, "min_scale": 0.0, "scales": [63] * 12,
                                          "high_bits": [0] * 32, "values": [0x11] * 128}]},
            {"qtype": "q6_k", "blocks": [{"scale": 0.1, "scales": [1] * 16,
                                          "low_bits": [0x11] * 128, "high_bits": [0] * 64}]},
        ]})
    # backends/cpu/src/tests.rs:209-257: SIMD output rows within 1e-4 of scalar
    cases.append({
        "name": "simd_output_rows_match_scalar", "source": "backends/cpu/src/tests.rs:209-257",
        "op": "simd_vs_scalar", "lhs_shape": [3, 32],
        "lhs": [i / 17.0 - 2.0 for i in range(96)], "rhs_shape": [32, 3],
        "q8_blocks": [{"scale": 0.13 + c * 0.07,
                       "values": [((i % 128) % 15) - 7 for i in range(32)]} for c in range(3)],
        "q4_blocks": [{"scale": 0.21 + c * 0.03, "values": [i % 16 for i in range(32)]}
                      for c in range(3)],
        "expect": "abs", "tolerance": 1e-4})
    # backends/cpu/src/tests.rs:259-278: threaded Q8 matmul bit-equal to scalar
    cases.append({
        "name": "threaded_q8_equals_scalar", "source": "backends/cpu/src/tests.rs:259-278",
        "op": "threaded_vs_scalar", "qtype": "q8_0", "lhs_shape": [8, 32], "lhs_fill": 1.0,
        "rhs_shape": [32, 1], "blocks": [{"scale": 0.5, "values": [1] * 32}], "threads": 4,
        "expect": "equal", "expected": [16.0] * 8})
    return cases


def wire_vectors():
    # format/src/gguf/tests.rs:163-212
    q4_values = [i % 16 for i in range(32)]
    standard_q6 = [0x12] * 128 + [0x34] * 64 + [0xFE] * 16 + [0x00, 0x38]
    legacy_q4 = [0x00, 0x38, 0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE,
                 0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE]
    legacy_q6 = standard_q6[208:] + standard_q6[192:208] + standard_q6[:192]
    return [
        {"name": "q4_0_standard_and_legacy", "source": "format/src/gguf/tests.rs:163-212",
         "qtype": "q4_0", "block": {"scale": 0.5, "values": q4_values},
         "legacy_bytes": legacy_q4},
        {"name": "q6_k_standard_and_legacy", "source": "format/src/gguf/tests.rs:163-212",
         "qtype": "q6_k",
         "block": {"scale": 0.5, "scales": [-2] * 16, "low_bits": [0x12] * 128,
                   "high_bits": [0x34] * 64},
         "standard_bytes": standard_q6, "legacy_bytes": legacy_q6},
        {"name": "q4_k_round_trip_144", "source": "format/src/gguf/tests.rs:214-231",
         "qtype": "q4_k",
         "block": {"scale": 0.125, "min_scale": 0.25, "scales": [63] * 12,
                   "values": [0x21] * 128},
         "wire_size": 144},
        {"name": "f16_half_is_0x3800", "source": "format/src/gguf/tests.rs:191",
         "f32": 0.5, "f16_le_bytes": [0x00, 0x38]},
    ]


def quantizer_bounds():
    return [
        # quant/src/lib.rs:39-48
        {"name": "q8_0_ramp", "source": "crates/quantinfer-quant/src/lib.rs:39-48",
         "qtype": "q8_0", "input": [float(v) for v in range(32)],
         "check": "abs_at", "index": 31, "target": 31.0, "bound": 0.3},
        # quant/src/lib.rs:66-87
        {"name": "q4_0_ramp", "source": "crates/quantinfer-quant/src/lib.rs:66-87",
         "qtype": "q4_0", "input": [v / 4.0 - 4.0 for v in range(32)],
         "check": "max_abs", "bound": 0.4},
        # quant/src/lib.rs:123-135
        {"name": "q4_k_ramp", "source": "crates/quantinfer-quant/src/lib.rs:123-135",
         "qtype": "q4_k", "input": [i / 128.0 - 1.0 for i in range(256)],
         "check": "max_abs", "bound": 0.2},
        # quant/src/lib.rs:137-148
        {"name": "q6_k_ramp", "source": "crates/quantinfer-quant/src/lib.rs:137-148",
         "qtype": "q6_k", "input": [i / 128.0 - 1.0 for i in range(256)],
         "check": "max_abs", "bound": 0.2},
        # quant schemes/k_grid_tests.rs:158-179: sub-grid loss
        {"name": "k_quant_subgrid_loss", "source": "quant/src/schemes/k_grid_tests.rs:158-179",
         "qtypes": ["q4_k", "q5_k", "q6_k"], "input_fill": 1.0e-8, "n": 256,
         "check": "all_zero_and_rel_l2_one"},
        # quant schemes/k_grid_tests.rs:182-196: subnormal f16 scales still resolve
        {"name": "k_quant_subnormal_scale", "source": "quant/src/schemes/k_grid_tests.rs:182-196",
         "qtypes": ["q4_k", "q5_k", "q6_k"], "input_fill": 5.0e-7, "n": 256,
         "check": "rel_l2_below", "bound": 0.1},
        # quant schemes/k_grid_tests.rs:148-155: f32::MAX has no finite f16 scale
        {"name": "k_quant_reject_f32_max", "source": "quant/src/schemes/k_grid_tests.rs:148-155",
         "qtypes": ["q4_k", "q5_k", "q6_k"], "input_fill": 3.4028234663852886e38, "n": 256,
         "check": "rejected"},
        # quant/src/lib.rs:50-64
        {"name": "reject_unaligned_and_nan", "source": "crates/quantinfer-quant/src/lib.rs:50-64",
         "qtype": "q8_0", "unaligned_n": 31, "nan_n": 32, "check": "rejected_both"},
    ]


def numerical_gate():
    # crates/quantinfer-runtime/tests/numerical_gates.rs:15-86
    return {
        "name": "explicit_weight_and_logit_gates",
        "source": "crates/quantinfer-runtime/tests/numerical_gates.rs:15-86",
        "input": "sin(0.17*i)*0.75 for i<64, shape [2,32]",
        "weight": "cos(0.11*i)*0.4 for i<256, shape [32,8]",
        "q8_weight_error_below": 0.01, "q4_weight_error_below": 0.08,
        "q8_logit_max_below": 0.02, "q8_logit_mse_below": 1e-4,
        "q8_top4_overlap_at_least": 3, "q4_top4_overlap_at_least": 2,
    }


def linear_layout_case():
    # crates/quantinfer-runtime/src/linear/tests.rs:78-159 (the matrix and bound)
    return {
        "name": "non_square_layouts_vs_f64",
        "source": "crates/quantinfer-runtime/src/linear/tests.rs:78-159",
        "inner": 256, "columns": 32, "rows": 3,
        "input": "(i*19 % 97)/97 - 0.5",
        "value": "((i*23 + o*7 + i//11) % 211) * 0.00373 - 0.39",
        "bound": "abs(actual - expected) < 1e-4 + 1e-5*abs(expected)",
    }


def decoder_cases():
    return [
        # backends/cpu/src/tests.rs:136-143: half-split RoPE rotation
        {"name": "half_split_rope_rotation", "source": "backends/cpu/src/tests.rs:136-143",
         "op": "apply_rope", "input_shape": [1, 1, 4], "input": [1.0, 2.0, 3.0, 4.0],
         "cos": [0.0, 1.0], "sin": [1.0, 0.0], "expected": [-3.0, 2.0, 1.0, 4.0]},
        # crates/quantinfer-runtime/src/qwen3/tests.rs:22-99: the constant-filled
        # one-layer model; prefill [1, 2] then decode [3]
        {"name": "qwen3_filled_prefill_decode", "source": "runtime/src/qwen3/tests.rs:22-99",
         "config": {"vocab": 16, "hidden": 8, "intermediate": 16, "layers": 1, "heads": 2,
                    "kv_heads": 1, "head_dim": 4, "max_positions": 32, "eps": 1e-6,
                    "theta": 1000000.0},
         "fill": {"embedding": 0.01, "norms": 1.0, "projections": 0.01, "lm_head": 0.01},
         "prefill_tokens": [1, 2], "decode_tokens": [3],
         "expected_prefill_logits_shape": [2, 16], "expected_length_after_prefill": 2,
         "expected_decode_logits_shape": [1, 16], "expected_length_after_decode": 3},
    ]


def main():
    data = {
        "about": "Known answers transcribed from aiqubits/quantinfer tests (data only).",
        "known_answers": known_answers(),
        "wire": wire_vectors(),
        "quantizer_bounds": quantizer_bounds(),
        "numerical_gate": numerical_gate(),
        "linear_layout": linear_layout_case(),
        "decoder": decoder_cases(),
    }
    path = os.path.join(HERE, "reference_known_answers.json")
    with open(path, "w") as f:
        json.dump(data, f, indent=1)
    print(path)


if __name__ == "__main__":
    main()
