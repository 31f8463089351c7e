"""Pin the oracle against the reference's own known-answer tests
(transcribed in tests/golden/reference_known_answers.json) and the GGUF
wire vectors."""
import numpy as np
import pytest

from oracle import pyoracle as po
from tests.helpers import blocks_from_dicts, lhs_from_case, load_golden

GOLDEN = load_golden()
CASES = {c["name"]: c for c in GOLDEN["known_answers"]}


def _q(name):
    return po.QTYPES[name]


def test_f32_matrix_product():
    c = CASES["f32_matrix_product"]
    x = lhs_from_case(c)
    w = np.asarray(c["rhs"], dtype=np.float32).reshape(c["rhs_shape"])
    assert po.matmul_f32(x, w).ravel().tolist() == c["expected"]


@pytest.mark.parametrize("name", ["q8_0_ones_scale_two", "q4_0_code_eight_is_zero",
                                  "q4_k_0x99", "q5_k_0x99"])
def test_scalar_known_answers(name):
    c = CASES[name]
    q = _q(c["qtype"])
    x = lhs_from_case(c)
    blocks = blocks_from_dicts(q, c["blocks"])
    k, n = c["rhs_shape"]
    for y in (po.matmul_row_major(q, x, blocks, n), po.matmul_output_rows(q, x, blocks, n)):
        if c["expect"] == "equal":
            assert y.ravel().tolist() == c["expected"]
        else:
            assert y.ravel()[0] > c["bound"]


def test_q4_k_0x99_closed_form():
    # The reference only asserts > 200; the closed form pins the sub-block scale
    # unpack: scales [63;12] decode to sc = 63 for sub-blocks 0-3 and
    # (63 & 15) | ((63 >> 6) << 4) = 15 for 4-7, and 0x99 gives code 9 everywhere.
    c = CASES["q4_k_0x99"]
    blocks = blocks_from_dicts(po.Q4_K, c["blocks"])
    deq = po.dequantize(po.Q4_K, blocks)
    f = np.float32
    hi = f(f(f(0.1) * f(63)) * f(9)) - f(f(0.0) * f(63 & 63))
    lo = f(f(f(0.1) * f(15)) * f(9)) - f(f(0.0) * f(15))
    assert np.array_equal(deq, np.array([hi] * 128 + [lo] * 128, dtype=np.float32))
    acc = f(0)
    for v in deq:
        acc = f(acc + f(f(1.0) * v))
    y = po.matmul_output_rows(po.Q4_K, lhs_from_case(c), blocks, 1)
    assert y[0, 0] == acc


def test_k_quant_output_rows_equal_row_major():
    c = CASES["k_quant_output_rows_equal_row_major"]
    x = lhs_from_case(c)
    for v in c["variants"]:
        q = _q(v["qtype"])
        blocks = blocks_from_dicts(q, v["blocks"])
        a = po.matmul_output_rows(q, x, blocks, 1)
        b = po.matmul_row_major(q, x, blocks, 1)
        assert a.tobytes() == b.tobytes()


def test_simd_within_tolerance_of_scalar():
    c = CASES["simd_output_rows_match_scalar"]
    x = lhs_from_case(c)
    isas = [i for i in (1, 2) if po.simd_available(i)]
    if not isas:
        pytest.skip("host has neither AVX2 nor AVX-512")
    for qname, key in (("q8_0", "q8_blocks"), ("q4_0", "q4_blocks")):
        q = _q(qname)
        blocks = blocks_from_dicts(q, c[key])
        scalar = po.matmul_output_rows(q, x, blocks, 3)
        for isa in isas:
            simd = po.matmul_output_rows_simd(q, isa, x, blocks, 3)
            assert np.max(np.abs(simd - scalar)) < c["tolerance"]


def test_threaded_equals_scalar():
    c = CASES["threaded_q8_equals_scalar"]
    x = lhs_from_case(c)
    blocks = blocks_from_dicts(po.Q8_0, c["blocks"])
    scalar = po.matmul_row_major(po.Q8_0, x, blocks, 1)
    threaded = po.matmul_output_rows(po.Q8_0, x, blocks, 1, threads=c["threads"])
    assert scalar.ravel().tolist() == c["expected"]
    assert threaded.tobytes() == scalar.tobytes()


# ---------------------------------------------------------------- wire

WIRE = {w["name"]: w for w in GOLDEN["wire"]}


def test_q4_0_standard_and_legacy_bytes():
    w = WIRE["q4_0_standard_and_legacy"]
    blocks = blocks_from_dicts(po.Q4_0, [w["block"]])
    std = po.wire_pack(po.Q4_0, blocks)
    # writer.rs:197-211: byte j = v[j] | v[j+16] << 4 after the f16 scale
    v = w["block"]["values"]
    assert std.tolist() == [0x00, 0x38] + [v[j] | (v[j + 16] << 4) for j in range(16)]
    assert po.wire_unpack(po.Q4_0, std).tobytes() == blocks.tobytes()
    legacy = po.wire_unpack(po.Q4_0, np.array(w["legacy_bytes"], dtype=np.uint8), legacy=True)
    assert legacy.tobytes() == blocks.tobytes()


def test_q6_k_standard_and_legacy_bytes():
    w = WIRE["q6_k_standard_and_legacy"]
    blocks = blocks_from_dicts(po.Q6_K, [w["block"]])
    assert po.wire_pack(po.Q6_K, blocks).tolist() == w["standard_bytes"]
    std = po.wire_unpack(po.Q6_K, np.array(w["standard_bytes"], dtype=np.uint8))
    leg = po.wire_unpack(po.Q6_K, np.array(w["legacy_bytes"], dtype=np.uint8), legacy=True)
    assert std.tobytes() == blocks.tobytes() == leg.tobytes()


def test_q4_k_round_trip_144():
    w = WIRE["q4_k_round_trip_144"]
    blocks = blocks_from_dicts(po.Q4_K, [w["block"]])
    b = po.wire_pack(po.Q4_K, blocks)
    assert b.size == w["wire_size"]
    assert po.wire_unpack(po.Q4_K, b).tobytes() == blocks.tobytes()


@pytest.mark.parametrize("qname", ["q8_0", "q4_0", "q4_k", "q5_k", "q6_k"])
def test_wire_round_trip_of_quantized_data(qname):
    q = _q(qname)
    vals = po.fill_normal(11, 256 * 8, 0.02, 0.005, 0.2)
    blocks = po.storage_precision(q, po.quantize(q, vals))
    again = po.wire_unpack(q, po.wire_pack(q, blocks))
    assert again.tobytes() == blocks.tobytes()
    assert po.wire_pack(q, blocks).size == po.WIRE_BYTES[q] * blocks.size


def test_wire_rejects_non_finite_scale():
    bad = np.zeros(34, dtype=np.uint8)
    bad[0:2] = [0x00, 0x7C]  # +inf
    with pytest.raises(po.OracleError):
        po.wire_unpack(po.Q8_0, bad)
