"""Pin the oracle's CpuScalar matmuls (output rows, row major, f32).

- bit-equal to the independent numpy sequential-f32 restatement (the CpuScalar
  accumulation order, backends/cpu/src/matmul.rs:146-157 and :319-330);
- within |a-e| < 1e-4 + 1e-5|e| of an f64 brute force over the dequantized
  weights (runtime/src/linear/tests.rs:137-155), on the reference's own
  256x32x3 matrix through the GGUF wire round trip;
- threaded bit-equal to scalar (cpu tests.rs:156-177);
- the reference's rejections of malformed shapes.
"""
import numpy as np
import pytest

from oracle import pyoracle as po
from tests import numpy_ref
from tests.helpers import load_golden, reference_bound_ok

f32 = np.float32
ALL = [po.Q8_0, po.Q4_0, po.Q4_K, po.Q5_K, po.Q6_K]


@pytest.mark.parametrize("qtype", ALL)
@pytest.mark.parametrize("m", [1, 3])
def test_output_rows_equal_sequential_f32_restatement(qtype, m):
    k, n = 512, 24
    blocks = po.make_weights(qtype, k, n, seed=100 + qtype, outliers=qtype >= po.Q4_K)
    x = po.fill_normal(200 + m, m * k).reshape(m, k)
    y = po.matmul_output_rows(qtype, x, blocks, n)
    w = numpy_ref.DEQUANT[qtype](blocks).reshape(n, k)
    assert y.tobytes() == numpy_ref.sequential_f32(x, w).tobytes()
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    assert reference_bound_ok(y, exact)


@pytest.mark.parametrize("qtype", ALL)
def test_row_major_equal_sequential_f32_restatement(qtype):
    k, n, m = 64, 256, 2
    blocks = po.make_weights(qtype, k, n, seed=300 + qtype)
    x = po.fill_normal(400, m * k).reshape(m, k)
    y = po.matmul_row_major(qtype, x, blocks, n)
    # row major: element (k, n) at flat index k*N + n (matmul.rs:162-168)
    w_kn = numpy_ref.DEQUANT[qtype](blocks).reshape(k, n)
    assert y.tobytes() == numpy_ref.sequential_f32(x, w_kn.T).tobytes()


def test_f32_matmul_equal_sequential_restatement():
    x = po.fill_normal(1, 3 * 40).reshape(3, 40)
    w = po.fill_normal(2, 40 * 37).reshape(40, 37)
    assert po.matmul_f32(x, w).tobytes() == numpy_ref.sequential_f32(x, w.T).tobytes()


@pytest.mark.parametrize("qtype", ALL)
def test_threaded_bit_equal(qtype):
    k, n, m = 256, 16, 7
    blocks = po.make_weights(qtype, k, n, seed=7)
    x = po.fill_normal(8, m * k).reshape(m, k)
    a = po.matmul_output_rows(qtype, x, blocks, n)
    b = po.matmul_output_rows(qtype, x, blocks, n, threads=3)
    assert a.tobytes() == b.tobytes()


def test_reference_layout_matrix_through_wire_round_trip():
    """runtime/src/linear/tests.rs:78-159 (output-rows physical order)."""
    case = load_golden()["linear_layout"]
    inner, columns, rows = case["inner"], case["columns"], case["rows"]
    x = np.array([(i * 19 % 97) / f32(97.0) - f32(0.5) for i in range(rows * inner)],
                 dtype=f32).reshape(rows, inner)
    val = lambda i, o: f32(((i * 23 + o * 7 + i // 11) % 211)) * f32(0.00373) - f32(0.39)
    physical = np.array([val(i, o) for o in range(columns) for i in range(inner)], dtype=f32)
    for q in ALL:
        blocks = po.quantize(q, physical)
        blocks = po.wire_unpack(q, po.wire_pack(q, blocks))  # GGUF f16 storage
        y = po.matmul_output_rows(q, x, blocks, columns)
        w = po.dequantize(q, blocks).reshape(columns, inner)
        exact = x.astype(np.float64) @ w.astype(np.float64).T
        assert reference_bound_ok(y, exact), q


@pytest.mark.parametrize("qtype", ALL)
def test_rejects_malformed_shapes(qtype):
    bs = po.BLOCK_ELEMS[qtype]
    blocks = po.make_weights(qtype, bs, 2, seed=1)
    x = np.ones((1, bs), dtype=f32)
    with pytest.raises(po.OracleError):  # inner mismatch (matmul.rs:136-140)
        po.matmul_output_rows(qtype, np.ones((1, 2 * bs), dtype=f32), blocks, 2)
    with pytest.raises(po.OracleError):  # block count (matmul.rs:306-313)
        po.matmul_output_rows(qtype, x, blocks[:1], 2)
    with pytest.raises(po.OracleError):  # zero outputs
        po.matmul_output_rows(qtype, x, blocks[:0], 0)


def test_simd_variants_within_tolerance_on_random_data():
    isas = [i for i in (1, 2) if po.simd_available(i)]
    if not isas:
        pytest.skip("no AVX2/AVX-512 on this host")
    for q in (po.Q8_0, po.Q4_0):
        blocks = po.make_weights(q, 1024, 16, seed=5)
        x = po.fill_normal(6, 2 * 1024).reshape(2, 1024)
        scalar = po.matmul_output_rows(q, x, blocks, 16)
        for isa in isas:
            simd = po.matmul_output_rows_simd(q, isa, x, blocks, 16)
            assert np.max(np.abs(simd - scalar)) < 1e-4


# ---------------------------------------------- summation order, by arithmetic
#
# CpuScalar adds the products one at a time, k ascending, into one f32 sum
# (backends/cpu/src/matmul.rs:146-157 output rows, :319-330 K-quants, :25-31
# row major, :92-117 F32). Four products 2^24, 1, 1, -2^24 decide the order
# by f32 rounding alone: 2^24 + 1 rounds back to 2^24 (ties to even), so
# - left to right:                          ((2^24 + 1) + 1) - 2^24 = 0
# - per block, then the blocks (pairs in different blocks):
#                                           (2^24 + 1) + (1 - 2^24) = 1
# - pairwise:                               the same grouping       = 1
# - right to left:                          ((-2^24 + 1) + 1) + 2^24 = 2
# The expected 0 is that arithmetic, not a restatement of the loop.

TWO24 = float(2 ** 24)


def _unit_weight_blocks(qtype, k, ones):
    """One output of K weights that are 0 except 1.0 at the positions in
    `ones`, built from the block fields (Appendix formulas: Q8_0 scale*code,
    Q4_0 scale*(code - 8), Q4_K/Q5_K (d*sc)*q - dmin*m, Q6_K (d*sc)*(q - 32))."""
    dt = po.BLOCK_DTYPES[qtype]
    bs = po.BLOCK_ELEMS[qtype]
    b = np.zeros(k // bs, dtype=dt)
    b["scale"] = 1.0
    for pos in ones:
        blk, l = divmod(pos, bs)
        if qtype == po.Q8_0:
            b["values"][blk, l] = 1
        elif qtype == po.Q4_0:
            b["values"][blk, l] = 9
        elif qtype in (po.Q4_K, po.Q5_K):
            # l in the first 32 elements: low nibble of qs[l]; sc = 1, m = 0
            assert l < 32
            b["values"][blk, l] |= 1
        else:
            assert l < 32  # Q6_K: ql[l] low nibble, high bits 2 (q = 33)
            b["low_bits"][blk, l] |= 1
    if qtype == po.Q4_0:
        b["values"][b["values"] == 0] = 8
    if qtype in (po.Q4_K, po.Q5_K):
        b["min_scale"] = 0.0
        b["scales"][:] = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]  # sc_j = 1, m_j = 0
    if qtype == po.Q6_K:
        b["high_bits"][:] = 0xAA  # every q's high bits 2: q = 32 + low nibble
        b["scales"][:] = 1
    return b


@pytest.mark.parametrize("qtype", ALL)
def test_output_rows_sum_order_known_answer(qtype):
    bs = po.BLOCK_ELEMS[qtype]
    k = 2 * bs
    ones = [0, 1, bs, bs + 1]  # two products in each block
    blocks = _unit_weight_blocks(qtype, k, ones)
    w = po.dequantize(qtype, blocks)
    assert sorted(np.flatnonzero(w).tolist()) == ones and np.all(w[ones] == 1.0)
    x = np.zeros((1, k), dtype=f32)
    x[0, ones] = [TWO24, 1.0, 1.0, -TWO24]
    assert po.matmul_output_rows(qtype, x, blocks, 1)[0, 0] == 0.0
    # the same products reversed in k give 2
    x[0, ones] = [-TWO24, 1.0, 1.0, TWO24]
    assert po.matmul_output_rows(qtype, x, blocks, 1)[0, 0] == 2.0


def test_row_major_and_f32_sum_order_known_answer():
    k, n = 64, 3
    w = np.zeros((k, n), dtype=f32)
    ones = [0, 1, 32, 33]
    w[ones, :] = 1.0
    x = np.zeros((1, k), dtype=f32)
    x[0, ones] = [TWO24, 1.0, 1.0, -TWO24]
    assert np.all(po.matmul_f32(x, w) == 0.0)
    blocks = _unit_weight_blocks(po.Q8_0, k * n, [o * n + c for o in ones for c in range(n)])
    assert np.all(po.matmul_row_major(po.Q8_0, x, blocks, n) == 0.0)


def test_product_order_known_answer():
    """sum += x * (scale * code) (matmul.rs:150-155): the weight is rounded
    first. Q8_0, scale 0.1f, code 3, x = 1.3f: fl(1.3f * fl(0.1f * 3)) has
    bits 0x3EC7AE15, while fl(fl(1.3f * 0.1f) * 3) would be 0x3EC7AE14."""
    b = np.zeros(1, dtype=po.BLOCK_DTYPES[po.Q8_0])
    b["scale"] = f32(0.1)
    b["values"][0, 0] = 3
    x = np.zeros((1, 32), dtype=f32)
    x[0, 0] = f32(1.3)
    y = po.matmul_output_rows(po.Q8_0, x, b, 1)
    assert y.view(np.uint32)[0, 0] == 0x3EC7AE15
