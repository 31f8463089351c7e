"""Pin the oracle's quantizers and dequantizers.

- dequantizers: against the independent numpy restatement (tests/numpy_ref.py)
  on random blocks covering every code, scale byte and high bit;
- K-quant quantizers: the reference's exhaustive nearest-codebook oracle
  (quant/src/schemes/k_grid_tests.rs:23-145) restated as a brute-force search,
  d == f16(d), plus the edge cases of k_grid_tests.rs:148-196;
- Q8_0/Q4_0 quantizers: brute-force nearest code for the stored scale and the
  round-trip bounds of quant/src/lib.rs tests;
- the explicit weight/logit gates of runtime/tests/numerical_gates.rs:15-86.
"""
import numpy as np
import pytest

from oracle import pyoracle as po
from tests import numpy_ref
from tests.helpers import load_golden

f32 = np.float32


def _random_blocks(qtype, count, seed):
    rng = np.random.default_rng(seed)
    b = np.zeros(count, dtype=po.BLOCK_DTYPES[qtype])
    raw = rng.integers(0, 256, size=(count, po.BLOCK_DTYPES[qtype].itemsize), dtype=np.uint8)
    b = raw.view(po.BLOCK_DTYPES[qtype]).ravel().copy()
    b["scale"] = rng.standard_normal(count).astype(f32) * f32(0.01)
    if "min_scale" in b.dtype.names:
        b["min_scale"] = rng.standard_normal(count).astype(f32) * f32(0.01)
    if qtype == po.Q4_0:
        b["values"] &= 15
    return b


@pytest.mark.parametrize("qtype", [po.Q8_0, po.Q4_0, po.Q4_K, po.Q5_K, po.Q6_K])
def test_dequantize_matches_independent_restatement(qtype):
    b = _random_blocks(qtype, 512, 3 + qtype)
    ours = po.dequantize(qtype, b)
    ref = numpy_ref.DEQUANT[qtype](b)
    assert ours.tobytes() == ref.tobytes()
    # the per-element value() used by the matmuls is the same function
    idx = np.random.default_rng(1).integers(0, ours.size, 300)
    for i in idx:
        assert np.float32(po.value(qtype, b, int(i))).tobytes() == ours[i].tobytes()


def _k_grid_input():
    """quant/src/schemes/k_grid_tests.rs:7-22, evaluated in f32 left to right."""
    vals = []
    for block in range(4):
        for index in range(256):
            value = f32((index * 17 + block * 31) % 67) - f32(33.0)
            factor = f32(0.27) + f32(index // 32) * f32(0.09)
            v = f32(f32(f32(value / f32(19.0)) * f32(block + 1)) * f32(0.031))
            vals.append(f32(f32(v * factor) - f32(0.012)))
    vals += [0.0] * 256 + [-0.002] * 256 + [1.0e-8] * 256
    return np.array(vals, dtype=f32)


def _best_ok(value, code, codes, scale, mn):
    """k_grid_tests.rs:35-46"""
    err = lambda c: abs(scale * c - mn - float(value))
    expected = min(err(c) for c in codes)
    tol = (abs(scale) * 64.0 + abs(mn) + abs(float(value))) * float(np.finfo(f32).eps) + 1e-300
    return err(code) <= expected + tol


def _sc_m(scales, sub):
    if sub < 4:
        return scales[sub] & 63, scales[4 + sub] & 63
    i = sub - 4
    return (scales[8 + i] & 15) | ((scales[i] >> 6) << 4), (scales[8 + i] >> 4) | ((scales[4 + i] >> 6) << 4)


@pytest.mark.parametrize("qtype", [po.Q4_K, po.Q5_K])
def test_q4_q5_k_use_nearest_points_of_stored_codebook(qtype):
    x = _k_grid_input()
    blocks = po.quantize(qtype, x)
    top = 15 if qtype == po.Q4_K else 31
    for bi, blk in enumerate(blocks):
        d = float(blk["scale"])
        dmin = float(blk["min_scale"])
        assert f32(np.float16(blk["scale"])) == blk["scale"]
        assert f32(np.float16(blk["min_scale"])) == blk["min_scale"]
        for index in range(256):
            s, m = _sc_m(blk["scales"].astype(int), index // 32)
            g, w = index // 64, index % 64
            byte = int(blk["values"][g * 32 + w % 32])
            code = byte & 15 if w < 32 else byte >> 4
            if qtype == po.Q5_K:
                code |= ((int(blk["high_bits"][w % 32]) >> (2 * g + w // 32)) & 1) << 4
            assert _best_ok(x[bi * 256 + index], code, range(top + 1), d * s, dmin * m)


def test_q6_k_uses_nearest_points_of_stored_codebook():
    x = _k_grid_input()
    blocks = po.quantize(po.Q6_K, x)
    for bi, blk in enumerate(blocks):
        d = float(blk["scale"])
        assert f32(np.float16(blk["scale"])) == blk["scale"]
        for index in range(256):
            half, stripe, col = index // 128, index % 128 // 32, index % 32
            low = int(blk["low_bits"][half * 64 + stripe % 2 * 32 + col])
            low = low & 15 if stripe < 2 else low >> 4
            high = (int(blk["high_bits"][half * 32 + col]) >> (stripe * 2)) & 3
            code = (low | (high << 4)) - 32
            assert _best_ok(x[bi * 256 + index], code, range(-32, 32),
                            d * float(blk["scales"][index // 16]), 0.0)


@pytest.mark.parametrize("qtype", [po.Q8_0, po.Q4_0])
def test_q8_q4_codes_are_nearest_for_the_block_scale(qtype):
    x = po.fill_normal(5, 32 * 400, 0.02)
    blocks = po.quantize(qtype, x)
    lo, hi, off = (-127, 127, 0) if qtype == po.Q8_0 else (-8, 7, 8)
    for bi in range(0, 400, 7):
        blk = blocks[bi]
        scale = float(blk["scale"])
        # scale = absmax / levels in f32 (q8.rs:18-19, q4.rs:18-19)
        levels = f32(127.0) if qtype == po.Q8_0 else f32(7.0)
        assert blk["scale"] == f32(np.max(np.abs(x[bi * 32:(bi + 1) * 32])) / levels)
        for i in range(32):
            code = int(blk["values"][i]) - off
            v = float(x[bi * 32 + i])
            best = min(abs(scale * c - v) for c in range(lo, hi + 1))
            assert abs(scale * code - v) <= best + abs(v) * 1e-6 + 1e-30


def test_quantizer_bounds_from_reference_tests():
    for case in load_golden()["quantizer_bounds"]:
        if "qtype" in case and "input" in case:
            q = po.QTYPES[case["qtype"]]
            x = np.array(case["input"], dtype=f32)
            deq = po.dequantize(q, po.quantize(q, x))
            if case["check"] == "abs_at":
                assert abs(deq[case["index"]] - case["target"]) < case["bound"], case["name"]
            else:
                assert np.max(np.abs(deq - x)) < case["bound"], case["name"]
        elif case["check"] == "rejected_both":
            with pytest.raises(po.OracleError):
                po.quantize(po.Q8_0, np.ones(case["unaligned_n"], dtype=f32))
            with pytest.raises(po.OracleError):
                po.quantize(po.Q8_0, np.full(case["nan_n"], np.nan, dtype=f32))
            with pytest.raises(po.OracleError):
                po.quantize(po.Q4_0, np.full(case["nan_n"], np.nan, dtype=f32))
        else:
            for qname in case["qtypes"]:
                q = po.QTYPES[qname]
                x = np.full(case["n"], case["input_fill"], dtype=f32)
                if case["check"] == "rejected":
                    with pytest.raises(po.OracleError):
                        po.quantize(q, x)
                    continue
                deq = po.dequantize(q, po.quantize(q, x)).astype(np.float64)
                ref = x.astype(np.float64)
                rel = np.sqrt(np.sum((ref - deq) ** 2)) / np.sqrt(np.sum(ref ** 2))
                if case["check"] == "all_zero_and_rel_l2_one":
                    assert np.all(deq == 0.0) and rel == 1.0, (case["name"], qname)
                else:
                    assert rel < case["bound"], (case["name"], qname)


def test_explicit_weight_and_logit_gates():
    g = load_golden()["numerical_gate"]
    x = (np.sin(np.arange(64, dtype=f32) * f32(0.17)) * f32(0.75)).astype(f32).reshape(2, 32)
    w = (np.cos(np.arange(256, dtype=f32) * f32(0.11)) * f32(0.4)).astype(f32).reshape(32, 8)
    q8 = po.quantize(po.Q8_0, w.ravel())
    q4 = po.quantize(po.Q4_0, w.ravel())
    assert np.max(np.abs(po.dequantize(po.Q8_0, q8) - w.ravel())) < g["q8_weight_error_below"]
    assert np.max(np.abs(po.dequantize(po.Q4_0, q4) - w.ravel())) < g["q4_weight_error_below"]
    f = po.matmul_f32(x, w)
    y8 = po.matmul_row_major(po.Q8_0, x, q8, 8)
    y4 = po.matmul_row_major(po.Q4_0, x, q4, 8)
    assert np.max(np.abs(f - y8)) < g["q8_logit_max_below"]
    assert np.mean((f - y8) ** 2) < g["q8_logit_mse_below"]
    top = lambda v: list(np.argsort(-v.ravel(), kind="stable")[:4])
    assert len(set(top(f)) & set(top(y8))) >= g["q8_top4_overlap_at_least"]
    assert len(set(top(f)) & set(top(y4))) >= g["q4_top4_overlap_at_least"]


@pytest.mark.parametrize("qtype", [po.Q8_0, po.Q4_0, po.Q4_K, po.Q5_K, po.Q6_K])
def test_storage_precision_rounds_scales_only(qtype):
    b = po.quantize(qtype, po.fill_normal(9, 256 * 4, 0.02))
    s = po.storage_precision(qtype, b)
    assert np.array_equal(s["scale"], b["scale"].astype(np.float16).astype(f32))
    for name in b.dtype.names:
        if name not in ("scale", "min_scale"):
            assert np.array_equal(s[name], b[name])


def test_block_validation_matches_core():
    b = np.zeros(1, dtype=po.BLOCK_DTYPES[po.Q4_0])
    b["values"] = 15
    assert po.validate_blocks(po.Q4_0, b, 32)
    b["values"][0, 3] = 16  # core quantized/q4.rs:36-44
    assert not po.validate_blocks(po.Q4_0, b, 32)
    c = np.zeros(1, dtype=po.BLOCK_DTYPES[po.Q8_0])
    c["scale"] = np.inf  # core quantized/q8.rs:34-38
    assert not po.validate_blocks(po.Q8_0, c, 32)
    assert not po.validate_blocks(po.Q8_0, np.zeros(1, dtype=po.BLOCK_DTYPES[po.Q8_0]), 64)


# ----------------------------------------------------------------- Q5_K pin
#
# The dequantizer's fifth-bit decode (quant/src/schemes/q5_k.rs:96-135,
# backends/cpu/src/matmul.rs:217-258) is pinned twice, without retyping it:
#  - by the quantizer: its placement of the fifth bit is held by the
#    reference's own nearest-codebook test above (k_grid_tests.rs:82-113 reads
#    the bit as 2*group + within/32), so dequantize(quantize(x)) must land on
#    the nearest point of each sub-block's grid {d*sc*c - dmin*m : c = 0..31},
#    which is computed here from the block's scales alone;
#  - by a hand-worked block whose low and high nibbles differ and whose high
#    bits form a checkerboard, so that reading bit 2g+1 for the low half (or
#    2g for the high half) changes every element by 16*d*sc.


@pytest.mark.parametrize("seed", [11, 12])
def test_q5_k_dequantize_lands_on_nearest_grid_point(seed):
    # N(0, 0.02^2) with 0.5% N(0, 0.2^2) outliers, as BASELINE configs[2]
    x = po.fill_normal(seed, 256 * 96, 0.02, 0.005, 0.2)
    blocks = po.quantize(po.Q5_K, x)
    deq = po.dequantize(po.Q5_K, blocks).astype(np.float64)
    codes = np.arange(32, dtype=np.float64)
    checked = 0
    for bi, blk in enumerate(blocks):
        d, dmin = float(blk["scale"]), float(blk["min_scale"])
        for sub in range(8):
            s, m = _sc_m(blk["scales"].astype(int), sub)
            a, b = d * s, dmin * m
            grid = a * codes - b
            lo = bi * 256 + sub * 32
            xs = x[lo:lo + 32].astype(np.float64)
            nearest = np.min(np.abs(grid[None, :] - xs[:, None]), axis=1)
            err = np.abs(deq[lo:lo + 32] - xs)
            # f32 evaluation of (d*sc)*q - dmin*m: a few ulps of its operands
            tol = (abs(a) * 32.0 + abs(b)) * 4.0 * float(np.finfo(f32).eps) + 1e-30
            assert np.all(err <= nearest + tol), (bi, sub)
            # inside the grid the nearest point is at most half a step away
            inside = (xs >= -b) & (xs <= a * 31.0 - b)
            assert np.all(err[inside] <= 0.5 * a + tol), (bi, sub)
            checked += int(inside.sum())
    assert checked > 0.9 * x.size


def test_q5_k_dequantize_hand_worked_block():
    b = np.zeros(1, dtype=po.BLOCK_DTYPES[po.Q5_K])
    b["scale"] = 0.5
    b["min_scale"] = 0.25
    # sc0..3 = 1, 2, 3, 4 and m0..3 = 5, 6, 7, 8 (6-bit fields, top bits 0);
    # bytes 8..11 = 0x21: sc4..7 = 1, m4..7 = 2
    b["scales"][0] = [1, 2, 3, 4, 5, 6, 7, 8, 0x21, 0x21, 0x21, 0x21]
    b["values"] = 0x3A     # low nibble 10, high nibble 3
    b["high_bits"] = 0x55  # bits 0, 2, 4, 6: the low half's fifth bit only
    sc = [1, 2, 3, 4, 1, 1, 1, 1]
    mn = [5, 6, 7, 8, 2, 2, 2, 2]
    deq = po.dequantize(po.Q5_K, b)
    # sub-block j = 2g (elements 64g + [0, 32)): q = 10 + 16 = 26;
    # sub-block j = 2g + 1 (elements 64g + [32, 64)): q = 3
    expected = np.empty(256, dtype=np.float64)
    for j in range(8):
        q = 26 if j % 2 == 0 else 3
        expected[32 * j:32 * (j + 1)] = 0.5 * sc[j] * q - 0.25 * mn[j]
    # e.g. element 0: 0.5*1*26 - 0.25*5 = 11.75; element 32: 0.5*2*3 - 0.25*6 = 1.5
    assert expected[0] == 11.75 and expected[32] == 1.5 and expected[255] == 1.0
    assert np.array_equal(deq.astype(np.float64), expected)
    # the checkerboard the other way round: the high half's bit only
    b["high_bits"] = 0xAA
    deq = po.dequantize(po.Q5_K, b)
    for j in range(8):
        q = 10 if j % 2 == 0 else 19
        expected[32 * j:32 * (j + 1)] = 0.5 * sc[j] * q - 0.25 * mn[j]
    assert np.array_equal(deq.astype(np.float64), expected)
    for i in (0, 37, 100, 255):
        assert po.value(po.Q5_K, b, i) == expected[i]
