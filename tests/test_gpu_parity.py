"""GPU parity of the HIP path against the oracle, through the C ABI.

Bars:
- dequantize: bit-exact against the reference dequantize_* (oracle) for
  every block type, f16 and f32 scale planes, subnormal f16 scales included;
- EXACT mode: bit-identical to CpuScalar (oracle) in both layouts;
- F32 mode (the decode GEMV), three checks:
  (1) normwise against the CPU reference result r (oracle CpuScalar, f32):
      max_i |y_i - r_i| / max_i |r_i| <= 1e-5;
  (2) componentwise against the f64 product e of the dequantized weights:
      max_i |y_i - e_i| / max(|e_i|, sum_k |x_k w_ik| / 64) <= 1e-5
      (relative error wherever the dot product's condition number is <= 64);
  (3) the reference's own bound |y - e| < 1e-4 + 1e-5|e|
      (runtime/src/linear/tests.rs:152).
"""
import numpy as np
import pytest

import quantinfer_amd as qa
from oracle import pyoracle as po
from tests.helpers import (KAPPA_CAP, blocks_from_dicts, guarded_rel_err, lhs_from_case,
                           load_golden, normwise_rel_err, reference_bound_ok)

pytestmark = pytest.mark.gpu

ALL_Q = [qa.Q8_0, qa.Q4_0, qa.Q4_K, qa.Q5_K, qa.Q6_K]
NAMES = {qa.Q8_0: "q8_0", qa.Q4_0: "q4_0", qa.Q4_K: "q4_k", qa.Q5_K: "q5_k", qa.Q6_K: "q6_k"}
F32_TOL = 1e-5


@pytest.fixture(scope="module")
def ctx():
    c = qa.Context(0)
    yield c
    c.close()


def _wide_blocks(qtype, count, seed):
    """Random codes with f32 scales that are not f16-representable (as the
    reference's hand-built test blocks, e.g. scale 0.1)."""
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(count, po.BLOCK_DTYPES[qtype].itemsize), dtype=np.uint8)
    b = raw.view(po.BLOCK_DTYPES[qtype]).ravel().copy()
    b["scale"] = (rng.standard_normal(count) * 0.01 + 0.001).astype(np.float32)
    b["scale"] += np.float32(1e-9)
    if "min_scale" in b.dtype.names:
        b["min_scale"] = (rng.standard_normal(count) * 0.01).astype(np.float32)
    if qtype == po.Q4_0:
        b["values"] &= 15
    return b


def _f32_checks(y, x, blocks, qtype, n):
    """(componentwise error vs f64, normwise error vs the CPU reference, bound ok)"""
    k = x.shape[1]
    w = po.dequantize(qtype, blocks).reshape(n, k)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    cpu = po.matmul_output_rows(qtype, x, blocks, n, threads=8)
    return (guarded_rel_err(y, exact, x, w), normwise_rel_err(y, cpu),
            reference_bound_ok(y, exact))


def _assert_f32(y, x, blocks, qtype, n, what=""):
    comp, norm, ok = _f32_checks(y, x, blocks, qtype, n)
    assert comp <= F32_TOL and norm <= F32_TOL and ok, (what, comp, norm, ok)


# ------------------------------------------------------------------ dequant

@pytest.mark.parametrize("qtype", ALL_Q, ids=lambda q: NAMES[q])
def test_dequant_bit_exact_f16_scales(ctx, qtype):
    k, n = 1024, 48
    blocks = po.make_weights(qtype, k, n, seed=1000 + qtype, outliers=True)
    w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
    assert w.info().f16_scales == 1
    assert w.dequantize().tobytes() == po.dequantize(qtype, blocks).tobytes()


@pytest.mark.parametrize("qtype", ALL_Q, ids=lambda q: NAMES[q])
def test_dequant_bit_exact_row_major(ctx, qtype):
    """Row-major images, tiled (N = 512, K = 40: a partial last tile) and, for
    Q8_0/Q4_0, planar (N = 96): the flat block order of the reference."""
    shapes = [(40, 512)] + ([(40, 96)] if po.BLOCK_ELEMS[qtype] == 32 else [])
    for k, n in shapes:
        blocks = po.make_weights(qtype, n, k, seed=1050 + qtype + n, outliers=True)  # [K][N/bs]
        w = ctx.weights(qtype, qa.ROW_MAJOR, k, n, blocks)
        assert w.dequantize().tobytes() == po.dequantize(qtype, blocks).tobytes(), (k, n)
        w.free()


@pytest.mark.parametrize("qtype", ALL_Q, ids=lambda q: NAMES[q])
def test_dequant_bit_exact_f32_scales(ctx, qtype):
    bs = po.BLOCK_ELEMS[qtype]
    blocks = _wide_blocks(qtype, 64, 7 + qtype)
    w = ctx.weights(qtype, qa.OUTPUT_ROWS, bs * 8, 8, blocks)
    assert w.info().f16_scales == 0
    assert w.dequantize().tobytes() == po.dequantize(qtype, blocks).tobytes()


@pytest.mark.parametrize("qtype", [qa.Q4_K, qa.Q5_K, qa.Q6_K], ids=lambda q: NAMES[q])
def test_dequant_bit_exact_subnormal_f16_scales(ctx, qtype):
    # N(0, 0.02^2) weights give Q5_K/Q6_K super-block scales below f16's
    # smallest normal (6.1e-5); Q4_K gets there with a smaller weight scale.
    vals = po.fill_normal(77, 256 * 64, 0.02 if qtype != qa.Q4_K else 0.002)
    blocks = po.quantize(qtype, vals)
    assert np.any(blocks["scale"] < 6.103515625e-05), "fixture must contain subnormal d"
    w = ctx.weights(qtype, qa.OUTPUT_ROWS, 256 * 8, 8, blocks)
    assert w.dequantize().tobytes() == po.dequantize(qtype, blocks).tobytes()


# --------------------------------------------------------------- exact mode

@pytest.mark.parametrize("qtype", ALL_Q, ids=lambda q: NAMES[q])
@pytest.mark.parametrize("m", [1, 3])
def test_exact_mode_output_rows_bit_identical(ctx, qtype, m):
    k, n = 512, 40
    blocks = po.make_weights(qtype, k, n, seed=2000 + qtype, outliers=True)
    x = po.fill_normal(3000 + m, m * k).reshape(m, k)
    w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
    y = w.linear(x, qa.MODE_EXACT)
    assert y.tobytes() == po.matmul_output_rows(qtype, x, blocks, n).tobytes()


@pytest.mark.parametrize("qtype", ALL_Q, ids=lambda q: NAMES[q])
def test_exact_mode_row_major_bit_identical(ctx, qtype):
    k, n, m = 48 if qtype in (qa.Q8_0, qa.Q4_0) else 64, 256, 2
    blocks = po.make_weights(qtype, k, n, seed=2100 + qtype)
    x = po.fill_normal(3100, m * k).reshape(m, k)
    w = ctx.weights(qtype, qa.ROW_MAJOR, k, n, blocks)
    y = w.linear(x, qa.MODE_EXACT)
    assert y.tobytes() == po.matmul_row_major(qtype, x, blocks, n).tobytes()


def _assert_f32_row_major(y, x, blocks, qtype, n, what=""):
    """The F32-mode bars (componentwise vs f64, normwise vs CpuScalar, the
    reference's bound) for blocks along N: the dequantized values in block
    order are W row-major [K, N]."""
    k = x.shape[1]
    w = po.dequantize(qtype, blocks).reshape(k, n)
    exact = x.astype(np.float64) @ w.astype(np.float64)
    cpu = po.matmul_row_major(qtype, x, blocks, n)
    comp = guarded_rel_err(y, exact, x, w.T)
    norm = normwise_rel_err(y, cpu)
    assert comp <= F32_TOL and norm <= F32_TOL and reference_bound_ok(y, exact), (what, comp, norm)


@pytest.mark.parametrize("qtype", ALL_Q, ids=lambda q: NAMES[q])
def test_f32_row_major_gemv_tolerance(ctx, qtype):
    """Row-major (blocks along N) weights in F32/AUTO mode: the blocks-along-N
    GEMV (K split over the grid) within the F32 bars, and deterministic. N a
    multiple of 256 takes the tiled image (2 rows per launch; K = 200 leaves a
    partial last tile of 8 rows), Q8_0/Q4_0 with N = 128 the planar one (4 rows
    per launch)."""
    bs = po.BLOCK_ELEMS[qtype]
    for k, n in ((96, 4 * bs), (200, 512), (1024, 8 * bs), (4096, 2048 if bs == 32 else 4096)):
        blocks = po.make_weights(qtype, n, k, seed=2200 + qtype + k, outliers=qtype >= qa.Q4_K)
        w = ctx.weights(qtype, qa.ROW_MAJOR, k, n, blocks)
        for m in (1, 3, 6):
            x = po.fill_normal(3200 + m + k, m * k).reshape(m, k)
            y = w.linear(x, qa.MODE_F32)
            _assert_f32_row_major(y, x, blocks, qtype, n, (k, n, m))
            assert w.linear(x, qa.MODE_AUTO).tobytes() == y.tobytes()
        w.free()


@pytest.mark.parametrize("qtype", ALL_Q, ids=lambda q: NAMES[q])
def test_f32_row_major_many_rows_tolerance(ctx, qtype):
    """16 to 4100 rows on tiled row-major images, within the F32 bars and
    deterministic. K a multiple of 4 takes the row-major GEMM (16- and 32-row
    tiles, K parts summed in order or one part; K = 200 with a partial last
    tile, 4100 rows in a 4096-row chunk and a 4-row one); K = 42 keeps the
    GEMV's 2-row launches (an odd count ends with a 1-row launch)."""
    for k, n, ms in ((200, 512, (16, 128, 4100)), (4096, 4096, (16, 130)), (14336, 1024, (17, 300)),
                     (42, 256, (20, 130)), (1024, 12288, (128,))):
        blocks = po.make_weights(qtype, n, k, seed=2300 + qtype + k, outliers=qtype >= qa.Q4_K)
        w = ctx.weights(qtype, qa.ROW_MAJOR, k, n, blocks)
        for m in ms:
            x = po.fill_normal(3300 + m + k, m * k).reshape(m, k)
            y = w.linear(x, qa.MODE_F32)
            _assert_f32_row_major(y, x, blocks, qtype, n, (k, n, m))
            assert w.linear(x, qa.MODE_AUTO).tobytes() == y.tobytes()
        w.free()


@pytest.mark.parametrize("qtype", ALL_Q, ids=lambda q: NAMES[q])
def test_row_major_slice_weights_are_the_dequantized_ones(ctx, qtype):
    """The row-major GEMM's f32 weights (dequantized in LDS) equal the
    reference's dequantized values: with one-hot activation rows (row i picks
    weight row k_i) the outputs are those weight rows (every other product is
    zero, added exactly), here at K = 4100 and N = 4096 (K parts whose partial
    sums are added in order, a 4-row partial last tile)."""
    k, n = 4100, 4096
    blocks = po.make_weights(qtype, n, k, seed=2350 + qtype, outliers=qtype >= qa.Q4_K)
    w = ctx.weights(qtype, qa.ROW_MAJOR, k, n, blocks)
    picks = np.concatenate([[0, 1, 15, 16, 2047, 2048, 2049, 4095, 4096, 4099],
                            np.random.default_rng(qtype).integers(0, k, 120)])
    x = np.zeros((picks.size, k), np.float32)
    x[np.arange(picks.size), picks] = 1.0
    y = w.linear(x, qa.MODE_F32)
    want = po.dequantize(qtype, blocks).reshape(k, n)[picks]
    assert np.array_equal(y, want)
    w.free()


@pytest.mark.parametrize("qtype", ALL_Q, ids=lambda q: NAMES[q])
def test_row_major_f32_block_scales(ctx, qtype):
    """Row-major tiled images with f32 block scales (random codes, scales not
    f16-exact): F32 mode within the bars with one split (K = 48) and with a
    split sum (K = 1024), 1 to 20 rows; EXACT mode and dequantize
    bit-identical."""
    n = 512
    for k in (48, 1024):
        count = k * n // po.BLOCK_ELEMS[qtype]
        blocks = _wide_blocks(qtype, count, 2400 + qtype + k)
        if qtype >= qa.Q4_K:
            # random sub-scales put K-quant weights up to about 130 in
            # magnitude; scaled by 2^-6 (still not f16-exact) they stay near
            # 2, where CpuScalar itself meets the reference's absolute bound
            # (at K = 1024 it does not for the unscaled Q4_K/Q5_K/Q6_K blocks)
            for f in ("scale", "min_scale"):
                if f in blocks.dtype.names:
                    blocks[f] *= np.float32(1.0 / 64.0)
        w = ctx.weights(qtype, qa.ROW_MAJOR, k, n, blocks)
        assert w.info().f16_scales == 0
        assert w.dequantize().tobytes() == po.dequantize(qtype, blocks).tobytes()
        for m in (1, 2, 3, 20):
            x = po.fill_normal(3400 + m + k, m * k).reshape(m, k)
            _assert_f32_row_major(w.linear(x, qa.MODE_F32), x, blocks, qtype, n, (k, m))
        x = po.fill_normal(3410 + k, 2 * k).reshape(2, k)
        assert w.linear(x, qa.MODE_EXACT).tobytes() == po.matmul_row_major(qtype, x, blocks, n).tobytes()
        w.free()


def test_exact_mode_f32_weights_bit_identical(ctx):
    """EXACT mode on F32 weights is CpuScalar's sequential-k matmul bit for
    bit (N = 1001 is not a multiple of 4, the width the streaming GEMV needs:
    AUTO falls back to the same exact kernel there)."""
    k = 300
    for n in (1000, 1001):
        wt = po.fill_normal(5, k * n, 0.02).reshape(k, n)
        w = ctx.weights(qa.F32, qa.ROW_MAJOR, k, n, wt)
        for m in (1, 3, 17):
            x = po.fill_normal(6 + m, m * k).reshape(m, k)
            ref = po.matmul_f32(x, wt).tobytes()
            assert w.linear(x, qa.MODE_EXACT).tobytes() == ref
            if n % 4:
                assert w.linear(x, qa.MODE_AUTO).tobytes() == ref


def test_exact_mode_wide_scales_bit_identical(ctx):
    for qtype in ALL_Q:
        bs = po.BLOCK_ELEMS[qtype]
        blocks = _wide_blocks(qtype, 32, 40 + qtype)
        k, n = bs * 4, 8
        x = po.fill_normal(41, 2 * k).reshape(2, k)
        w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
        assert w.linear(x, qa.MODE_EXACT).tobytes() == \
            po.matmul_output_rows(qtype, x, blocks, n).tobytes()


def test_reference_known_answers_on_gpu(ctx):
    cases = {c["name"]: c for c in load_golden()["known_answers"]}
    for name in ("q8_0_ones_scale_two", "q4_0_code_eight_is_zero", "q4_k_0x99", "q5_k_0x99"):
        c = cases[name]
        q = po.QTYPES[c["qtype"]]
        blocks = blocks_from_dicts(q, c["blocks"])
        x = lhs_from_case(c)
        k, n = c["rhs_shape"]
        for layout in (qa.ROW_MAJOR, qa.OUTPUT_ROWS):
            w = ctx.weights(q, layout, k, n, blocks)
            for mode in (qa.MODE_EXACT, qa.MODE_F32):
                y = w.linear(x, mode)
                if c["expect"] == "equal":
                    assert y.ravel().tolist() == c["expected"], (name, layout, mode)
                else:
                    assert y.ravel()[0] > c["bound"]
                    assert y.ravel()[0] == po.matmul_row_major(q, x, blocks, n).ravel()[0] or \
                        mode == qa.MODE_F32
    c = cases["threaded_q8_equals_scalar"]
    blocks = blocks_from_dicts(qa.Q8_0, c["blocks"])
    w = ctx.weights(qa.Q8_0, qa.OUTPUT_ROWS, 32, 1, blocks)
    assert w.linear(lhs_from_case(c), qa.MODE_F32).ravel().tolist() == c["expected"]


# ---------------------------------------------------------- F32 GEMV path

@pytest.mark.parametrize("qtype", ALL_Q, ids=lambda q: NAMES[q])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 11, 16, 17, 40, 64])
def test_f32_gemv_tolerance_small(ctx, qtype, m):
    k, n = 1024, 70  # n not a multiple of the row tile: exercises the ragged tile
    blocks = po.make_weights(qtype, k, n, seed=4000 + qtype, outliers=True)
    x = po.fill_normal(5000 + m, m * k).reshape(m, k)
    w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
    _assert_f32(w.linear(x, qa.MODE_F32), x, blocks, qtype, n, m)


@pytest.mark.parametrize("qtype", ALL_Q, ids=lambda q: NAMES[q])
def test_f32_gemv_split_k_deterministic(ctx, qtype):
    # few output rows and a long K force split-K with the last-block reduction
    k, n = 14336, 12
    blocks = po.make_weights(qtype, k, n, seed=4100 + qtype, outliers=True)
    w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
    for m in (1, 8, 16):
        x = po.fill_normal(4200 + m, m * k).reshape(m, k)
        y = w.linear(x, qa.MODE_F32)
        _assert_f32(y, x, blocks, qtype, n, m)
        for _ in range(3):
            assert w.linear(x, qa.MODE_F32).tobytes() == y.tobytes()


@pytest.mark.parametrize("qtype", [qa.Q8_0, qa.Q4_0], ids=lambda q: NAMES[q])
@pytest.mark.parametrize("k", [96, 288, 4000])
def test_planar_gemv_tolerance(ctx, qtype, k):
    """K a multiple of 32 but not of 256: the planar image and its GEMV
    (qi_gemv.hip), ragged N, 1 to 16 rows (one launch per 16-row chunk) and
    17 (a second chunk)."""
    for n in (1, 17, 100):
        blocks = po.make_weights(qtype, k, n, seed=4300 + k + n + qtype, outliers=True)
        w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
        assert w.info().f16_scales == 1
        for m in (1, 3, 16, 17):
            x = po.fill_normal(4400 + m + n, m * k).reshape(m, k)
            y = w.linear(x, qa.MODE_F32)
            comp, norm, ok = _f32_checks(y, x, blocks, qtype, n)
            # with one output per row the normwise check (1) is the elementwise
            # relative error the tolerance section rules out for cancelled dot
            # products (the CPU result's own error dominates); (2) and (3) hold
            assert comp <= F32_TOL and ok and (n == 1 or norm <= F32_TOL), ((k, n, m), comp, norm, ok)
            assert w.linear(x, qa.MODE_F32).tobytes() == y.tobytes()
        w.free()


@pytest.mark.parametrize("qtype", [qa.Q4_K, qa.Q5_K, qa.Q6_K], ids=lambda q: NAMES[q])
def test_f32_gemv_wide_scales_k_quants(ctx, qtype):
    """K-quant images with f32 d/dmin (not f16-exact): the one-row GEMV and
    the 2-16 row kernels in their f32-scale form, at 3 tiles (one-tile
    workgroups) and 257 tiles (four-tile workgroups), within the F32 bars."""
    for k, n, ms in ((1024, 48, (1, 2, 5, 8, 16)), (1024, 4112, (1, 8, 16))):
        # quantized N(0, 0.02^2) weights whose super-block scales are moved
        # off the f16 grid (realistic magnitudes, f32 scale planes)
        blocks = po.make_weights(qtype, k, n, seed=90 + qtype + n, outliers=True)
        blocks["scale"] *= np.float32(1.0001)
        if "min_scale" in blocks.dtype.names:
            blocks["min_scale"] *= np.float32(1.0001)
        w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
        assert w.info().f16_scales == 0
        for m in ms:
            x = po.fill_normal(4400 + m, m * k).reshape(m, k)
            _assert_f32(w.linear(x, qa.MODE_F32), x, blocks, qtype, n, (n, m))
        w.free()


@pytest.mark.parametrize("qtype", [qa.Q4_0, qa.Q4_K, qa.Q5_K, qa.Q6_K], ids=lambda q: NAMES[q])
def test_f32_gemv_offset_cancellation(ctx, qtype):
    """The formats with an offset (w = a q - b) at few windows per output,
    where a sum x q and b sum x of uncentred codes cancel in f32 to about
    3.5e-5 of sum |x w| (Q4_K, K = 256, 16 rows): centred codes keep every
    kernel within 1e-5. K = 256 and 2048 take the 2-16 row kernel's zero
    points, K = 2304 its fixed centre; 1 row is the one-row kernel."""
    for k, n in ((256, 8192), (2048, 2048), (2304, 2048)):
        blocks = po.make_weights(qtype, k, n, seed=77 + qtype + k, outliers=True)
        w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
        for m in (1, 8, 16):
            x = po.fill_normal(4500 + m + k, m * k).reshape(m, k)
            _assert_f32(w.linear(x, qa.MODE_F32), x, blocks, qtype, n, (k, n, m))
        w.free()


# F32 mode from 33 rows on output rows: the split-half GEMM
# (qi_gemm_split.hip). (K, N, rows): one unit per row (the offsets' largest
# share, as in the cancellation case above), K parts over the grid with a
# ragged last tile, a partial last 64-row tile, and a 512-row prompt.
SPLIT_SHAPES = [(256, 8192, (48, 64, 200)), (12288, 1000, (48, 130)), (4096, 4096, (33, 50, 100, 512)),
                (1024, 24576, (65,))]


@pytest.mark.parametrize("qtype", ALL_Q, ids=lambda q: NAMES[q])
@pytest.mark.parametrize("shape", SPLIT_SHAPES, ids=lambda s: f"K{s[0]}-N{s[1]}")
def test_f32_split_gemm_tolerance(ctx, qtype, shape):
    k, n, ms = shape
    blocks = po.make_weights(qtype, k, n, seed=4600 + qtype + k, outliers=True)
    w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
    for m in ms:
        x = po.fill_normal(4700 + m + k, m * k).reshape(m, k)
        y = w.linear(x, qa.MODE_F32)
        _assert_f32(y, x, blocks, qtype, n, (k, n, m))
        assert w.linear(x, qa.MODE_F32).tobytes() == y.tobytes()  # deterministic
        if m >= 128:  # AUTO keeps the f16 GEMM from 128 rows; below, the same kernel
            continue
        assert w.linear(x, qa.MODE_AUTO).tobytes() == y.tobytes()
    w.free()


def test_f32_split_gemm_row_chunks(ctx):
    """Calls above 4096 rows run in 4096-row launches (bounded activation
    records): 4156 rows equal the 4096-row and 60-row calls of the same rows
    bit for bit, within the F32 bars."""
    qtype, k, n, m = qa.Q4_K, 512, 80, 4156
    blocks = po.make_weights(qtype, k, n, seed=4950, outliers=True)
    w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
    x = po.fill_normal(4951, m * k).reshape(m, k)
    y = w.linear(x, qa.MODE_F32)
    _assert_f32(y, x, blocks, qtype, n, "chunks")
    assert w.linear(np.ascontiguousarray(x[:4096]), qa.MODE_F32).tobytes() == y[:4096].tobytes()
    assert w.linear(np.ascontiguousarray(x[4096:]), qa.MODE_F32).tobytes() == y[4096:].tobytes()
    w.free()


@pytest.mark.parametrize("qtype", ALL_Q, ids=lambda q: NAMES[q])
def test_f32_split_gemm_wide_scales_and_scaled_rows(ctx, qtype):
    """f32 d / dmin (not f16-exact), and activation rows of very different
    magnitudes (1e-6 to 1e4) in one call: each (row, unit) takes its own
    power-of-two scale. Bars (1) and (2) are relative and hold for every row;
    the reference's absolute bound (3) is stated for N(0, 1) activations and
    is checked on the rows of scale <= 1. (Q8_0 / Q4_0 with f32 block scales
    keep the GEMV: their scales are not exact in the f16 weight halves.)"""
    k, n, m = 2048, 272, 48
    blocks = po.make_weights(qtype, k, n, seed=4800 + qtype, outliers=True)
    blocks["scale"] *= np.float32(1.0001)
    if "min_scale" in blocks.dtype.names:
        blocks["min_scale"] *= np.float32(1.0001)
    w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
    assert w.info().f16_scales == 0
    scales = 10.0 ** np.linspace(-6, 4, m)
    x = po.fill_normal(4900, m * k).reshape(m, k) * scales.astype(np.float32)[:, None]
    y = w.linear(x, qa.MODE_F32)
    comp, norm, _ = _f32_checks(y, x, blocks, qtype, n)
    assert comp <= F32_TOL and norm <= F32_TOL, (comp, norm)
    low = scales <= 1.0
    assert _f32_checks(y[low], x[low], blocks, qtype, n)[2]
    w.free()


def test_f32_gemv_unrounded_scales(ctx):
    # quantize_q8_0 output without storage rounding keeps f32 scales
    for qtype in (qa.Q8_0, qa.Q4_0):
        blocks = po.quantize(qtype, po.fill_normal(4300, 2048 * 33, 0.02))
        w = ctx.weights(qtype, qa.OUTPUT_ROWS, 2048, 33, blocks)
        assert w.info().f16_scales == 0
        x = po.fill_normal(4301, 3 * 2048).reshape(3, 2048)
        _assert_f32(w.linear(x, qa.MODE_F32), x, blocks, qtype, 33)


# ------------------------------------------------ BASELINE.json config shapes

CONFIGS = [
    # (qtype, K, N, M list, outliers) -- configs[0..2] of BASELINE.json
    (qa.Q8_0, 4096, 4096, [1], False),
    (qa.Q4_0, 4096, 4096, [1, 4, 8, 16], False),
    # 20 rows: a 16-row chunk with K parts and a 4-row chunk of one-tile workgroups
    (qa.Q4_0, 4096, 1024, [1, 4, 16, 20], False),
    (qa.Q4_0, 4096, 12288, [1, 4, 16], False),
    (qa.Q4_0, 12288, 4096, [1, 4, 16], False),
    # 12 and 16 rows: activation records built once per call (more than 8
    # units per K part), also with K parts (14336 x 4096)
    (qa.Q4_K, 4096, 14336, [1, 8, 12], True),
    (qa.Q4_K, 14336, 4096, [1, 8, 16], True),
    (qa.Q5_K, 4096, 14336, [1, 8], True),
    (qa.Q5_K, 14336, 4096, [1, 8, 16], True),
    (qa.Q6_K, 4096, 14336, [1, 8], True),
    (qa.Q6_K, 14336, 4096, [1, 8], True),
    (qa.Q8_0, 4096, 14336, [1], False),
]


@pytest.mark.parametrize("cfg", CONFIGS, ids=lambda c: f"{NAMES[c[0]]}-K{c[1]}-N{c[2]}")
def test_config_shapes_f32_tolerance(ctx, cfg):
    qtype, k, n, ms, outliers = cfg
    blocks = po.make_weights(qtype, k, n, seed=0x5EED0000 + qtype, outliers=outliers)
    w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
    wd = po.dequantize(qtype, blocks).reshape(n, k).astype(np.float64)
    absw = np.abs(wd)
    for m in ms:
        x = po.fill_normal(0x5EED1000 + m, m * k).reshape(m, k)
        y = w.linear(x, qa.MODE_F32)
        exact = x.astype(np.float64) @ wd.T
        denom = np.maximum(np.abs(exact), (np.abs(x.astype(np.float64)) @ absw.T) / KAPPA_CAP)
        comp = float(np.max(np.abs(y - exact) / denom))
        norm = normwise_rel_err(y, po.matmul_output_rows(qtype, x, blocks, n, threads=8))
        print(f"cfg {NAMES[qtype]} K={k} N={n} M={m}: componentwise {comp:.2e} normwise {norm:.2e}")
        assert comp <= F32_TOL and norm <= F32_TOL, (m, comp, norm)
        assert reference_bound_ok(y, exact)


@pytest.mark.parametrize("qtype,k,n,ms", [
    (qa.Q4_K, 8960, 1536, [2, 3, 4]),   # 35 units: 7 K parts of 5
    (qa.Q4_0, 6400, 1024, [5, 8, 16]),  # 25 units: 5 K parts of 5
    (qa.Q6_K, 6400, 1024, [8]),
], ids=["q4_k-K8960-N1536", "q4_0-K6400-N1024", "q6_k-K6400-N1024"])
def test_gemv_rows_uneven_k_parts(ctx, qtype, k, n, ms):
    """2-16 rows on shapes whose unit count does not divide into the first
    split count tried: the planner returns the count the launch runs."""
    blocks = po.make_weights(qtype, k, n, seed=0x5EED6200 + k + qtype, outliers=True)
    w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
    for m in ms:
        x = po.fill_normal(0x5EED6300 + m, m * k).reshape(m, k)
        _assert_f32(w.linear(x, qa.MODE_F32), x, blocks, qtype, n, f"K={k} N={n} M={m}")
    w.free()


@pytest.mark.parametrize("n", [20496, 20500, 24576, 24580])
def test_q4_k_gemv_six_tile_workgroups(ctx, n):
    """One row, K=4096, 1281-1536 output tiles: the six-tile, two-wavefront
    launch (the decoder's fused gate|up shape, N=24576), a ragged last tile
    (20500) and the one-tile launch just past its range (24580)."""
    k = 4096
    blocks = po.make_weights(qa.Q4_K, k, n, seed=0x5EED6000 + n, outliers=True)
    w = ctx.weights(qa.Q4_K, qa.OUTPUT_ROWS, k, n, blocks)
    x = po.fill_normal(0x5EED6100, k).reshape(1, k)
    y = w.linear(x, qa.MODE_F32)
    w.free()
    _assert_f32(y, x, blocks, qa.Q4_K, n, f"N={n}")


def test_config_q4_k_exact_mode_full_size(ctx):
    k, n = 4096, 14336
    blocks = po.make_weights(qa.Q4_K, k, n, seed=0x5EED0003, outliers=True)
    x = po.fill_normal(0x5EED2001, k).reshape(1, k)
    w = ctx.weights(qa.Q4_K, qa.OUTPUT_ROWS, k, n, blocks)
    assert w.linear(x, qa.MODE_EXACT).tobytes() == \
        po.matmul_output_rows(qa.Q4_K, x, blocks, n, threads=8).tobytes()


# ------------------------------------------------------------ ABI behaviour

def test_linear_device_matches_host_path(ctx):
    from quantinfer_amd import hiprt
    k, n, m = 4096, 512, 3
    blocks = po.make_weights(qa.Q4_K, k, n, seed=9, outliers=True)
    w = ctx.weights(qa.Q4_K, qa.OUTPUT_ROWS, k, n, blocks)
    x = po.fill_normal(10, m * k).reshape(m, k)
    xd = hiprt.DeviceBuffer.from_array(x)
    yd = hiprt.DeviceBuffer(m * n * 4)
    stream = hiprt.Stream()
    w.linear_device(xd.ptr, m, yd.ptr, qa.MODE_F32, stream.handle)
    stream.synchronize()
    assert yd.to_array(np.float32, (m, n)).tobytes() == w.linear(x, qa.MODE_F32).tobytes()
    out = hiprt.DeviceBuffer(k * n * 4)
    w.dequantize_device(out.ptr, stream.handle)
    stream.synchronize()
    assert out.to_array(np.float32, k * n).tobytes() == po.dequantize(qa.Q4_K, blocks).tobytes()
    stream.destroy()


@pytest.mark.parametrize("qtype,m,k,n,note", [
    (qa.Q4_K, 128, 256, 4096, "y 2 MiB: the kernels write into the pinned host buffer"),
    (qa.Q4_K, 128, 256, 16384, "y 8 MiB: pinned staging and a device-to-host copy"),
    (qa.Q8_0, 4200, 4096, 256, "x 66 MiB: copies from and to the caller's memory"),
    (qa.Q4_K, 2, 4096, 512, "small again after the buffers grew"),
])
def test_host_path_copy_regimes(ctx, qtype, m, k, n, note):
    """qi_hip_linear moves x and y through pinned buffers, writes outputs up
    to 4 MiB from the kernels into pinned host memory, and copies larger ones
    directly: every regime returns the device-buffer entry point's result bit
    for bit (AUTO mode: GEMV or GEMM by M)."""
    from quantinfer_amd import hiprt
    print(f"host path {m}x{k}x{n}: {note}", flush=True)
    blocks = po.make_weights(qtype, k, n, seed=21, outliers=False)
    w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
    x = po.fill_normal(22, m * k).reshape(m, k)
    xd = hiprt.DeviceBuffer.from_array(x)
    yd = hiprt.DeviceBuffer(m * n * 4)
    stream = hiprt.Stream()
    w.linear_device(xd.ptr, m, yd.ptr, qa.MODE_AUTO, stream.handle)
    stream.synchronize()
    want = yd.to_array(np.float32, (m, n))
    got = w.linear(x, qa.MODE_AUTO)
    assert got.tobytes() == want.tobytes()
    assert np.isfinite(got).all()
    stream.destroy()
    xd.free()
    yd.free()
    w.free()


def test_gpu_error_paths(ctx):
    blocks = po.make_weights(qa.Q8_0, 64, 4, seed=1)
    w = ctx.weights(qa.Q8_0, qa.OUTPUT_ROWS, 64, 4, blocks)
    lib = qa.lib()
    x = np.ones((1, 64), dtype=np.float32)
    y = np.empty((1, 4), dtype=np.float32)
    assert lib.qi_hip_linear(ctx.handle, w.handle, x.ctypes.data, 0, y.ctypes.data, 0) == qa.INVALID_INPUT
    assert lib.qi_hip_linear(ctx.handle, w.handle, x.ctypes.data, 1, y.ctypes.data, 9) == qa.INVALID_INPUT
    with pytest.raises(ValueError):
        w.linear(np.ones((1, 32), dtype=np.float32))
    with qa.Context(0) as other:
        assert lib.qi_hip_linear(other.handle, w.handle, x.ctypes.data, 1, y.ctypes.data, 0) == \
            qa.INVALID_INPUT
    assert ctx.device_name()


# ------------------------------------------------ MFMA prefill GEMM (f16 operands)

# Bars of the MFMA mode (f16 activations and weights, f32 accumulation):
#   normwise  max_i |y_i - e_i| / max_i |e_i| <= 2e-3, against the f64 product
#             e and against the CPU reference (CpuScalar, on sampled rows);
#   componentwise max_i |y_i - e_i| / max(|e_i|, sum_k |x_k w_ik| / 16) <= 2e-3:
#             relative error wherever the dot product's condition number is
#             <= 16. f16 operands carry a unit roundoff of 4.9e-4, so an output
#             that cancels 64-fold (the F32 mode's cap) is beyond 2e-3 for any
#             f16 arithmetic.
MFMA_TOL = 2e-3
MFMA_KAPPA = 16.0


def _mfma_checks(y, x, blocks, qtype, n, cpu_rows=None):
    """(componentwise vs f64, normwise vs f64, normwise vs CpuScalar on rows)"""
    k = x.shape[1]
    w = po.dequantize(qtype, blocks).reshape(n, k).astype(np.float64)
    exact = x.astype(np.float64) @ w.T
    comp = guarded_rel_err(y, exact, x, w, kappa=MFMA_KAPPA)
    norm = normwise_rel_err(y, exact)
    rows = np.arange(x.shape[0]) if cpu_rows is None else cpu_rows
    cpu = po.matmul_output_rows(qtype, np.ascontiguousarray(x[rows]), blocks, n, threads=8)
    return comp, norm, normwise_rel_err(y[rows], cpu)


@pytest.mark.parametrize("qtype", ALL_Q, ids=lambda q: NAMES[q])
@pytest.mark.parametrize("m", [1, 5, 128, 200])
def test_mfma_gemm_tolerance_small(ctx, qtype, m):
    # N = 300 leaves a partial 128-output block and a partial 16-output tile
    k, n = 1024, 300
    blocks = po.make_weights(qtype, k, n, seed=6000 + qtype, outliers=True)
    x = po.fill_normal(6100 + m, m * k).reshape(m, k)
    w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
    y = w.linear(x, qa.MODE_MFMA)
    comp, norm, cpu = _mfma_checks(y, x, blocks, qtype, n)
    assert comp <= MFMA_TOL and norm <= MFMA_TOL and cpu <= MFMA_TOL, (comp, norm, cpu)
    if m >= 128:  # AUTO picks the GEMM from 128 rows on
        assert w.linear(x, qa.MODE_AUTO).tobytes() == y.tobytes()


@pytest.mark.parametrize("qtype", [qa.Q4_K, qa.Q5_K], ids=lambda q: NAMES[q])
@pytest.mark.parametrize("m", [5, 200, 512])
def test_lds_gemm_both_kernels(ctx, qtype, m, monkeypatch):
    """Q4_K and Q5_K with f16 scales run the LDS-staged GEMM;
    QI_HIP_GEMM_REG=1 the register-weight GEMM. Both meet the MFMA bars
    (K = 2048 at M = 512 runs 8 K-splits of one unit each, the shortest
    per-workgroup K range), and their results are identical: the same f16
    fragments go through the same matrix instructions in the same order."""
    k, n = 2048, 300
    blocks = po.make_weights(qtype, k, n, seed=6200 + m + qtype, outliers=True)
    x = po.fill_normal(6300 + m, m * k).reshape(m, k)
    w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
    y_lds = w.linear(x, qa.MODE_MFMA)
    monkeypatch.setenv("QI_HIP_GEMM_REG", "1")
    y_reg = w.linear(x, qa.MODE_MFMA)
    monkeypatch.delenv("QI_HIP_GEMM_REG")
    for y in (y_lds, y_reg):
        comp, norm, cpu = _mfma_checks(y, x, blocks, qtype, n)
        assert comp <= MFMA_TOL and norm <= MFMA_TOL and cpu <= MFMA_TOL, (m, comp, norm, cpu)
    assert y_lds.tobytes() == y_reg.tobytes()


def test_mfma_gemm_wide_scales(ctx):
    """f32 (not f16-exact) block scales through the GEMM, which rounds them to
    f16 operands; the scales stay in f16's normal range (beyond it the GEMM
    refuses the weight, tests/test_gpu_robustness.py)."""
    for qtype in ALL_Q:
        blocks = _wide_blocks(qtype, 2 * 1024 // po.BLOCK_ELEMS[qtype] * 16, 70 + qtype)
        s = blocks["scale"]
        blocks["scale"] = np.where(np.abs(s) < 1e-3, np.copysign(np.float32(1e-3) + np.abs(s), s), s)
        if qtype in (qa.Q4_K, qa.Q5_K):
            blocks["min_scale"] = np.abs(blocks["min_scale"])
        k, n = 2048 // 2, 32
        blocks = blocks[: n * k // po.BLOCK_ELEMS[qtype]]
        x = po.fill_normal(71, 130 * k).reshape(130, k)
        w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
        assert w.info().f16_scales == 0
        y = w.linear(x, qa.MODE_MFMA)
        wd = po.dequantize(qtype, blocks).reshape(n, k).astype(np.float64)
        exact = x.astype(np.float64) @ wd.T
        assert normwise_rel_err(y, exact) <= MFMA_TOL, NAMES[qtype]


# BASELINE.json configs[3], the full cross product: Q8_0 and Q4_K weights x
# (K=4096, N=4096), (K=4096, N=12288), (K=12288, N=4096) x M in {128, 512,
# 2048} (18 points; M=128 and 512 run K-split GEMMs, M=2048 none).
GEMM_SHAPES = [(qt, k, n) for qt in (qa.Q8_0, qa.Q4_K)
               for k, n in ((4096, 4096), (4096, 12288), (12288, 4096))]
GEMM_MS = (128, 512, 2048)


@pytest.mark.parametrize("cfg", GEMM_SHAPES, ids=lambda c: f"{NAMES[c[0]]}-K{c[1]}-N{c[2]}")
def test_config_shapes_mfma_tolerance(ctx, cfg):
    qtype, k, n = cfg
    blocks = po.make_weights(qtype, k, n, seed=0x5EED0010 + qtype, outliers=qtype != qa.Q8_0)
    w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
    rng = np.random.default_rng(3)
    for m in GEMM_MS:
        x = po.fill_normal(0x5EED3000 + m, m * k).reshape(m, k)
        y = w.linear(x, qa.MODE_MFMA)
        # the CPU reference (CpuScalar) on 32 sampled rows, the f64 product on all
        rows = np.sort(rng.choice(m, size=min(m, 32), replace=False))
        comp, norm, cpu = _mfma_checks(y, x, blocks, qtype, n, cpu_rows=rows)
        print(f"mfma {NAMES[qtype]} M={m} K={k} N={n}: comp {comp:.2e} norm {norm:.2e} cpu {cpu:.2e}",
              flush=True)
        assert comp <= MFMA_TOL and norm <= MFMA_TOL and cpu <= MFMA_TOL, (m, comp, norm, cpu)
        assert w.linear(x, qa.MODE_AUTO).tobytes() == y.tobytes()  # AUTO picks the GEMM here


# ------------------------------------------------ direct GGUF upload
@pytest.mark.parametrize("qtype", ALL_Q, ids=lambda q: NAMES[q])
def test_gguf_upload_same_results(ctx, qtype):
    """A weight uploaded from GGUF wire bytes (qi_hip_weights_create_gguf)
    dequantizes bit-exactly and multiplies byte-identically to the one uploaded
    from the logical blocks."""
    k, n = 1024, 80
    blocks = po.make_weights(qtype, k, n, seed=7000 + qtype, outliers=True)
    wire = po.wire_pack(qtype, blocks)
    wg = ctx.weights_gguf(qtype, qa.OUTPUT_ROWS, k, n, wire)
    wl = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
    assert wg.info().device_bytes == wl.info().device_bytes
    assert wg.dequantize().tobytes() == po.dequantize(qtype, blocks).tobytes()
    x = po.fill_normal(7100 + qtype, 3 * k).reshape(3, k)
    for mode in (qa.MODE_F32, qa.MODE_EXACT, qa.MODE_MFMA):
        assert wg.linear(x, mode).tobytes() == wl.linear(x, mode).tobytes(), mode
    wg.free()
    wl.free()


# ------------------------------------------- F32 weights (the dense matmul)
#
# backends/cpu/src/backend.rs:48-60 -> matmul.rs:92-117: W row-major [K, N]
# f32. F32/AUTO mode: the streaming GEMV up to 16 rows, the f32 matrix-core GEMM above;
# both judged by the F32 bars against CpuScalar's sequential f32 sums and the
# f64 product.

def _f32w_checks(y, x, w, rows=None):
    rows = np.arange(x.shape[0]) if rows is None else rows
    xs = np.ascontiguousarray(x[rows])
    cpu = po.matmul_f32(xs, w)
    exact = xs.astype(np.float64) @ w.astype(np.float64)
    return (guarded_rel_err(y[rows], exact, xs, np.ascontiguousarray(w.T)),
            normwise_rel_err(y[rows], cpu))


@pytest.mark.parametrize("m", [1, 2, 3, 8, 11, 16, 17, 128, 300])
def test_f32_weights_tolerance(ctx, m):
    k, n = 2048, 1000
    w = po.fill_normal(9800, k * n, 0.02).reshape(k, n)
    x = po.fill_normal(9801 + m, m * k).reshape(m, k)
    wt = ctx.weights(qa.F32, qa.ROW_MAJOR, k, n, w)
    y = wt.linear(x, qa.MODE_F32)
    comp, norm = _f32w_checks(y, x, w)
    assert comp <= F32_TOL and norm <= F32_TOL, (m, comp, norm)
    assert wt.linear(x, qa.MODE_AUTO).tobytes() == y.tobytes()
    assert wt.linear(x, qa.MODE_F32).tobytes() == y.tobytes()  # deterministic


@pytest.mark.parametrize("k,n,m", [(4096, 4096, 130), (2048, 8192, 300)])
def test_f32_weights_gemm_every_output(ctx, k, n, m):
    """The F32 bars over every output of larger products (532 K and 2.5 M
    outputs), where a single accumulation chain over K exceeded 1e-5
    componentwise."""
    w = po.fill_normal(9900 + m, k * n, 0.02).reshape(k, n)
    wt = ctx.weights(qa.F32, qa.ROW_MAJOR, k, n, w)
    x = po.fill_normal(9950 + m, m * k).reshape(m, k)
    y = wt.linear(x, qa.MODE_F32)
    comp, norm = _f32w_checks(y, x, w)
    assert comp <= F32_TOL and norm <= F32_TOL, (k, n, m, comp, norm)
    wt.free()


@pytest.mark.parametrize("k,n", [(1022, 1000), (4096, 260), (256, 4100)])
def test_f32_weights_gemm_edges(ctx, k, n):
    """K not a multiple of 4 (the GEMM's 16-byte x loads): 8-row GEMV chunks
    instead; N past a tile boundary by 4 columns; 17-128 rows across the
    GEMM's three tile heights."""
    w = po.fill_normal(9830 + k, k * n, 0.02).reshape(k, n)
    wt = ctx.weights(qa.F32, qa.ROW_MAJOR, k, n, w)
    for m in (17, 33, 65, 128):
        x = po.fill_normal(9831 + m, m * k).reshape(m, k)
        y = wt.linear(x, qa.MODE_F32)
        comp, norm = _f32w_checks(y, x, w)
        assert comp <= F32_TOL and norm <= F32_TOL, (k, n, m, comp, norm)
    wt.free()


def test_f32_weights_lm_head_shape(ctx):
    """The unchanged runtime's LM head: [4096, 151936] f32 (a Q6_K head
    dequantized at load, runtime/src/qwen3/loader.rs:47-61), one decode row
    (GEMV) and 17, 128 and 512 rows (GEMM: the 32-, 128- and 128-row tiles),
    on sampled outputs rows."""
    k, n = 4096, 151936
    w = po.fill_normal(9810, k * n, 0.02).reshape(k, n)
    wt = ctx.weights(qa.F32, qa.ROW_MAJOR, k, n, w)
    for m in (1, 17, 128, 512):
        x = po.fill_normal(9811 + m, m * k).reshape(m, k)
        y = wt.linear(x, qa.MODE_AUTO)
        rows = np.array([0, m // 2, m - 1]) if m > 1 else np.array([0])
        cols = np.random.default_rng(m).choice(n, 4096, replace=False)
        ws = np.ascontiguousarray(w[:, cols])
        comp, norm = _f32w_checks(np.ascontiguousarray(y[:, cols]), x, ws, rows)
        print(f"f32 head M={m}: comp {comp:.2e} norm {norm:.2e}", flush=True)
        assert comp <= F32_TOL and norm <= F32_TOL, (m, comp, norm)


def test_f32_weights_nonfinite_activations(ctx):
    k, n = 1024, 512
    w = po.fill_normal(9820, k * n, 0.02).reshape(k, n)
    w[:, 7] = 0.0  # Inf * 0 is NaN in the reference
    wt = ctx.weights(qa.F32, qa.ROW_MAJOR, k, n, w)
    for m in (1, 5, 40):
        x = po.fill_normal(9821, m * k).reshape(m, k)
        x[0, 3] = np.inf
        if m > 1:
            x[1, 9] = np.nan
        y = wt.linear(x, qa.MODE_F32)
        ref = po.matmul_f32(x, w)
        bad = [0, 1] if m > 1 else [0]
        assert np.array_equal(y[bad], ref[bad], equal_nan=True), m
        assert np.isnan(y[0, 7]) and np.isinf(y[0, 0])
        if m > 2:
            assert normwise_rel_err(y[2:], ref[2:]) <= F32_TOL
