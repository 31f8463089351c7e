"""GPU behaviour at the edges of the input domain and of the calling contract,
through the C ABI, checked against the oracle.

- Non-finite activations: the reference accepts NaN and +-Inf in the lhs
  tensor (core tensor.rs:179-196) and CpuScalar carries them into the outputs
  (backends/cpu/src/matmul.rs:146-157): a row with a NaN gives NaN outputs, a
  row with an infinite activation gives +-Inf or NaN per output depending on
  the signs and zeros of the weights. Every fast kernel recomputes a
  non-finite output in the reference's order, so such rows must equal
  CpuScalar exactly (NaN where NaN, the same infinity elsewhere); the finite
  rows of the same call keep their usual bars.
- Values outside the f16 operands of the matrix-core GEMM: activations beyond
  65504 overflow to infinity in f16 and are recomputed exactly; weights whose
  scales lie outside f16's normal range take the f32 kernels in AUTO mode and
  are refused in MFMA mode.
- Workspaces shared by calls on different caller streams, calls from two host
  threads on one context, and closing a context before freeing its weights.
"""
import threading

import numpy as np
import pytest

import quantinfer_amd as qa
from oracle import pyoracle as po
from tests.helpers import guarded_rel_err, normwise_rel_err
from tests.test_gpu_parity import ALL_Q, F32_TOL, MFMA_KAPPA, MFMA_TOL, NAMES, _assert_f32

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = qa.Context(0)
    yield c
    c.close()


def _poison(x):
    """Row 0: one NaN; row 1: one +Inf; row 2: -Inf and +Inf; other rows finite."""
    x = x.copy()
    x[0, 7] = np.nan
    x[1, x.shape[1] // 2 + 3] = np.inf
    x[2, 0] = -np.inf
    x[2, 1] = np.inf
    return x


def _check_nonfinite_rows(y, ref, rows):
    for r in rows:
        assert not np.isfinite(ref[r]).any(), r  # every output of such a row is NaN or +-Inf
        assert np.array_equal(y[r], ref[r], equal_nan=True), (r, y[r][:8], ref[r][:8])


@pytest.mark.parametrize("qtype", ALL_Q, ids=lambda q: NAMES[q])
@pytest.mark.parametrize("mode,m", [(qa.MODE_F32, 4), (qa.MODE_F32, 9), (qa.MODE_F32, 48), (qa.MODE_EXACT, 4),
                                    (qa.MODE_MFMA, 5), (qa.MODE_AUTO, 130)],
                         ids=["f32-m4", "f32-m9", "f32-m48", "exact-m4", "mfma-m5", "auto-m130"])
def test_nonfinite_activations_output_rows(ctx, qtype, mode, m):
    k, n = 512, 48
    blocks = po.make_weights(qtype, k, n, seed=8100 + qtype, outliers=True)
    x = _poison(po.fill_normal(8200 + m, m * k).reshape(m, k))
    w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
    y = w.linear(x, mode)
    ref = po.matmul_output_rows(qtype, x, blocks, n, threads=8)
    _check_nonfinite_rows(y, ref, (0, 1, 2))
    fin = x[3:]
    if mode == qa.MODE_EXACT:
        assert y[3:].tobytes() == ref[3:].tobytes()
    elif mode == qa.MODE_F32:
        _assert_f32(y[3:], fin, blocks, qtype, n, "finite rows")
    else:
        wd = po.dequantize(qtype, blocks).reshape(n, k).astype(np.float64)
        exact = fin.astype(np.float64) @ wd.T
        assert guarded_rel_err(y[3:], exact, fin, wd, kappa=MFMA_KAPPA) <= MFMA_TOL
        assert normwise_rel_err(y[3:], exact) <= MFMA_TOL


def test_nonfinite_activations_one_row(ctx):
    """M = 1 (the decode GEMV's single-row kernels) for every format."""
    k, n = 1024, 64
    for qtype in ALL_Q:
        blocks = po.make_weights(qtype, k, n, seed=8300 + qtype)
        w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
        for bad in (np.nan, np.inf, -np.inf):
            x = po.fill_normal(8400, k).reshape(1, k)
            x[0, 513] = bad
            for mode in (qa.MODE_F32, qa.MODE_AUTO, qa.MODE_EXACT):
                y = w.linear(x, mode)
                ref = po.matmul_output_rows(qtype, x, blocks, n)
                assert np.array_equal(y, ref, equal_nan=True), (NAMES[qtype], bad, mode)


@pytest.mark.parametrize("qtype", [qa.Q8_0, qa.Q4_0], ids=lambda q: NAMES[q])
def test_nonfinite_activations_planar_gemv(ctx, qtype):
    """K a multiple of 32 but not of 256: the planar f32 GEMV."""
    k, n, m = 96, 40, 5
    blocks = po.make_weights(qtype, k, n, seed=8500 + qtype)
    x = _poison(po.fill_normal(8501, m * k).reshape(m, k))
    w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
    y = w.linear(x, qa.MODE_F32)
    ref = po.matmul_output_rows(qtype, x, blocks, n)
    _check_nonfinite_rows(y, ref, (0, 1, 2))
    _assert_f32(y[3:], x[3:], blocks, qtype, n, "finite rows")


@pytest.mark.parametrize("qtype", ALL_Q, ids=lambda q: NAMES[q])
@pytest.mark.parametrize("k", [512, 48], ids=["k-split", "one-split"])
def test_nonfinite_activations_row_major(ctx, qtype, k):
    """NaN/Inf activations on row-major weights: non-finite outputs are
    recomputed in the reference's order by the GEMV at 1 and 2 rows (K = 512
    in its split sum, K = 48 in the GEMV itself) and by the row-major GEMM
    from 3 rows (K = 512 in the sum of its 4 parts, K = 48 in the GEMM itself:
    three tiles, one part; 9, 20 and 130 rows on its 16- and 32-row tiles)."""
    n, m = 256, 4
    blocks = po.make_weights(qtype, n, k, seed=8600 + qtype)  # [K, N] blocks along N
    x = _poison(po.fill_normal(8601, m * k).reshape(m, k))
    w = ctx.weights(qtype, qa.ROW_MAJOR, k, n, blocks)
    ref = po.matmul_row_major(qtype, x, blocks, n)
    for mode in (qa.MODE_F32, qa.MODE_EXACT):
        y = w.linear(x, mode)
        _check_nonfinite_rows(y, ref, (0, 1, 2))
    for m1 in (1, 2, 9, 20, 130):  # the GEMV at 1 and 2 rows, the GEMM's 16- and 32-row tiles
        x1 = po.fill_normal(8602, m1 * k).reshape(m1, k)
        x1[0, 5] = np.inf
        y1 = w.linear(x1, qa.MODE_F32)
        ref1 = po.matmul_row_major(qtype, x1, blocks, n)
        _check_nonfinite_rows(y1, ref1, (0,))
        assert np.isfinite(y1[1:]).all()
        if m1 > 1:
            assert normwise_rel_err(y1[1:], ref1[1:]) <= F32_TOL


@pytest.mark.parametrize("qtype", [qa.Q8_0, qa.Q4_K, qa.Q6_K], ids=lambda q: NAMES[q])
@pytest.mark.parametrize("m,n", [(130, 96), (2048, 4096)], ids=["k-split", "no-split"])
def test_activations_beyond_f16_range_in_gemm(ctx, qtype, m, n):
    """|x| > 65504 is infinite as an f16 operand: the GEMM recomputes those
    rows' outputs in the reference's order (bit-identical), with a K split
    (130 x 1024 x 96: 4 splits of one unit) and without (2048 x 1024 x 4096:
    256 row x column blocks)."""
    k = 1024
    blocks = po.make_weights(qtype, k, n, seed=8700 + qtype)
    w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
    x = po.fill_normal(8701 + m, m * k).reshape(m, k)
    big = [0, 77, m - 1]
    for r in big:
        x[r, 100 + r % 50] = 1.0e5
    y = w.linear(x, qa.MODE_AUTO)
    ref_rows = po.matmul_output_rows(qtype, np.ascontiguousarray(x[big]), blocks, n, threads=8)
    assert y[big].tobytes() == ref_rows.tobytes()
    rest = np.setdiff1d(np.arange(m), big)[:64]
    wd = po.dequantize(qtype, blocks).reshape(n, k).astype(np.float64)
    exact = x[rest].astype(np.float64) @ wd.T
    assert normwise_rel_err(y[rest], exact) <= MFMA_TOL


def _q8_blocks_with_scale(k, n, scale, seed):
    rng = np.random.default_rng(seed)
    b = np.zeros(n * k // 32, dtype=po.BLOCK_DTYPES[po.Q8_0])
    b["values"] = rng.integers(-127, 128, size=(b.size, 32), dtype=np.int8)
    b["scale"] = (np.float32(scale) * (1.0 + 0.1 * rng.standard_normal(b.size))).astype(np.float32)
    return b


@pytest.mark.parametrize("scale", [1.0e3, 1.0e-7])
def test_scales_outside_f16_range(ctx, scale):
    """Q8_0 block scales of 1e3 (weights overflow f16) or 1e-7 (scales are f16
    subnormals): AUTO at 130 rows takes the f32 kernels and meets the f32
    bars; MFMA mode refuses the weight (UNSUPPORTED)."""
    k, n, m = 512, 64, 130
    blocks = _q8_blocks_with_scale(k, n, scale, 8800)
    w = ctx.weights(qa.Q8_0, qa.OUTPUT_ROWS, k, n, blocks)
    x = po.fill_normal(8801, m * k).reshape(m, k)
    y = w.linear(x, qa.MODE_AUTO)
    # the f32 bars (1) and (2); the reference's absolute 1e-4 term is for
    # unit-scale weights, so it does not apply to outputs near 1e6 or 1e-4
    wd = po.dequantize(qa.Q8_0, blocks).reshape(n, k).astype(np.float64)
    exact = x.astype(np.float64) @ wd.T
    assert guarded_rel_err(y, exact, x, wd) <= F32_TOL
    assert normwise_rel_err(y, po.matmul_output_rows(qa.Q8_0, x, blocks, n, threads=8)) <= F32_TOL
    with pytest.raises(qa.QiError) as e:
        w.linear(x, qa.MODE_MFMA)
    assert e.value.status == qa.UNSUPPORTED


# ------------------------------------------------ calling contract

def test_workspaces_ordered_across_streams(ctx):
    """Calls on different caller streams share the context's workspaces (the
    GEMM's f16 activations, its split-K partials, the multi-row GEMV's
    activation records). With no host synchronization between them, each
    call's output must still be its own: an M=512 GEMM on stream A, an M=512
    GEMM with other activations and an M=8 GEMV on stream B, then a
    synchronous call on the context's stream."""
    from quantinfer_amd import hiprt
    k, n = 4096, 4096
    blocks = po.make_weights(qa.Q4_K, k, n, seed=8900, outliers=True)
    w = ctx.weights(qa.Q4_K, qa.OUTPUT_ROWS, k, n, blocks)
    xs = {name: po.fill_normal(8901 + i, m * k).reshape(m, k)
          for i, (name, m) in enumerate((("a", 512), ("b", 512), ("c", 8), ("d", 200)))}
    ref = {name: w.linear(x, qa.MODE_AUTO) for name, x in xs.items()}  # one at a time
    sa, sb = hiprt.Stream(), hiprt.Stream()
    dev = {name: (hiprt.DeviceBuffer.from_array(x), hiprt.DeviceBuffer(x.shape[0] * n * 4))
           for name, x in xs.items() if name != "d"}
    for _ in range(3):
        w.linear_device(dev["a"][0].ptr, 512, dev["a"][1].ptr, qa.MODE_AUTO, sa.handle)
        w.linear_device(dev["b"][0].ptr, 512, dev["b"][1].ptr, qa.MODE_AUTO, sb.handle)
        w.linear_device(dev["c"][0].ptr, 8, dev["c"][1].ptr, qa.MODE_AUTO, sb.handle)
        yd = w.linear(xs["d"], qa.MODE_AUTO)
        sa.synchronize()
        sb.synchronize()
        for name in ("a", "b", "c"):
            got = dev[name][1].to_array(np.float32, (xs[name].shape[0], n))
            assert got.tobytes() == ref[name].tobytes(), name
        assert yd.tobytes() == ref["d"].tobytes()
    sa.destroy()
    sb.destroy()


def test_two_host_threads_on_one_context(ctx):
    """Handles may cross threads: two threads call one context concurrently
    (the mutex serializes the calls) and each gets its own results."""
    k, n = 2048, 1024
    jobs = []
    for i, qtype in enumerate((qa.Q4_K, qa.Q8_0)):
        blocks = po.make_weights(qtype, k, n, seed=9000 + i)
        w = ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
        xs = [po.fill_normal(9010 + 10 * i + j, m * k).reshape(m, k) for j, m in enumerate((1, 4, 130))]
        jobs.append((w, xs, [w.linear(x, qa.MODE_AUTO) for x in xs]))
    errors = []

    def run(w, xs, refs):
        try:
            for _ in range(20):
                for x, r in zip(xs, refs):
                    if w.linear(x, qa.MODE_AUTO).tobytes() != r.tobytes():
                        errors.append("mismatch")
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=run, args=job) for job in jobs]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors[:3]


def test_close_before_free_and_free_before_close():
    k, n = 256, 32
    blocks = po.make_weights(qa.Q4_K, k, n, seed=9100)
    x = po.fill_normal(9101, k).reshape(1, k)
    # close first: calls on the weights fail cleanly, the free releases the context
    c = qa.Context(0)
    w = c.weights(qa.Q4_K, qa.OUTPUT_ROWS, k, n, blocks)
    y = w.linear(x, qa.MODE_F32)
    c.close()
    with pytest.raises(qa.QiError) as e:
        w.linear(x, qa.MODE_F32)
    assert e.value.status == qa.INVALID_INPUT
    w.free()
    # free first, then close
    c2 = qa.Context(0)
    w2 = c2.weights(qa.Q4_K, qa.OUTPUT_ROWS, k, n, blocks)
    assert w2.linear(x, qa.MODE_F32).tobytes() == y.tobytes()
    w2.free()
    assert w2.handle is None
    c2.close()
