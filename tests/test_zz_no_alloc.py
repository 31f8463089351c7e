"""qi_hip_linear_device_noalloc, the linear call that allocates nothing,
against qi_hip_linear_device through the C ABI.

Both entry points run the same kernels (the same plan); the no-allocation one
takes its workspaces from the library's fixed per-GPU scratch array instead
of the context's grown buffers, so its outputs must equal the allocating
call's bit for bit. Each case makes two no-allocation calls in a row on one
stream, the second with fewer rows (the scratch keeps the first call's
contents), and a call that needs more scratch than the array holds is
refused with QI_HIP_INVALID_INPUT.
"""
import numpy as np
import pytest

import quantinfer_amd as qa
from oracle import pyoracle as po

pytestmark = pytest.mark.gpu


def _noalloc():
    return qa.lib().qi_hip_linear_device_noalloc  # the C entry point (argument types set by qa.lib())


@pytest.fixture(scope="module")
def ctx():
    c = qa.Context(0)
    yield c
    c.close()


CASES = [
    # (qtype, layout, K, N, first M, second M, mode): what the plan uses
    (qa.Q4_K, qa.OUTPUT_ROWS, 4096, 4096, 512, 8, qa.MODE_AUTO),     # GEMM + split-K partials, then 8-row GEMV K parts
    (qa.Q8_0, qa.OUTPUT_ROWS, 4096, 12288, 2048, 130, qa.MODE_AUTO),  # GEMM without, then with a K split
    (qa.Q6_K, qa.OUTPUT_ROWS, 4096, 1024, 200, 1, qa.MODE_MFMA),     # the Q6_K GEMM, then one row
    (qa.Q5_K, qa.OUTPUT_ROWS, 1024, 512, 16, 3, qa.MODE_F32),        # 2-16 row GEMV with K parts
    (qa.Q4_0, qa.OUTPUT_ROWS, 4096, 12288, 16, 9, qa.MODE_F32),      # 2-16 row GEMV, activation records
    (qa.Q6_K, qa.OUTPUT_ROWS, 14336, 4096, 16, 9, qa.MODE_F32),      # Q6_K 2-16 rows: records and K parts
    (qa.Q4_K, qa.OUTPUT_ROWS, 4096, 1024, 100, 50, qa.MODE_F32),     # split-half GEMM: records and K parts
    (qa.Q4_0, qa.ROW_MAJOR, 4096, 4096, 9, 1, qa.MODE_F32),          # row-major GEMM K parts, then the GEMV's
    (qa.Q4_K, qa.ROW_MAJOR, 4096, 4096, 130, 2, qa.MODE_F32),        # row-major GEMM, 32-row tiles, then 2-row GEMV
    (qa.Q4_K, qa.OUTPUT_ROWS, 512, 64, 5, 2, qa.MODE_EXACT),         # no workspace
    (qa.F32, qa.ROW_MAJOR, 1024, 2000, 40, 12, qa.MODE_F32),          # F32 weights: GEMM, then GEMV K parts
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"q{c[0]}-l{c[1]}-{c[2]}x{c[3]}-m{c[4]}-{c[5]}-mode{c[6]}")
def test_noalloc_equals_linear_device(ctx, case):
    from quantinfer_amd import hiprt
    qtype, layout, k, n, m1, m2, mode = case
    print(f"no-alloc case {case}", flush=True)
    if qtype == qa.F32:
        blocks = po.fill_normal(9500, k * n, 0.02).reshape(k, n)
    elif layout == qa.OUTPUT_ROWS:
        blocks = po.make_weights(qtype, k, n, seed=9500 + qtype, outliers=qtype >= qa.Q4_K)
    else:
        blocks = po.make_weights(qtype, n, k, seed=9500 + qtype)
    w = ctx.weights(qtype, layout, k, n, blocks)
    stream = hiprt.Stream()
    f = _noalloc()
    outs = {}
    for m in (m1, m2):
        x = po.fill_normal(9600 + m, m * k).reshape(m, k)
        xd = hiprt.DeviceBuffer.from_array(x)
        ya, yb = hiprt.DeviceBuffer(m * n * 4), hiprt.DeviceBuffer(m * n * 4)
        w.linear_device(xd.ptr, m, ya.ptr, mode, stream.handle)
        stream.synchronize()
        outs[m] = (xd, ya, yb)
    # two no-allocation calls back to back, the second smaller, no host sync between
    for m in (m1, m2):
        xd, _, yb = outs[m]
        assert f(ctx.handle, w.handle, xd.ptr, m, yb.ptr, mode, stream.handle) == qa.OK, \
            qa.lib().qi_hip_last_error().decode()
    stream.synchronize()
    for m in (m1, m2):
        _, ya, yb = outs[m]
        a = ya.to_array(np.float32, (m, n))
        b = yb.to_array(np.float32, (m, n))
        assert a.tobytes() == b.tobytes(), m
        assert np.isfinite(a).all()
    stream.destroy()
    w.free()


def test_noalloc_refuses_calls_beyond_its_scratch(ctx):
    """4096 rows of K = 12288 need 96 MiB of f16 activations: more than the
    64 MiB the array holds."""
    from quantinfer_amd import hiprt
    k, n, m = 12288, 256, 4096
    blocks = po.make_weights(qa.Q8_0, k, n, seed=9700)
    w = ctx.weights(qa.Q8_0, qa.OUTPUT_ROWS, k, n, blocks)
    xd, yd = hiprt.DeviceBuffer(m * k * 4), hiprt.DeviceBuffer(m * n * 4)
    st = _noalloc()(ctx.handle, w.handle, xd.ptr, m, yd.ptr, qa.MODE_AUTO, None)
    assert st == qa.INVALID_INPUT
    assert "scratch" in qa.lib().qi_hip_last_error().decode()
    w.free()
