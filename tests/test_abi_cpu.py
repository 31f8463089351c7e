"""CPU tests of the C-ABI library: it loads, exports every entry point that
include/qi_hip.h declares, reports a missing device as UNSUPPORTED, and its
host-side validation and packing (qi_hip_pack_weights, the same code path as
qi_hip_weights_create) match the reference rules and the oracle's GGUF wire
bytes. No compute call is made here."""
import ctypes
import os
import re

import numpy as np
import pytest

import quantinfer_amd as qa
from oracle import pyoracle as po

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ALL_Q = [qa.Q8_0, qa.Q4_0, qa.Q4_K, qa.Q5_K, qa.Q6_K]


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "qi_hip.h")).read()
    return sorted(set(re.findall(r"\b(qi_hip_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = qa.lib()
    names = declared_symbols()
    assert len(names) >= 13
    for name in names:
        assert hasattr(lib, name), name
    assert lib.qi_hip_abi_version() == 1


def test_block_structs_match_reference_layout():
    for q in ALL_Q:
        assert qa.BLOCK_DTYPES[q] == po.BLOCK_DTYPES[q]
    assert [qa.BLOCK_DTYPES[q].itemsize for q in ALL_Q] == [36, 36, 148, 180, 212]


def test_open_without_device_is_unsupported():
    try:
        c = qa.Context(0)
    except qa.QiError as err:
        assert err.status == qa.UNSUPPORTED
        assert qa.lib().qi_hip_last_error().decode()
    else:
        c.close()
        pytest.skip("a gfx950 device is visible")


def _planes(qtype, image, count, f16):
    """Split an image into its planes (offsets: 256-byte aligned, in the order
    qs, qh, sc, d, dmin)."""
    sizes = {qa.Q8_0: (32, 0, 0, False), qa.Q4_0: (16, 0, 0, False), qa.Q4_K: (128, 0, 12, True),
             qa.Q5_K: (128, 32, 12, True), qa.Q6_K: (128, 64, 16, False)}[qtype]
    sb = 2 if f16 else 4
    al = lambda x: (x + 255) // 256 * 256
    off = 0
    out = {}
    for name, per in (("qs", sizes[0]), ("qh", sizes[1]), ("sc", sizes[2]), ("d", sb),
                      ("dmin", sb if sizes[3] else 0)):
        out[name] = image[off:off + per * count]
        off = al(off + per * count)
    return out


@pytest.mark.parametrize("qtype", ALL_Q)
def test_packed_planes_hold_exactly_the_wire_bytes(qtype):
    k, n = 512, 6
    blocks = po.make_weights(qtype, k, n, seed=21 + qtype, outliers=True)
    image, f16 = qa.pack_weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
    assert f16
    count = blocks.size
    p = _planes(qtype, image, count, True)
    wire = po.wire_pack(qtype, blocks).reshape(count, po.WIRE_BYTES[qtype])
    if qtype == qa.Q8_0:
        assert np.array_equal(p["d"].view("<u2"), wire[:, 0:2].copy().view("<u2").ravel())
        assert np.array_equal(p["qs"].reshape(count, 32), wire[:, 2:34])
    elif qtype == qa.Q4_0:
        assert np.array_equal(p["d"].view("<u2"), wire[:, 0:2].copy().view("<u2").ravel())
        assert np.array_equal(p["qs"].reshape(count, 16), wire[:, 2:18])
    elif qtype in (qa.Q4_K, qa.Q5_K):
        assert np.array_equal(p["d"].view("<u2"), wire[:, 0:2].copy().view("<u2").ravel())
        assert np.array_equal(p["dmin"].view("<u2"), wire[:, 2:4].copy().view("<u2").ravel())
        assert np.array_equal(p["sc"].reshape(count, 12), wire[:, 4:16])
        if qtype == qa.Q4_K:
            assert np.array_equal(p["qs"].reshape(count, 128), wire[:, 16:144])
        else:
            assert np.array_equal(p["qh"].reshape(count, 32), wire[:, 16:48])
            assert np.array_equal(p["qs"].reshape(count, 128), wire[:, 48:176])
    else:
        assert np.array_equal(p["qs"].reshape(count, 128), wire[:, 0:128])
        assert np.array_equal(p["qh"].reshape(count, 64), wire[:, 128:192])
        assert np.array_equal(p["sc"].reshape(count, 16), wire[:, 192:208])
        assert np.array_equal(p["d"].view("<u2"), wire[:, 208:210].copy().view("<u2").ravel())
    payload = sum(v.size for v in p.values())
    assert payload == po.WIRE_BYTES[qtype] * count  # the image of an f16 tensor has wire size


def test_unrounded_scales_switch_to_f32_planes():
    # quantize_q8_0 keeps absmax/127 unrounded (quant/src/schemes/q8.rs:19)
    blocks = po.quantize(po.Q8_0, po.fill_normal(3, 64 * 4, 0.02))
    image, f16 = qa.pack_weights(qa.Q8_0, qa.OUTPUT_ROWS, 64, 4, blocks)
    assert not f16
    p = _planes(qa.Q8_0, image, blocks.size, False)
    assert np.array_equal(p["d"].view("<f4"), blocks["scale"])


def _expect_invalid(*args):
    with pytest.raises(qa.QiError) as err:
        qa.pack_weights(*args)
    assert err.value.status == qa.INVALID_INPUT
    return str(err.value)


def test_validation_follows_reference_rules():
    b = po.make_weights(po.Q8_0, 64, 2, seed=1)
    # block count must match the shape (core quantized/q8.rs:29-33)
    _expect_invalid(qa.Q8_0, qa.OUTPUT_ROWS, 64, 3, b)
    # zero dimensions (core tensor.rs:85-93)
    _expect_invalid(qa.Q8_0, qa.OUTPUT_ROWS, 0, 2, b[:0])
    # output rows need K % 32 == 0 (backends/cpu/src/matmul.rs:136-140) ...
    _expect_invalid(qa.Q8_0, qa.OUTPUT_ROWS, 48, 4, np.concatenate([b, b[:2]])[:6])
    # ... while row major only needs K*N % 32 == 0
    qa.pack_weights(qa.Q8_0, qa.ROW_MAJOR, 48, 4, np.concatenate([b, b])[:6])
    # Q4_0 codes must fit in four bits (core quantized/q4.rs:36-44)
    q4 = po.make_weights(po.Q4_0, 32, 1, seed=2)
    q4["values"][0, 5] = 16
    assert "four bits" in _expect_invalid(qa.Q4_0, qa.OUTPUT_ROWS, 32, 1, q4)
    # finite scales (core quantized/q8.rs:34-38, k.rs:171-178)
    bad = b.copy()
    bad["scale"][1] = np.nan
    _expect_invalid(qa.Q8_0, qa.OUTPUT_ROWS, 64, 2, bad)
    k5 = po.make_weights(po.Q5_K, 256, 1, seed=3)
    k5["min_scale"][0] = np.inf
    _expect_invalid(qa.Q5_K, qa.OUTPUT_ROWS, 256, 1, k5)
    # K-quant output rows need K % 256 == 0 (matmul.rs:299-314)
    k4 = po.make_weights(po.Q4_K, 256, 2, seed=4)
    _expect_invalid(qa.Q4_K, qa.OUTPUT_ROWS, 128, 4, k4)
    # unknown type / layout
    _expect_invalid(9, qa.OUTPUT_ROWS, 64, 2, b)
    _expect_invalid(qa.Q8_0, 7, 64, 2, b)
    # F32 weights are row-major [K, N] with K*N values
    w = np.ones(12, dtype=np.float32)
    qa.pack_weights(qa.F32, qa.ROW_MAJOR, 3, 4, w)
    _expect_invalid(qa.F32, qa.ROW_MAJOR, 3, 5, w)
    _expect_invalid(qa.F32, qa.OUTPUT_ROWS, 3, 4, w)


def test_null_arguments_are_invalid_not_crashes():
    lib = qa.lib()
    assert lib.qi_hip_linear(None, None, None, 1, None, 0) == qa.INVALID_INPUT
    assert lib.qi_hip_linear_device(None, None, None, 1, None, 0, None) == qa.INVALID_INPUT
    assert lib.qi_hip_dequantize(None, None, None) == qa.INVALID_INPUT
    assert lib.qi_hip_weights_info_get(None, None) == qa.INVALID_INPUT
    assert lib.qi_hip_open(0, None) == qa.INVALID_INPUT
    size = ctypes.c_uint64(0)
    assert lib.qi_hip_pack_weights(1, 1, 32, 1, None, 1, None, ctypes.byref(size), None) == qa.INVALID_INPUT
    lib.qi_hip_close(None)
    lib.qi_hip_weights_free(None)
