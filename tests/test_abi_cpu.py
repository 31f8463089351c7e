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


def test_measurement_libraries_stay_out_of_the_product():
    """The streaming-read calibration lives in its own library and the
    timeline stamps only in the profiling build: the product library exports
    neither."""
    from quantinfer_amd import build as qb
    lib_syms = open(qa.LIB_PATH, "rb").read()
    assert b"qi_timeline_read" not in lib_syms and b"qi_calib_stream_read" not in lib_syms
    cal = ctypes.CDLL(qb.CALIB_LIB)
    assert hasattr(cal, "qi_calib_stream_read")
    if os.path.exists(qb.TIMELINE_LIB):
        tl = ctypes.CDLL(qb.TIMELINE_LIB)
        assert hasattr(tl, "qi_timeline_read") and hasattr(tl, "qi_timeline_clear")


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


SIZES = {qa.Q8_0: (32, 0, 0, False), qa.Q4_0: (16, 0, 0, False), qa.Q4_K: (128, 0, 12, True),
         qa.Q5_K: (128, 32, 12, True), qa.Q6_K: (128, 64, 16, False)}


def _planes(qtype, image, count, f16):
    """Split a planar image into its planes (offsets: 256-byte aligned, in the
    order qs, qh, sc, d, dmin)."""
    sizes = SIZES[qtype]
    sb = 2 if f16 else 4
    al = lambda x: (x + 255) // 256 * 256
    off = 0
    out = {}
    for name, per in (("qs", sizes[0]), ("qh", sizes[1]), ("sc", sizes[2]), ("d", sb),
                      ("dmin", sb if sizes[3] else 0)):
        out[name] = image[off:off + per * count]
        off = al(off + per * count)
    return out


def _check_wire_fields(qtype, fields, wire):
    """fields: per block (qs, qh, sc, d, dmin) byte arrays; wire: GGUF blocks."""
    count = wire.shape[0]
    qs, qh, sc, d, dmin = (np.asarray(f, dtype=np.uint8).reshape(count, -1) for f in fields)
    if qtype == qa.Q8_0:
        assert np.array_equal(d, wire[:, 0:2]) and np.array_equal(qs, wire[:, 2:34])
    elif qtype == qa.Q4_0:
        assert np.array_equal(d, wire[:, 0:2]) and np.array_equal(qs, wire[:, 2:18])
    elif qtype in (qa.Q4_K, qa.Q5_K):
        assert np.array_equal(d, wire[:, 0:2]) and np.array_equal(dmin, wire[:, 2:4])
        assert np.array_equal(sc, wire[:, 4:16])
        if qtype == qa.Q4_K:
            assert np.array_equal(qs, wire[:, 16:144])
        else:
            assert np.array_equal(qh, wire[:, 16:48]) and np.array_equal(qs, wire[:, 48:176])
    else:
        assert np.array_equal(qs, wire[:, 0:128]) and np.array_equal(qh, wire[:, 128:192])
        assert np.array_equal(sc, wire[:, 192:208]) and np.array_equal(d, wire[:, 208:210])


@pytest.mark.parametrize("qtype", ALL_Q)
def test_planar_image_holds_exactly_the_wire_bytes(qtype):
    # row-major weights keep one plane per field in the reference block order
    k, n = 512, 6
    blocks = po.make_weights(qtype, k, n, seed=21 + qtype, outliers=True)
    image, f16 = qa.pack_weights(qtype, qa.ROW_MAJOR, k, n, blocks)
    assert f16
    count = blocks.size
    p = _planes(qtype, image, count, True)
    wire = po.wire_pack(qtype, blocks).reshape(count, po.WIRE_BYTES[qtype])
    empty = np.zeros((count, 0), np.uint8)
    _check_wire_fields(qtype, [p["qs"], p["qh"] if p["qh"].size else empty, p["sc"] if p["sc"].size else empty,
                               p["d"], p["dmin"] if p["dmin"].size else empty], wire)
    payload = sum(v.size for v in p.values())
    assert payload == po.WIRE_BYTES[qtype] * count  # the image of an f16 tensor has wire size


def _kq_packed_from_fields(sc):
    """Tiled Q4_K/Q5_K scale bytes -> the GGUF 12-byte packing. The tiled
    record holds field g = sc[2g] | m[2g] << 6 | sc[2g+1] << 12 | m[2g+1] << 18
    at bytes 3g..3g+2; the GGUF packing (format gguf/writer.rs:216-219, read
    back by backends/cpu/src/matmul.rs:192-201) keeps sc[i], m[i] (i < 4) in the
    low 6 bits of bytes i, 4+i, their top bits holding bits 4-5 of sc[4+i],
    m[4+i], whose low 4 bits fill bytes 8+i."""
    sc = np.asarray(sc, dtype=np.uint32)
    f = [int(sc[3 * g]) | int(sc[3 * g + 1]) << 8 | int(sc[3 * g + 2]) << 16 for g in range(4)]
    s = [0] * 8
    m = [0] * 8
    for g in range(4):
        s[2 * g], m[2 * g] = f[g] & 63, (f[g] >> 6) & 63
        s[2 * g + 1], m[2 * g + 1] = (f[g] >> 12) & 63, (f[g] >> 18) & 63
    out = [0] * 12
    for i in range(4):
        out[i] = s[i] | ((s[4 + i] >> 4) << 6)
        out[4 + i] = m[i] | ((m[4 + i] >> 4) << 6)
        out[8 + i] = (s[4 + i] & 15) | ((m[4 + i] & 15) << 4)
    return np.asarray(out, dtype=np.uint8)


def _q6_scales_from_tiled(sc):
    """Tiled Q6_K sub-scales -> reference order: lane group g = 2ip + h holds
    sub-scales 8ip + 2h + {0, 1, 4, 5} at bytes 4g..4g+3."""
    out = np.zeros(16, dtype=np.uint8)
    for g in range(4):
        ip, h = divmod(g, 2)
        for j, off in enumerate((0, 1, 4, 5)):
            out[8 * ip + 2 * h + off] = sc[4 * g + j]
    return out


def _untile(qtype, image, k, n, f16):
    """Per-block fields of a tiled output-rows image, read back from the record
    arrangement: records of (16-output tile, 256-element unit) ordered
    [tile][unit]; inside a record the code slice of row c (its unit's code bytes
    in block order) is cut in four lane groups and 16-byte chunks, chunk q of
    group g at q*1024 + (16g + c)*16; qh chunk h at h*256 + c*16; scales at
    c*|sc| (K-quants regrouped per lane group, returned here in GGUF order); d
    entries at c*bpu + block; dmin at c. Also returns the bytes of the padding
    rows."""
    qsb, qhb, scb, has_dmin = SIZES[qtype]
    bpu = 8 if qtype in (qa.Q8_0, qa.Q4_0) else 1
    ss = 2 if f16 else 4
    slice_ = qsb * bpu
    off_qh = 16 * slice_
    off_sc = off_qh + 16 * qhb
    off_d = off_sc + 16 * scb
    off_dm = off_d + 16 * bpu * ss
    rec_bytes = -(-(off_dm + (16 * ss if has_dmin else 0)) // 16) * 16
    tiles, units = -(-n // 16), k // 256
    assert image.size == tiles * units * rec_bytes + 256
    nb = k // (32 if bpu == 8 else 256)
    fields = [[] for _ in range(5)]
    pad = []
    for row in range(tiles * 16):
        t, c = divmod(row, 16)
        for u in range(units):
            rec = image[(t * units + u) * rec_bytes:(t * units + u + 1) * rec_bytes]
            quarter = slice_ // 4
            code = np.concatenate([rec[q * 1024 + (16 * g + c) * 16:][:16]
                                   for g in range(4) for q in range(quarter // 16)])
            qh = np.concatenate([rec[off_qh + h * 256 + c * 16:][:16] for h in range(qhb // 16)] or [[]])
            sc = rec[off_sc + c * scb:][:scb]
            if qtype in (qa.Q4_K, qa.Q5_K):
                sc = _kq_packed_from_fields(sc)
            elif qtype == qa.Q6_K:
                sc = _q6_scales_from_tiled(sc)
            per = [(code[bi * qsb:(bi + 1) * qsb], qh, sc, rec[off_d + (c * bpu + bi) * ss:][:ss],
                    rec[off_dm + c * ss:][:ss] if has_dmin else np.zeros(0, np.uint8)) for bi in range(bpu)]
            if row < n:
                for blk in per:
                    for i in range(5):
                        fields[i].append(blk[i])
            else:
                pad.extend(np.concatenate(blk) for blk in per)
    assert len(fields[0]) == n * nb
    return [np.concatenate(f) if f and f[0].size else np.zeros((n * nb, 0), np.uint8) for f in fields], pad


@pytest.mark.parametrize("qtype", ALL_Q)
def test_tiled_image_holds_exactly_the_wire_bytes(qtype):
    # output rows with K a multiple of 256: tile records; 21 outputs leave
    # 11 padding rows in the second tile, which must read as zero
    k, n = 512, 21
    blocks = po.make_weights(qtype, k, n, seed=41 + qtype, outliers=True)
    image, f16 = qa.pack_weights(qtype, qa.OUTPUT_ROWS, k, n, blocks)
    assert f16
    fields, pad = _untile(qtype, image, k, n, True)
    wire = po.wire_pack(qtype, blocks).reshape(blocks.size, po.WIRE_BYTES[qtype])
    _check_wire_fields(qtype, fields, wire)
    assert pad and not any(p.any() for p in pad)


@pytest.mark.parametrize("qtype", ALL_Q)
def test_tiled_row_major_image_holds_exactly_the_wire_bytes(qtype):
    # row major with N a multiple of 256: the records of the output-rows
    # arrangement with a row per k (its N / bs blocks, flat block k * N/bs + b);
    # K = 40 leaves 8 padding rows in the third tile
    k, n = 40, 512
    blocks = po.make_weights(qtype, n, k, seed=43 + qtype, outliers=True)  # [K][N/bs] blocks along N
    image, f16 = qa.pack_weights(qtype, qa.ROW_MAJOR, k, n, blocks)
    assert f16
    fields, pad = _untile(qtype, image, n, k, True)
    wire = po.wire_pack(qtype, blocks).reshape(blocks.size, po.WIRE_BYTES[qtype])
    _check_wire_fields(qtype, fields, wire)
    assert pad and not any(p.any() for p in pad)


def test_tiled_image_with_unrounded_scales_keeps_f32_entries():
    blocks = po.quantize(po.Q8_0, po.fill_normal(5, 256 * 3, 0.02))
    image, f16 = qa.pack_weights(qa.Q8_0, qa.OUTPUT_ROWS, 256, 3, blocks)
    assert not f16
    fields, _ = _untile(qa.Q8_0, image, 256, 3, False)
    assert np.array_equal(fields[3].view("<f4"), blocks["scale"])


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


# ------------------------------------------------ direct GGUF upload (host image)
GOLDEN = os.path.join(ROOT, "tests", "golden", "reference_known_answers.json")
NAME_Q = {"q4_0": qa.Q4_0, "q6_k": qa.Q6_K, "q4_k": qa.Q4_K}


def _golden_block(qtype, spec):
    b = np.zeros(1, dtype=po.BLOCK_DTYPES[qtype])
    for field, value in spec.items():
        b[field][0] = value
    return b


def test_gguf_upload_matches_reference_wire_vectors():
    """The reference's own standard and legacy wire bytes (format/src/gguf/
    tests.rs:163-212) decode to the image of the block they encode."""
    import json
    cases = [e for e in json.load(open(GOLDEN))["wire"] if e.get("qtype") in NAME_Q and "block" in e]
    assert {e["qtype"] for e in cases} >= {"q4_0", "q6_k"}
    for e in cases:
        q = NAME_Q[e["qtype"]]
        k = po.BLOCK_ELEMS[q]
        block = _golden_block(q, e["block"])
        want, _ = qa.pack_weights(q, qa.OUTPUT_ROWS, k, 1, block)
        for key, legacy in (("standard_bytes", False), ("legacy_bytes", True)):
            if key in e:
                got, f16 = qa.pack_gguf(q, qa.OUTPUT_ROWS, k, 1, bytes(e[key]), legacy=legacy)
                assert f16 and got.tobytes() == want.tobytes(), (e["name"], key)
        if "standard_bytes" not in e:
            wire = po.wire_pack(q, block)
            got, _ = qa.pack_gguf(q, qa.OUTPUT_ROWS, k, 1, wire)
            assert got.tobytes() == want.tobytes(), e["name"]


@pytest.mark.parametrize("qtype", ALL_Q, ids=lambda q: po.NAMES[q] if hasattr(po, "NAMES") else str(q))
def test_gguf_upload_equals_logical_upload(qtype):
    """Standard wire bytes from the oracle's GGUF writer restatement give the
    same device image as the logical blocks, for the tiled (K % 256 == 0) and
    the planar (K % 256 != 0, Q8_0/Q4_0) images and both layouts."""
    shapes = [(512, 48, qa.OUTPUT_ROWS)]
    if po.BLOCK_ELEMS[qtype] == 32:
        shapes += [(96, 40, qa.OUTPUT_ROWS), (64, 96, qa.ROW_MAJOR)]
    else:
        shapes += [(256, 512, qa.ROW_MAJOR)]
    for k, n, layout in shapes:
        blocks = po.make_weights(qtype, k, n, seed=0x66 + qtype + k, outliers=True)
        if layout == qa.ROW_MAJOR:
            blocks = po.make_weights(qtype, n, k, seed=0x67 + qtype)  # [K][N/bs] blocks along N
        want, wf16 = qa.pack_weights(qtype, layout, k, n, blocks)
        got, gf16 = qa.pack_gguf(qtype, layout, k, n, po.wire_pack(qtype, blocks))
        assert wf16 and gf16
        assert got.tobytes() == want.tobytes(), (k, n, layout)


@pytest.mark.parametrize("qtype", [qa.Q4_0, qa.Q6_K], ids=["q4_0", "q6_k"])
def test_gguf_upload_legacy_layout(qtype):
    """Random legacy-layout bytes with finite f16 scales: the library's reader
    equals the oracle's restatement of decode.rs (legacy branches :168-172,
    :288-290)."""
    rng = np.random.default_rng(0x1E6 + qtype)
    wb = {qa.Q4_0: 18, qa.Q6_K: 210}[qtype]
    k, n = (64, 8) if qtype == qa.Q4_0 else (256, 8)
    count = n * k // po.BLOCK_ELEMS[qtype]
    raw = np.frombuffer(rng.bytes(count * wb), dtype=np.uint8).copy().reshape(count, wb)
    scale = np.float16(rng.uniform(0.001, 0.01, count)).view(np.uint8).reshape(count, 2)
    at = 0 if qtype == qa.Q4_0 else 0  # legacy: d first for both
    raw[:, at:at + 2] = scale
    logical = po.wire_unpack(qtype, raw.tobytes(), legacy=True)
    want, _ = qa.pack_weights(qtype, qa.OUTPUT_ROWS, k, n, logical)
    got, _ = qa.pack_gguf(qtype, qa.OUTPUT_ROWS, k, n, raw.tobytes(), legacy=True)
    assert got.tobytes() == want.tobytes()
    # the standard reader on the same bytes decodes something else
    if qtype == qa.Q4_0:
        std, _ = qa.pack_gguf(qtype, qa.OUTPUT_ROWS, k, n, raw.tobytes(), legacy=False)
        assert std.tobytes() != want.tobytes()


def test_gguf_upload_errors():
    blocks = po.make_weights(po.Q8_0, 64, 2, seed=9)
    wire = po.wire_pack(po.Q8_0, blocks)
    for bad, what in ((wire[:-1], "byte length"), (wire[:34], "does not match")):
        with pytest.raises(qa.QiError) as e:
            qa.pack_gguf(qa.Q8_0, qa.OUTPUT_ROWS, 64, 2, bad)
        assert e.value.status == qa.INVALID_INPUT
    inf = wire.copy()
    inf[34:36] = np.frombuffer(np.float16(np.inf).tobytes(), dtype=np.uint8)
    with pytest.raises(qa.QiError) as e:
        qa.pack_gguf(qa.Q8_0, qa.OUTPUT_ROWS, 64, 2, inf)
    assert e.value.status == qa.INVALID_INPUT and "non-finite" in str(e.value)
    k4 = po.wire_pack(po.Q4_K, po.make_weights(po.Q4_K, 256, 1, seed=10))
    k4[2:4] = np.frombuffer(np.float16(np.nan).tobytes(), dtype=np.uint8)  # dmin
    with pytest.raises(qa.QiError) as e:
        qa.pack_gguf(qa.Q4_K, qa.OUTPUT_ROWS, 256, 1, k4)
    assert e.value.status == qa.INVALID_INPUT
    with pytest.raises(qa.QiError) as e:
        qa.pack_gguf(9, qa.OUTPUT_ROWS, 256, 1, k4)
    assert e.value.status == qa.UNSUPPORTED
    # F32 passes little-endian values through
    vals = np.arange(12, dtype=np.float32)
    got, _ = qa.pack_gguf(qa.F32, qa.ROW_MAJOR, 3, 4, vals.tobytes())
    want, _ = qa.pack_weights(qa.F32, qa.ROW_MAJOR, 3, 4, vals)
    assert got.tobytes() == want.tobytes()


# ------------------------------------------------------ host quantizer

def _quantizer_inputs():
    from tests.test_oracle_quantizers import _k_grid_input
    yield "normal_outliers", po.fill_normal(0x5EED0002, 256 * 200, 0.02, 0.005, 0.2)
    yield "k_grid", _k_grid_input()
    yield "unit_normal", po.fill_normal(3, 256 * 40, 1.0)
    yield "zeros_and_tiny", np.concatenate([np.zeros(256, np.float32), np.full(256, 1e-8, np.float32),
                                            np.full(256, -3e-39, np.float32)])
    yield "large", po.fill_normal(4, 256 * 8, 300.0)


@pytest.mark.parametrize("qtype", ALL_Q)
@pytest.mark.parametrize("storage_f16", [False, True])
def test_quantize_equals_oracle_quantizer(qtype, storage_f16):
    """qi_hip_quantize produces the oracle's (the reference quantizer's) blocks
    byte for byte, with and without f16 storage rounding, for any thread count."""
    for name, x in _quantizer_inputs():
        ref = po.quantize(qtype, x)
        if storage_f16:
            ref = po.storage_precision(qtype, ref)
        for threads in (1, 3, 0):
            ours = qa.quantize(qtype, x, storage_f16=storage_f16, threads=threads)
            assert ours.tobytes() == ref.tobytes(), (name, threads)


@pytest.mark.parametrize("qtype", ALL_Q)
def test_quantize_rejects_what_the_reference_rejects(qtype):
    bs = qa.BLOCK_ELEMS[qtype]
    x = np.ones(bs, dtype=np.float32)
    x[3] = np.nan
    with pytest.raises(qa.QiError) as e:
        qa.quantize(qtype, x)
    assert e.value.status == qa.INVALID_INPUT
    x[3] = np.inf
    with pytest.raises(qa.QiError):
        qa.quantize(qtype, x)
    # element count not a multiple of the block size; output count mismatch
    out = np.zeros(1, qa.BLOCK_DTYPES[qtype])
    x[3] = 1.0
    assert qa.lib().qi_hip_quantize(qtype, x.ctypes.data, bs - 1, 0, out.ctypes.data, 0, 1) == qa.INVALID_INPUT
    assert qa.lib().qi_hip_quantize(qtype, x.ctypes.data, bs, 0, out.ctypes.data, 2, 1) == qa.INVALID_INPUT
    assert qa.lib().qi_hip_quantize(qtype, x.ctypes.data, bs, 0, out.ctypes.data, 1, 1) == qa.OK
    # f32::MAX input: the K-quant super-block scale overflows f16
    # (k_grid_tests.rs:148-155); Q8_0/Q4_0 keep f32 scales unless stored as f16
    big = np.full(bs, np.finfo(np.float32).max, dtype=np.float32)
    if qtype in (qa.Q4_K, qa.Q5_K, qa.Q6_K):
        with pytest.raises(qa.QiError):
            qa.quantize(qtype, big)
        with pytest.raises(po.OracleError):
            po.quantize(qtype, big)
    else:
        assert qa.quantize(qtype, big).tobytes() == po.quantize(qtype, big).tobytes()
        with pytest.raises(qa.QiError):
            qa.quantize(qtype, big, storage_f16=True)


def test_synth_normal_equals_oracle_generator():
    for args in ((0x5EED0002, 1 << 21, 0.02, 0.005, 0.2), (7, 1000, 1.0, 0.0, 0.0),
                 (1, 300001, 0.02, 0.5, 0.2)):
        ref = po.fill_normal(*args)
        for threads in (1, 5, 0):
            assert qa.synth_normal(*args, threads=threads).tobytes() == ref.tobytes()


# ------------------------------------------- the Rust crate (backends/hip)

def test_rust_crate_builds_the_same_sources_and_flags():
    """backends/hip/build.rs compiles the translation units listed in
    quantinfer_amd/csrc/sources.txt (the list build.py builds), with build.py's
    code-generation flags."""
    from quantinfer_amd import build as qb
    rs = open(os.path.join(ROOT, "backends", "hip", "build.rs")).read()
    assert 'join("sources.txt")' in rs and "quantinfer_amd/csrc" in rs
    listed = [ln.strip() for ln in open(os.path.join(ROOT, "quantinfer_amd", "csrc", "sources.txt"))
              if ln.strip() and not ln.startswith("#")]
    assert listed == qb.SOURCES
    for f in listed:
        assert os.path.exists(os.path.join(ROOT, "quantinfer_amd", "csrc", f)), f
    # every file under csrc that defines code is listed
    code = sorted(f for f in os.listdir(os.path.join(ROOT, "quantinfer_amd", "csrc"))
                  if f.endswith((".hip", ".cpp")))
    assert sorted(listed) == code
    flags = re.search(r"const FLAGS: &\[&str\] = &\[(.*?)\];", rs, re.S).group(1)
    rs_flags = re.findall(r'"([^"]+)"', flags)
    codegen = [f for f in qb.FLAGS if not f.startswith("-W")]
    assert rs_flags == codegen
    per_file = re.search(r"const FILE_FLAGS: &\[\(&str, &\[&str\]\)\] = &\[(.*?)\];", rs, re.S).group(1)
    rs_per_file = {m.group(1): re.findall(r'"([^"]+)"', m.group(2))
                   for m in re.finditer(r'\("([^"]+)",\s*&\[(.*?)\]\)', per_file, re.S)}
    assert rs_per_file == qb.FILE_FLAGS


def test_rust_ffi_declares_every_header_function():
    ffi = open(os.path.join(ROOT, "backends", "hip", "src", "ffi.rs")).read()
    declared = sorted(set(re.findall(r"pub fn (qi_hip_[a-z_0-9]+)\s*\(", ffi)))
    assert declared == declared_symbols()
    # block structs: the header's field order and sizes
    for name, fields in (("Q8_0", ["scale", "values"]), ("Q4_0", ["scale", "values"]),
                         ("Q4K", ["scale", "min_scale", "scales", "values"]),
                         ("Q5K", ["scale", "min_scale", "scales", "high_bits", "values"]),
                         ("Q6K", ["scale", "scales", "low_bits", "high_bits"])):
        body = re.search(r"pub struct %s \{(.*?)\}" % name, ffi, re.S).group(1)
        assert re.findall(r"pub (\w+):", body) == fields, name


# ------------------------------------------- planner arithmetic (host only)

def _planner(name, *argtypes):
    fn = getattr(qa.lib(), name)
    fn.argtypes = list(argtypes)
    fn.restype = ctypes.c_uint32
    return fn


def test_gemv_rows_split_count_gives_every_part_units():
    """The 2-16 row GEMVs' launches give each of their `s` K parts
    ceil(units/s) units and refuse a split count whose parts would not all
    hold units. The planners (qi::gemv_rows_splits for 2-8 rows,
    qi::gemv_half_splits for 9-16, host code in the library) must return a
    count the launch accepts for every shape: K = 8960, N = 1536 at 2-4 rows
    once asked for 8 parts of 5 units (7 parts cover K)."""
    for name, rows in (("_ZN2qi16gemv_rows_splitsEmmj", range(2, 9)), ("_ZN2qi16gemv_half_splitsEmmj", range(9, 17))):
        splits = _planner(name, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32)
        seen = set()
        for units in range(1, 129):
            k = 256 * units
            for n in list(range(16, 4097, 16)) + [4100, 12288, 14336]:
                for m in rows:
                    s = splits(k, n, m)
                    assert 1 <= s <= units, (name, k, n, m, s)
                    part = -(-units // s)
                    assert -(-units // part) == s, (name, k, n, m, s)
                    seen.add(s)
        assert len(seen) > 8  # the sweep reaches many split counts
        assert splits(8960, 1536, 2) == 7 and splits(6400, 1024, 8) == 5


def _rust_paths():
    """Every (crate, name) that backends/hip/src/*.rs takes from a
    quantinfer crate: `use quantinfer_x::{a, b}`, `use quantinfer_x::a` and
    qualified paths `quantinfer_x::Name` in the code."""
    src = os.path.join(ROOT, "backends", "hip", "src")
    used = set()
    for f in sorted(os.listdir(src)):
        text = open(os.path.join(src, f)).read()
        text = re.sub(r"//[^\n]*", "", text)  # comments name crates too
        for crate, body in re.findall(r"\buse\s+(quantinfer_\w+)::\{([^}]*)\}", text):
            used.update((crate, n.strip()) for n in body.split(",") if n.strip())
        for crate, name in re.findall(r"\buse\s+(quantinfer_\w+)::(\w+)\s*;", text):
            used.add((crate, name))
        for crate, name in re.findall(r"(?<!use )\b(quantinfer_\w+)::(\w+)\b(?!::\{)", text):
            used.add((crate, name))
    return used


def test_rust_crate_imports_exist_in_the_reference():
    """Each name the crate imports is public in the reference crate it is
    taken from (the committed list cites the line that exports it), and each
    crate it uses is a dependency in its Cargo.toml."""
    import json
    ref = json.load(open(os.path.join(ROOT, "tests", "golden", "reference_rust_exports.json")))
    used = _rust_paths()
    assert ("quantinfer_model", "Qwen3Config") in used
    for crate, name in sorted(used):
        assert name in ref["exports"].get(crate, {}), f"{crate}::{name} is not a public export"
        assert name not in ref["not_exported"].get(crate, {}), f"{crate}::{name}"
    cargo = open(os.path.join(ROOT, "backends", "hip", "Cargo.toml")).read()
    deps = set(re.findall(r"^([a-z0-9-]+)\s*=\s*\{\s*workspace\s*=\s*true", cargo, re.M))
    for crate in sorted({c for c, _ in used}):
        assert ref["packages"][crate] in deps, crate
