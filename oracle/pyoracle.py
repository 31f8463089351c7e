"""ctypes wrapper of the C oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package. See oracle.h for
what the oracle restates and oracle.c for how each part is pinned.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, Q8_0, Q4_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 3, 4, 5
QTYPES = {"q8_0": Q8_0, "q4_0": Q4_0, "q4_k": Q4_K, "q5_k": Q5_K, "q6_k": Q6_K}

# Logical blocks, field-for-field the reference core structs
# (core quantized/q8.rs:7-11, q4.rs:7-13, q4.rs:72-78, k.rs:7-14, k.rs:55-61).
BLOCK_DTYPES = {
    Q8_0: np.dtype([("scale", "<f4"), ("values", "i1", (32,))]),
    Q4_0: np.dtype([("scale", "<f4"), ("values", "u1", (32,))]),
    Q4_K: np.dtype([("scale", "<f4"), ("min_scale", "<f4"), ("scales", "u1", (12,)),
                    ("values", "u1", (128,))]),
    Q5_K: np.dtype([("scale", "<f4"), ("min_scale", "<f4"), ("scales", "u1", (12,)),
                    ("high_bits", "u1", (32,)), ("values", "u1", (128,))]),
    Q6_K: np.dtype([("scale", "<f4"), ("scales", "i1", (16,)), ("low_bits", "u1", (128,)),
                    ("high_bits", "u1", (64,))]),
}
BLOCK_ELEMS = {Q8_0: 32, Q4_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256}
WIRE_BYTES = {Q8_0: 34, Q4_0: 18, Q4_K: 144, Q5_K: 176, Q6_K: 210}


class OracleError(RuntimeError):
    pass


def build() -> str:
    """Compile liboracle.so with its Makefile (gcc, exact IEEE binary32)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(l: ctypes.CDLL) -> None:
    vp, sz, i32, fp = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p
    l.qo_f32_to_f16.argtypes = [ctypes.c_float]
    l.qo_f32_to_f16.restype = ctypes.c_uint16
    l.qo_f16_to_f32.argtypes = [ctypes.c_uint16]
    l.qo_f16_to_f32.restype = ctypes.c_float
    l.qo_f32_to_f16_array.argtypes = [fp, sz, vp]
    l.qo_f16_to_f32_array.argtypes = [vp, sz, fp]
    l.qo_stored_f16_scale.argtypes = [ctypes.c_float, ctypes.POINTER(ctypes.c_float)]
    for q in ("q8_0", "q4_0", "q4_k", "q5_k", "q6_k"):
        f = getattr(l, f"qo_quantize_{q}")
        f.argtypes = [fp, sz, vp]
        f.restype = i32
    l.qo_storage_precision.argtypes = [i32, vp, sz]
    l.qo_validate_blocks.argtypes = [i32, vp, sz, sz]
    l.qo_dequantize.argtypes = [i32, vp, sz, fp]
    l.qo_value.argtypes = [i32, vp, sz]
    l.qo_value.restype = ctypes.c_float
    for f in (l.qo_matmul_output_rows, l.qo_matmul_row_major):
        f.argtypes = [i32, fp, sz, sz, vp, sz, sz, fp]
        f.restype = i32
    l.qo_matmul_output_rows_threaded.argtypes = [i32, fp, sz, sz, vp, sz, sz, fp, i32]
    l.qo_matmul_f32.argtypes = [fp, sz, sz, fp, sz, fp]
    l.qo_simd_isa_available.argtypes = [i32]
    l.qo_matmul_output_rows_simd.argtypes = [i32, i32, fp, sz, sz, vp, sz, sz, fp]
    l.qo_wire_pack.argtypes = [i32, vp, sz, vp]
    l.qo_wire_unpack.argtypes = [i32, vp, sz, i32, vp]
    l.qo_fill_normal.argtypes = [ctypes.c_uint64, sz, ctypes.c_double, ctypes.c_double,
                                 ctypes.c_double, fp]
    l.qo_fill_normal.restype = None


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _check(status: int, what: str) -> None:
    if status != 0:
        raise OracleError(f"{what} rejected its input (status {status})")


# ----------------------------------------------------------------- f16

def f32_to_f16(values) -> np.ndarray:
    v = np.ascontiguousarray(values, dtype=np.float32).ravel()
    out = np.empty(v.size, dtype=np.uint16)
    lib().qo_f32_to_f16_array(_ptr(v), v.size, _ptr(out))
    return out


def f16_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16).ravel()
    out = np.empty(b.size, dtype=np.float32)
    lib().qo_f16_to_f32_array(_ptr(b), b.size, _ptr(out))
    return out


def stored_f16_scale(value: float) -> float:
    out = ctypes.c_float()
    _check(lib().qo_stored_f16_scale(ctypes.c_float(value), ctypes.byref(out)), "stored_f16_scale")
    return out.value


# ----------------------------------------------------------- quantizers

def quantize(qtype: int, values) -> np.ndarray:
    v = np.ascontiguousarray(values, dtype=np.float32).ravel()
    bs = BLOCK_ELEMS[qtype]
    out = np.zeros(v.size // bs if v.size % bs == 0 else 0, dtype=BLOCK_DTYPES[qtype])
    name = {Q8_0: "q8_0", Q4_0: "q4_0", Q4_K: "q4_k", Q5_K: "q5_k", Q6_K: "q6_k"}[qtype]
    _check(getattr(lib(), f"qo_quantize_{name}")(_ptr(v), v.size, _ptr(out)), f"quantize_{name}")
    return out


def storage_precision(qtype: int, blocks: np.ndarray) -> np.ndarray:
    out = np.ascontiguousarray(blocks.copy())
    _check(lib().qo_storage_precision(qtype, _ptr(out), out.size), "with_storage_precision")
    return out


def validate_blocks(qtype: int, blocks: np.ndarray, elements: int) -> bool:
    b = np.ascontiguousarray(blocks)
    return lib().qo_validate_blocks(qtype, _ptr(b), b.size, elements) == 0


def dequantize(qtype: int, blocks: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(blocks)
    out = np.empty(b.size * BLOCK_ELEMS[qtype], dtype=np.float32)
    _check(lib().qo_dequantize(qtype, _ptr(b), b.size, _ptr(out)), "dequantize")
    return out


def value(qtype: int, blocks: np.ndarray, index: int) -> float:
    b = np.ascontiguousarray(blocks)
    return lib().qo_value(qtype, _ptr(b), index)


# -------------------------------------------------------------- matmuls

def matmul_output_rows(qtype: int, x: np.ndarray, blocks: np.ndarray, n: int,
                       threads: int = 1) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    b = np.ascontiguousarray(blocks)
    y = np.empty((m, n), dtype=np.float32)
    if threads == 1:
        st = lib().qo_matmul_output_rows(qtype, _ptr(x), m, k, _ptr(b), b.size, n, _ptr(y))
    else:
        st = lib().qo_matmul_output_rows_threaded(qtype, _ptr(x), m, k, _ptr(b), b.size, n,
                                                  _ptr(y), threads)
    _check(st, "matmul_output_rows")
    return y


def matmul_row_major(qtype: int, x: np.ndarray, blocks: np.ndarray, n: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    b = np.ascontiguousarray(blocks)
    y = np.empty((m, n), dtype=np.float32)
    _check(lib().qo_matmul_row_major(qtype, _ptr(x), m, k, _ptr(b), b.size, n, _ptr(y)),
           "matmul_row_major")
    return y


def matmul_f32(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    m, k = x.shape
    k2, n = w.shape
    assert k == k2
    y = np.empty((m, n), dtype=np.float32)
    _check(lib().qo_matmul_f32(_ptr(x), m, k, _ptr(w), n, _ptr(y)), "matmul_f32")
    return y


def simd_available(isa: int) -> bool:
    return bool(lib().qo_simd_isa_available(isa))


def matmul_output_rows_simd(qtype: int, isa: int, x: np.ndarray, blocks: np.ndarray,
                            n: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    b = np.ascontiguousarray(blocks)
    y = np.empty((m, n), dtype=np.float32)
    _check(lib().qo_matmul_output_rows_simd(qtype, isa, _ptr(x), m, k, _ptr(b), b.size, n,
                                            _ptr(y)), "matmul_output_rows_simd")
    return y


# ---------------------------------------------------------- wire codecs

def wire_pack(qtype: int, blocks: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(blocks)
    out = np.zeros(b.size * WIRE_BYTES[qtype], dtype=np.uint8)
    _check(lib().qo_wire_pack(qtype, _ptr(b), b.size, _ptr(out)), "wire_pack")
    return out


def wire_unpack(qtype: int, data, legacy: bool = False) -> np.ndarray:
    d = np.ascontiguousarray(np.frombuffer(bytes(data), dtype=np.uint8)
                             if not isinstance(data, np.ndarray) else data, dtype=np.uint8)
    count = d.size // WIRE_BYTES[qtype]
    out = np.zeros(count, dtype=BLOCK_DTYPES[qtype])
    _check(lib().qo_wire_unpack(qtype, _ptr(d), count, int(legacy), _ptr(out)), "wire_unpack")
    return out


# --------------------------------------------------------------- inputs

def fill_normal(seed: int, n: int, std: float = 1.0, outlier_rate: float = 0.0,
                outlier_std: float = 0.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().qo_fill_normal(seed, n, std, outlier_rate, outlier_std, _ptr(out))
    return out


def make_weights(qtype: int, k: int, n: int, seed: int, storage_f16: bool = True,
                 outliers: bool = False) -> np.ndarray:
    """Synthetic output-rows weight of logical shape [K, N]: f32 [N, K] drawn
    from N(0, 0.02^2) (optionally 0.5% N(0, 0.2^2) outliers), quantized with the
    restated reference quantizer, then (for the "f16 scale" configs) rounded
    with with_storage_precision."""
    w = fill_normal(seed, n * k, 0.02, 0.005 if outliers else 0.0, 0.2)
    blocks = quantize(qtype, w)
    if storage_f16:
        blocks = storage_precision(qtype, blocks)
    return blocks
