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


class _Weight(ctypes.Structure):
    """qo_weight: a projection as f32 output rows (qtype F32) or output-rows blocks."""
    _fields_ = [("qtype", ctypes.c_int), ("data", ctypes.c_void_p)]
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
    l.qo_rms_norm.argtypes = [fp, sz, sz, fp, ctypes.c_float, fp]
    l.qo_softmax.argtypes = [fp, sz, sz, fp]
    l.qo_silu_mul.argtypes = [fp, fp, sz, fp]
    l.qo_rope_tables.argtypes = [ctypes.c_float, sz, sz, sz, fp, fp]
    l.qo_apply_rope.argtypes = [fp, sz, sz, sz, fp, fp, sz, fp]
    l.qo_embedding.argtypes = [fp, sz, sz, vp, sz, fp]
    l.qo_gqa_attention.argtypes = [fp, sz, sz, sz, sz, fp, fp, sz, sz, fp]
    l.qo_argmax.argtypes = [fp, sz, vp]
    l.qo_linear_rows.argtypes = [fp, sz, sz, fp, sz, fp, i32]
    l.qo_linear.argtypes = [fp, sz, sz, _Weight, sz, fp, i32]
    l.qo_qwen3_new.argtypes = [vp, fp, vp, fp, _Weight, sz, i32]
    l.qo_qwen3_new.restype = vp
    l.qo_qwen3_free.argtypes = [vp]
    l.qo_qwen3_free.restype = None
    l.qo_qwen3_length.argtypes = [vp]
    l.qo_qwen3_length.restype = sz
    l.qo_qwen3_reset.argtypes = [vp]
    l.qo_qwen3_reset.restype = None
    l.qo_qwen3_forward.argtypes = [vp, vp, sz, i32, fp]
    l.qo_qwen3_generate.argtypes = [vp, vp, sz, sz, ctypes.c_int32, vp, ctypes.POINTER(sz)]


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


# ------------------------------------------------------- Qwen3 decoder

def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def rms_norm(x, w, eps: float) -> np.ndarray:
    x = _f32(x)
    w = _f32(w)
    out = np.empty_like(x)
    dim = w.size
    _check(lib().qo_rms_norm(_ptr(x), x.size // dim, dim, _ptr(w), eps, _ptr(out)), "rms_norm")
    return out


def softmax(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    _check(lib().qo_softmax(_ptr(x), x.size // x.shape[-1], x.shape[-1], _ptr(out)), "softmax")
    return out


def silu_mul(g, u) -> np.ndarray:
    g, u = _f32(g), _f32(u)
    out = np.empty_like(g)
    _check(lib().qo_silu_mul(_ptr(g), _ptr(u), g.size, _ptr(out)), "silu_mul")
    return out


def rope_tables(theta: float, head_dim: int, start: int, length: int):
    c = np.empty((length, head_dim // 2), dtype=np.float32)
    s = np.empty_like(c)
    _check(lib().qo_rope_tables(theta, head_dim, start, length, _ptr(c), _ptr(s)), "rope_tables")
    return c, s


def apply_rope(x, cos, sin) -> np.ndarray:
    """x [tokens, heads, head_dim]; tables [1 or tokens, head_dim/2]."""
    x, cos, sin = _f32(x), _f32(cos), _f32(sin)
    t, h, d = x.shape
    rows = cos.size // (d // 2)
    out = np.empty_like(x)
    _check(lib().qo_apply_rope(_ptr(x), t, h, d, _ptr(cos), _ptr(sin), rows, _ptr(out)),
           "apply_rope")
    return out


def embedding(table, tokens) -> np.ndarray:
    table = _f32(table)
    tok = np.ascontiguousarray(tokens, dtype=np.int32)
    out = np.empty((tok.size, table.shape[1]), dtype=np.float32)
    _check(lib().qo_embedding(_ptr(table), table.shape[0], table.shape[1], _ptr(tok), tok.size,
                              _ptr(out)), "embedding")
    return out


def gqa_attention(q, keys, values, start: int) -> np.ndarray:
    """q [tq, heads, hd]; keys/values [tk, kv_heads, hd]."""
    q, keys, values = _f32(q), _f32(keys), _f32(values)
    tq, hq, hd = q.shape
    tk, hk, _ = keys.shape
    out = np.empty_like(q)
    _check(lib().qo_gqa_attention(_ptr(q), tq, hq, hk, hd, _ptr(keys), _ptr(values), tk, start,
                                  _ptr(out)), "gqa_attention")
    return out


def argmax(logits) -> int:
    x = _f32(logits)
    out = np.zeros(1, dtype=np.int32)
    _check(lib().qo_argmax(_ptr(x), x.size, _ptr(out)), "argmax")
    return int(out[0])


def linear_rows(x, w, threads: int = 1) -> np.ndarray:
    """y[m, n] = sum_k x[m, k] w[n, k] in the CpuScalar per-output order."""
    x, w = _f32(x), _f32(w)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), dtype=np.float32)
    _check(lib().qo_linear_rows(_ptr(x), m, k, _ptr(w), n, _ptr(y), threads), "linear_rows")
    return y


class Qwen3Config(ctypes.Structure):
    """The Qwen3Config fields the forward pass reads (quantinfer-model qwen3.rs:11-37)."""
    _fields_ = [("vocab", ctypes.c_uint32), ("hidden", ctypes.c_uint32),
                ("intermediate", ctypes.c_uint32), ("layers", ctypes.c_uint32),
                ("heads", ctypes.c_uint32), ("kv_heads", ctypes.c_uint32),
                ("head_dim", ctypes.c_uint32), ("max_positions", ctypes.c_uint32),
                ("eps", ctypes.c_float), ("theta", ctypes.c_float)]


NORM_FIELDS = ("input_norm", "q_norm", "k_norm", "post_norm")
PROJ_FIELDS = ("q", "k", "v", "o", "gate", "up", "down")
LAYER_FIELDS = NORM_FIELDS + PROJ_FIELDS


class _Layer(ctypes.Structure):
    _fields_ = [(f, ctypes.c_void_p) for f in NORM_FIELDS] + [(f, _Weight) for f in PROJ_FIELDS]


def _weight(w, keep: list) -> "_Weight":
    """A projection as f32 output rows [n, k], or a (qtype, blocks) pair of
    output-rows logical blocks."""
    if isinstance(w, tuple):
        qtype, blocks = w
        b = np.ascontiguousarray(blocks)
        if b.dtype != BLOCK_DTYPES[qtype]:
            raise ValueError("blocks do not match the block type")
        keep.append(b)
        return _Weight(qtype, b.ctypes.data)
    a = _f32(w)
    keep.append(a)
    return _Weight(F32, a.ctypes.data)


def linear(x, w, n: int, threads: int = 1) -> np.ndarray:
    """qo_linear: y[m, n] = x . w with w f32 output rows [n, k] or (qtype, blocks)."""
    x = _f32(x)
    m, k = x.shape
    keep = []
    y = np.empty((m, n), dtype=np.float32)
    _check(lib().qo_linear(_ptr(x), m, k, _weight(w, keep), n, _ptr(y), threads), "linear")
    return y


class Qwen3:
    """The oracle decoder. `layers` is a list of dicts keyed by LAYER_FIELDS:
    f32 norm vectors, and projections as dequantized f32 output rows [n, k] or
    as (qtype, blocks) pairs of output-rows logical blocks; `head` likewise
    ([vocab, hidden] output rows). Arrays are kept alive by this object."""

    def __init__(self, cfg: dict, embedding, layers, final_norm, head, capacity: int,
                 threads: int = 1):
        self.cfg = Qwen3Config(**cfg)
        self._keep = [_f32(embedding), _f32(final_norm)]
        head_w = _weight(head, self._keep)
        lay = (_Layer * len(layers))()
        for i, d in enumerate(layers):
            for f in NORM_FIELDS:
                a = _f32(d[f])
                self._keep.append(a)
                setattr(lay[i], f, a.ctypes.data)
            for f in PROJ_FIELDS:
                setattr(lay[i], f, _weight(d[f], self._keep))
        self._layers = lay
        self.vocab = cfg["vocab"]
        h = lib().qo_qwen3_new(ctypes.byref(self.cfg), _ptr(self._keep[0]), lay,
                               _ptr(self._keep[1]), head_w, capacity, threads)
        if not h:
            raise OracleError("qo_qwen3_new rejected its configuration")
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            lib().qo_qwen3_free(h)
            self._h = None

    @property
    def length(self) -> int:
        return int(lib().qo_qwen3_length(self._h))

    def reset(self) -> None:
        lib().qo_qwen3_reset(self._h)

    def forward(self, tokens, last_only: bool = False) -> np.ndarray:
        tok = np.ascontiguousarray(tokens, dtype=np.int32)
        rows = 1 if last_only else tok.size
        out = np.empty((rows, self.vocab), dtype=np.float32)
        _check(lib().qo_qwen3_forward(self._h, _ptr(tok), tok.size, int(last_only), _ptr(out)),
               "qwen3_forward")
        return out

    def generate(self, prompt, max_new: int, eos: int = -1) -> list:
        tok = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(max(max_new, 1), dtype=np.int32)
        count = ctypes.c_size_t(0)
        _check(lib().qo_qwen3_generate(self._h, _ptr(tok), tok.size, max_new, eos, _ptr(out),
                                       ctypes.byref(count)), "qwen3_generate")
        return [int(t) for t in out[:count.value]]
