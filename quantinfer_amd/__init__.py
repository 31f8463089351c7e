"""quantinfer_amd: MI355X (gfx950) quantized-linear backend for QuantInfer.

The product is the C-ABI library libqi_hip.so (include/qi_hip.h) built from
quantinfer_amd/csrc by quantinfer_amd/build.py. This module is ctypes
plumbing over that ABI for Python callers (tests, bench.py); it contains no
compute of its own and raises if the native library is missing.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqi_hip.so")

OK, INVALID_INPUT, UNSUPPORTED, RUNTIME_ERROR = 0, 1, 2, 3
F32, Q8_0, Q4_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 3, 4, 5
QTYPES = {"f32": F32, "q8_0": Q8_0, "q4_0": Q4_0, "q4_k": Q4_K, "q5_k": Q5_K, "q6_k": Q6_K}
ROW_MAJOR, OUTPUT_ROWS = 0, 1
MODE_AUTO, MODE_F32, MODE_EXACT, MODE_MFMA = 0, 1, 2, 3

# qi_hip_*_block (include/qi_hip.h), field-for-field the reference core structs.
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
BLOCK_ELEMS = {F32: 1, Q8_0: 32, Q4_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256}
WIRE_BYTES = {Q8_0: 34, Q4_0: 18, Q4_K: 144, Q5_K: 176, Q6_K: 210}


class QiError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[status {status}] {message}")
        self.status = status


class WeightsInfo(ctypes.Structure):
    _fields_ = [("qtype", ctypes.c_int32), ("layout", ctypes.c_int32), ("k", ctypes.c_uint64),
                ("n", ctypes.c_uint64), ("device_bytes", ctypes.c_uint64),
                ("f16_scales", ctypes.c_int32)]


class Qwen3Config(ctypes.Structure):
    """qi_hip_qwen3_config (the Qwen3Config fields the forward pass reads)."""
    _fields_ = [("vocab_size", ctypes.c_uint32), ("hidden_size", ctypes.c_uint32),
                ("intermediate_size", ctypes.c_uint32), ("num_hidden_layers", ctypes.c_uint32),
                ("num_attention_heads", ctypes.c_uint32), ("num_key_value_heads", ctypes.c_uint32),
                ("head_dim", ctypes.c_uint32), ("max_position_embeddings", ctypes.c_uint32),
                ("rms_norm_eps", ctypes.c_float), ("rope_theta", ctypes.c_float)]


class LinearWeight(ctypes.Structure):
    """qi_hip_linear_weight: logical blocks of one projection."""
    _fields_ = [("qtype", ctypes.c_int32), ("layout", ctypes.c_int32), ("data", ctypes.c_void_p),
                ("count", ctypes.c_uint64)]


PROJECTIONS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")
LAYER_NORMS = ("input_layernorm", "q_norm", "k_norm", "post_attention_layernorm")


class Qwen3Layer(ctypes.Structure):
    """qi_hip_qwen3_layer (Qwen3LayerWeights)."""
    _fields_ = ([(n, ctypes.c_void_p) for n in LAYER_NORMS] +
                [(p, LinearWeight) for p in PROJECTIONS])


class Qwen3Timing(ctypes.Structure):
    _fields_ = [("prefill_ms", ctypes.c_double), ("decode_ms", ctypes.c_double),
                ("prompt_tokens", ctypes.c_uint64), ("decode_steps", ctypes.c_uint64)]


_lib = None


def lib() -> ctypes.CDLL:
    """Load libqi_hip.so. Raises if it has not been built: there is no fallback."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with quantinfer_amd/build.py "
                               "(or __graft_entry__.build()); there is no CPU fallback")
        l = ctypes.CDLL(LIB_PATH)
        vp, u64, i32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int32
        l.qi_hip_abi_version.restype = i32
        l.qi_hip_last_error.restype = ctypes.c_char_p
        l.qi_hip_open.argtypes = [i32, ctypes.POINTER(vp)]
        l.qi_hip_close.argtypes = [vp]
        l.qi_hip_close.restype = None
        l.qi_hip_device_name.argtypes = [vp, ctypes.c_char_p, ctypes.c_size_t]
        l.qi_hip_weights_create.argtypes = [vp, i32, i32, u64, u64, vp, u64, ctypes.POINTER(vp)]
        l.qi_hip_weights_free.argtypes = [vp]
        l.qi_hip_weights_free.restype = None
        l.qi_hip_weights_info_get.argtypes = [vp, ctypes.POINTER(WeightsInfo)]
        l.qi_hip_linear.argtypes = [vp, vp, vp, u64, vp, i32]
        l.qi_hip_linear_device.argtypes = [vp, vp, vp, u64, vp, i32, vp]
        l.qi_hip_linear_device_noalloc.argtypes = [vp, vp, vp, u64, vp, i32, vp]
        l.qi_hip_dequantize.argtypes = [vp, vp, vp]
        l.qi_hip_dequantize_device.argtypes = [vp, vp, vp, vp]
        l.qi_hip_pack_weights.argtypes = [i32, i32, u64, u64, vp, u64, vp,
                                          ctypes.POINTER(u64), ctypes.POINTER(i32)]
        l.qi_hip_weights_create_gguf.argtypes = [vp, i32, i32, u64, u64, vp, u64, i32, ctypes.POINTER(vp)]
        l.qi_hip_pack_gguf.argtypes = [i32, i32, u64, u64, vp, u64, i32, vp, ctypes.POINTER(u64),
                                       ctypes.POINTER(i32)]
        l.qi_hip_quantize.argtypes = [i32, vp, u64, i32, vp, u64, i32]
        l.qi_hip_synth_normal.argtypes = [u64, u64, ctypes.c_double, ctypes.c_double, ctypes.c_double,
                                          vp, i32]
        u32 = ctypes.c_uint32
        l.qi_hip_qwen3_create.argtypes = [vp, ctypes.POINTER(Qwen3Config), ctypes.POINTER(vp)]
        l.qi_hip_qwen3_set_embedding.argtypes = [vp, vp]
        l.qi_hip_qwen3_set_layer.argtypes = [vp, u32, ctypes.POINTER(Qwen3Layer)]
        l.qi_hip_qwen3_set_output.argtypes = [vp, vp, ctypes.POINTER(LinearWeight)]
        l.qi_hip_qwen3_set_mode.argtypes = [vp, i32]
        l.qi_hip_qwen3_free.argtypes = [vp]
        l.qi_hip_qwen3_free.restype = None
        l.qi_hip_kv_cache_create.argtypes = [vp, u32, u32, u32, u32, ctypes.POINTER(vp)]
        l.qi_hip_kv_cache_length.argtypes = [vp, ctypes.POINTER(u64)]
        l.qi_hip_kv_cache_reset.argtypes = [vp]
        l.qi_hip_kv_cache_free.argtypes = [vp]
        l.qi_hip_kv_cache_free.restype = None
        l.qi_hip_qwen3_forward.argtypes = [vp, vp, vp, u64, vp, vp]
        l.qi_hip_qwen3_generate.argtypes = [vp, vp, vp, u64, u64, i32, vp, ctypes.POINTER(u64)]
        l.qi_hip_qwen3_last_timing.argtypes = [vp, ctypes.POINTER(Qwen3Timing)]
        for name in ("qi_hip_open", "qi_hip_device_name", "qi_hip_weights_create",
                     "qi_hip_weights_info_get", "qi_hip_linear", "qi_hip_linear_device",
                     "qi_hip_linear_device_noalloc",
                     "qi_hip_dequantize", "qi_hip_dequantize_device", "qi_hip_pack_weights",
                     "qi_hip_weights_create_gguf", "qi_hip_pack_gguf", "qi_hip_quantize", "qi_hip_synth_normal",
                     "qi_hip_qwen3_create", "qi_hip_qwen3_set_embedding", "qi_hip_qwen3_set_layer",
                     "qi_hip_qwen3_set_output", "qi_hip_qwen3_set_mode", "qi_hip_kv_cache_create",
                     "qi_hip_kv_cache_length", "qi_hip_kv_cache_reset", "qi_hip_qwen3_forward",
                     "qi_hip_qwen3_generate", "qi_hip_qwen3_last_timing"):
            getattr(l, name).restype = i32
        if l.qi_hip_abi_version() != 1:
            raise RuntimeError("libqi_hip.so ABI version mismatch")
        _lib = l
    return _lib


def _check(status: int) -> None:
    if status != OK:
        raise QiError(status, lib().qi_hip_last_error().decode())


def _ptr(a: np.ndarray) -> int:
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("array must be C-contiguous")
    return a.ctypes.data


def pack_weights(qtype: int, layout: int, k: int, n: int, blocks: np.ndarray):
    """Host-only device image (bytes, f16_scales) exactly as weights_create builds it."""
    b = np.ascontiguousarray(blocks)
    size = ctypes.c_uint64(0)
    f16 = ctypes.c_int32(0)
    _check(lib().qi_hip_pack_weights(qtype, layout, k, n, _ptr(b), b.size, None,
                                     ctypes.byref(size), ctypes.byref(f16)))
    out = np.zeros(size.value, dtype=np.uint8)
    _check(lib().qi_hip_pack_weights(qtype, layout, k, n, _ptr(b), b.size, _ptr(out),
                                     ctypes.byref(size), ctypes.byref(f16)))
    return out, bool(f16.value)


def pack_gguf(qtype: int, layout: int, k: int, n: int, wire, legacy: bool = False):
    """Host-only device image (bytes, f16_scales) of a GGUF tensor's wire blocks,
    exactly as weights_gguf builds it."""
    w = np.ascontiguousarray(np.frombuffer(bytes(wire), dtype=np.uint8) if not isinstance(wire, np.ndarray)
                             else wire.view(np.uint8).reshape(-1))
    size = ctypes.c_uint64(0)
    f16 = ctypes.c_int32(0)
    _check(lib().qi_hip_pack_gguf(qtype, layout, k, n, _ptr(w), w.size, int(legacy), None,
                                  ctypes.byref(size), ctypes.byref(f16)))
    out = np.zeros(size.value, dtype=np.uint8)
    _check(lib().qi_hip_pack_gguf(qtype, layout, k, n, _ptr(w), w.size, int(legacy), _ptr(out),
                                  ctypes.byref(size), ctypes.byref(f16)))
    return out, bool(f16.value)


def quantize(qtype: int, values, storage_f16: bool = False, threads: int = 0) -> np.ndarray:
    """Host-only: the reference quantizer's logical blocks of `values`
    (qi_hip_quantize), optionally with f16 storage rounding of the scales."""
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    out = np.zeros(v.size // BLOCK_ELEMS[qtype], dtype=BLOCK_DTYPES[qtype])
    _check(lib().qi_hip_quantize(qtype, _ptr(v), v.size, int(storage_f16), _ptr(out), out.size,
                                 threads))
    return out


def synth_normal(seed: int, n: int, std: float = 1.0, outlier_rate: float = 0.0,
                 outlier_std: float = 0.0, threads: int = 0) -> np.ndarray:
    """Host-only seeded synthetic values (qi_hip_synth_normal): N(0, std^2), a
    fraction `outlier_rate` drawn with outlier_std instead."""
    out = np.empty(n, dtype=np.float32)
    _check(lib().qi_hip_synth_normal(seed, n, std, outlier_rate, outlier_std, _ptr(out), threads))
    return out


class Context:
    """An open gfx950 device (qi_hip_open)."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        _check(lib().qi_hip_open(device, ctypes.byref(h)))
        self.handle = h

    def close(self) -> None:
        if self.handle:
            lib().qi_hip_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def device_name(self) -> str:
        buf = ctypes.create_string_buffer(256)
        _check(lib().qi_hip_device_name(self.handle, buf, 256))
        return buf.value.decode()

    def weights(self, qtype: int, layout: int, k: int, n: int, blocks: np.ndarray) -> "Weights":
        return Weights(self, qtype, layout, k, n, blocks)

    def weights_gguf(self, qtype: int, layout: int, k: int, n: int, wire,
                     legacy: bool = False) -> "Weights":
        """A resident weight from a GGUF tensor's wire block bytes
        (qi_hip_weights_create_gguf)."""
        w = np.ascontiguousarray(np.frombuffer(bytes(wire), dtype=np.uint8) if not isinstance(wire, np.ndarray)
                                 else wire.view(np.uint8).reshape(-1))
        h = ctypes.c_void_p()
        _check(lib().qi_hip_weights_create_gguf(self.handle, qtype, layout, k, n, _ptr(w), w.size,
                                                int(legacy), ctypes.byref(h)))
        return Weights._adopt(self, h, qtype, layout, k, n)


class Weights:
    """A resident weight of logical shape [K, N] (qi_hip_weights_create)."""

    @classmethod
    def _adopt(cls, ctx: "Context", handle, qtype: int, layout: int, k: int, n: int) -> "Weights":
        w = cls.__new__(cls)
        w.ctx, w.handle, w.qtype, w.layout, w.k, w.n = ctx, handle, qtype, layout, k, n
        return w

    def __init__(self, ctx: Context, qtype: int, layout: int, k: int, n: int, blocks: np.ndarray):
        b = np.ascontiguousarray(blocks)
        h = ctypes.c_void_p()
        _check(lib().qi_hip_weights_create(ctx.handle, qtype, layout, k, n, _ptr(b), b.size,
                                           ctypes.byref(h)))
        self.ctx, self.handle, self.qtype, self.layout, self.k, self.n = ctx, h, qtype, layout, k, n

    def free(self) -> None:
        if self.handle:
            lib().qi_hip_weights_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def info(self) -> WeightsInfo:
        out = WeightsInfo()
        _check(lib().qi_hip_weights_info_get(self.handle, ctypes.byref(out)))
        return out

    def linear(self, x: np.ndarray, mode: int = MODE_AUTO) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim != 2 or x.shape[1] != self.k:
            raise ValueError(f"x must be [M, {self.k}]")
        y = np.empty((x.shape[0], self.n), dtype=np.float32)
        _check(lib().qi_hip_linear(self.ctx.handle, self.handle, _ptr(x), x.shape[0], _ptr(y), mode))
        return y

    def linear_device(self, x_ptr: int, m: int, y_ptr: int, mode: int = MODE_AUTO,
                      stream: int = 0) -> None:
        _check(lib().qi_hip_linear_device(self.ctx.handle, self.handle, x_ptr, m, y_ptr, mode,
                                          stream or None))

    def dequantize(self) -> np.ndarray:
        out = np.empty(self.k * self.n, dtype=np.float32)
        _check(lib().qi_hip_dequantize(self.ctx.handle, self.handle, _ptr(out)))
        return out

    def dequantize_device(self, out_ptr: int, stream: int = 0) -> None:
        _check(lib().qi_hip_dequantize_device(self.ctx.handle, self.handle, out_ptr,
                                              stream or None))


def _linear_weight(qtype: int, layout: int, data: np.ndarray, keep: list) -> LinearWeight:
    d = np.ascontiguousarray(data)
    keep.append(d)
    return LinearWeight(qtype, layout, d.ctypes.data, d.size)


class KvCache:
    """A device KV cache (qi_hip_kv_cache_create; KvCache::new)."""

    def __init__(self, ctx: Context, layers: int, max_sequence_length: int, kv_heads: int,
                 head_dim: int):
        h = ctypes.c_void_p()
        _check(lib().qi_hip_kv_cache_create(ctx.handle, layers, max_sequence_length, kv_heads,
                                            head_dim, ctypes.byref(h)))
        self.ctx, self.handle = ctx, h

    @property
    def length(self) -> int:
        out = ctypes.c_uint64(0)
        _check(lib().qi_hip_kv_cache_length(self.handle, ctypes.byref(out)))
        return out.value

    def reset(self) -> None:
        _check(lib().qi_hip_kv_cache_reset(self.handle))

    def free(self) -> None:
        if self.handle:
            lib().qi_hip_kv_cache_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Qwen3:
    """A GPU-resident Qwen3 decoder (qi_hip_qwen3_*). `cfg` holds the
    qi_hip_qwen3_config fields; weights are given per layer as dicts with the
    four norms (f32 arrays) and the seven projections as (qtype, layout,
    blocks) triples of logical blocks."""

    def __init__(self, ctx: Context, cfg: dict):
        self.cfg = dict(cfg)
        c = Qwen3Config(**cfg)
        h = ctypes.c_void_p()
        _check(lib().qi_hip_qwen3_create(ctx.handle, ctypes.byref(c), ctypes.byref(h)))
        self.ctx, self.handle = ctx, h

    def set_embedding(self, table: np.ndarray) -> None:
        t = np.ascontiguousarray(table, dtype=np.float32)
        _check(lib().qi_hip_qwen3_set_embedding(self.handle, _ptr(t)))

    def set_layer(self, index: int, layer: dict) -> None:
        keep = []
        s = Qwen3Layer()
        for n in LAYER_NORMS:
            a = np.ascontiguousarray(layer[n], dtype=np.float32)
            keep.append(a)
            setattr(s, n, a.ctypes.data)
        for p in PROJECTIONS:
            qtype, layout, blocks = layer[p]
            setattr(s, p, _linear_weight(qtype, layout, blocks, keep))
        _check(lib().qi_hip_qwen3_set_layer(self.handle, index, ctypes.byref(s)))

    def set_output(self, final_norm: np.ndarray, head) -> None:
        keep = []
        fn = np.ascontiguousarray(final_norm, dtype=np.float32)
        hw = _linear_weight(*head, keep)
        _check(lib().qi_hip_qwen3_set_output(self.handle, _ptr(fn), ctypes.byref(hw)))

    def set_mode(self, mode: int) -> None:
        _check(lib().qi_hip_qwen3_set_mode(self.handle, mode))

    def kv_cache(self, max_sequence_length: int) -> KvCache:
        return KvCache(self.ctx, self.cfg["num_hidden_layers"], max_sequence_length,
                       self.cfg["num_key_value_heads"], self.cfg["head_dim"])

    def forward(self, cache: KvCache, tokens, logits: bool = True):
        """Returns (last-row logits or None, argmax token)."""
        tok = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty(self.cfg["vocab_size"], dtype=np.float32) if logits else None
        nxt = ctypes.c_int32(0)
        _check(lib().qi_hip_qwen3_forward(self.handle, cache.handle, _ptr(tok), tok.size,
                                          _ptr(out) if logits else None, ctypes.byref(nxt)))
        return out, nxt.value

    def generate(self, cache: KvCache, prompt, max_new_tokens: int, eos: int = -1) -> list:
        tok = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(max(max_new_tokens, 1), dtype=np.int32)
        count = ctypes.c_uint64(0)
        _check(lib().qi_hip_qwen3_generate(self.handle, cache.handle, _ptr(tok), tok.size,
                                           max_new_tokens, eos, _ptr(out), ctypes.byref(count)))
        return [int(t) for t in out[:count.value]]

    def last_timing(self) -> Qwen3Timing:
        t = Qwen3Timing()
        _check(lib().qi_hip_qwen3_last_timing(self.handle, ctypes.byref(t)))
        return t

    def free(self) -> None:
        if self.handle:
            lib().qi_hip_qwen3_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
