"""Vectorised numpy restatement of the block formulas and of the CpuScalar
accumulation order, written independently of oracle/oracle.c so the two can
check each other (a dropped term, a wrong shift or a transposed index in
either shows up as a mismatch).

Block formulas: backends/cpu/src/matmul.rs:162-280 and
quant/src/schemes/{q8,q4,q4_k,q5_k,q6_k}.rs (dequantize_*).
"""
import numpy as np

f32 = np.float32


def _kquant_sc_m(scales):
    """scales: [B,12] u8 -> (sc [B,8], m [B,8]) as u8 (matmul.rs:192-201)."""
    s = scales.astype(np.uint8)
    sc = np.empty((s.shape[0], 8), np.uint8)
    mn = np.empty((s.shape[0], 8), np.uint8)
    sc[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, mn


def dequant_q8_0(b):
    return (b["scale"][:, None] * b["values"].astype(f32)).astype(f32).ravel()


def dequant_q4_0(b):
    return (b["scale"][:, None] * (b["values"].astype(f32) - f32(8))).astype(f32).ravel()


def _k4_codes(values):
    """values [B,128] -> q [B,256]: element l uses byte 32*(l//64) + l%32,
    low nibble when l%64 < 32 (matmul.rs:202-209)."""
    v = values.reshape(-1, 4, 32)
    lo = v & 15
    hi = v >> 4
    return np.stack([lo, hi], axis=2).reshape(-1, 256)


def dequant_q4_k(b):
    sc, mn = _kquant_sc_m(b["scales"])
    q = _k4_codes(b["values"]).astype(f32)
    sub = np.arange(256) // 32
    d = b["scale"][:, None]
    dm = b["min_scale"][:, None]
    return ((d * sc[:, sub].astype(f32)) * q - dm * mn[:, sub].astype(f32)).astype(f32).ravel()


def dequant_q5_k(b):
    sc, mn = _kquant_sc_m(b["scales"])
    q = _k4_codes(b["values"]).astype(np.int32)
    l = np.arange(256)
    g, w = l // 64, l % 64
    bit = 2 * g + (w >= 32)
    hb = b["high_bits"][:, w % 32]
    q = q + 16 * ((hb >> bit) & 1)
    sub = l // 32
    d = b["scale"][:, None]
    dm = b["min_scale"][:, None]
    return ((d * sc[:, sub].astype(f32)) * q.astype(f32) - dm * mn[:, sub].astype(f32)).astype(f32).ravel()


def dequant_q6_k(b):
    l = np.arange(256)
    ip, r = l // 128, l % 128
    c, il = r // 32, r % 32
    byte = b["low_bits"][:, 64 * ip + np.where(c % 2 == 0, il, 32 + il)]
    low = np.where(c < 2, byte & 15, byte >> 4).astype(np.int32)
    high = ((b["high_bits"][:, 32 * ip + il] >> (2 * c)) & 3).astype(np.int32)
    q = low | (high << 4)
    sc = b["scales"][:, l // 16].astype(f32)
    return ((b["scale"][:, None] * sc) * (q - 32).astype(f32)).astype(f32).ravel()


DEQUANT = {1: dequant_q8_0, 2: dequant_q4_0, 3: dequant_q4_k, 4: dequant_q5_k, 5: dequant_q6_k}


def sequential_f32(x, w_rows):
    """CpuScalar order: for every output, acc = acc + x[k]*w[k] in f32, k
    ascending, no FMA. x [M,K], w_rows [N,K] -> y [M,N]."""
    x = x.astype(f32)
    w = w_rows.astype(f32)
    m, k = x.shape
    acc = np.zeros((m, w.shape[0]), f32)
    for i in range(k):
        acc = (acc + (x[:, i:i + 1] * w[None, :, i]).astype(f32)).astype(f32)
    return acc


# ------------------------------------------------------------------ Qwen3
# Float64 restatement of the Qwen3 forward pass (runtime/src/qwen3/mod.rs:
# 117-378, attention.rs:7-141, cpu backend.rs:172-298), vectorised and written
# without looking at oracle/qwen3.c: softmax attention over all cached keys,
# rotate-half RoPE, RMSNorm. It checks the C oracle within rounding, not bit
# for bit.

def _rms64(x, w, eps):
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return x / np.sqrt(ms + eps) * w


def _rope64(x, pos, theta):
    # x [T, heads, d]; pair (i, i + d/2) rotated by pos * theta^(-2i/d)
    d = x.shape[-1]
    half = d // 2
    inv = theta ** (-(2.0 * np.arange(half)) / d)
    ang = pos[:, None] * inv[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    a, b = x[..., :half], x[..., half:]
    return np.concatenate([a * c - b * s, a * s + b * c], axis=-1)


class Qwen3F64:
    """Same interface as the oracle model (cfg in oracle field names, layers
    as dicts of dequantized output-row weights), all arithmetic in float64."""

    def __init__(self, cfg, embedding, layers, final_norm, head):
        self.c = cfg
        self.emb = np.asarray(embedding, np.float64)
        self.layers = [{k: np.asarray(v, np.float64) for k, v in L.items()} for L in layers]
        self.fn = np.asarray(final_norm, np.float64)
        self.head = np.asarray(head, np.float64)
        self.keys = [np.zeros((0, cfg["kv_heads"], cfg["head_dim"])) for _ in layers]
        self.values = [np.zeros((0, cfg["kv_heads"], cfg["head_dim"])) for _ in layers]

    def forward(self, tokens):
        c = self.c
        hq, hk, d = c["heads"], c["kv_heads"], c["head_dim"]
        t = len(tokens)
        start = self.keys[0].shape[0]
        pos = np.arange(start, start + t, dtype=np.float64)
        h = self.emb[np.asarray(tokens)]
        for li, L in enumerate(self.layers):
            x = _rms64(h, L["input_norm"], c["eps"])
            q = (x @ L["q"].T).reshape(t, hq, d)
            k = (x @ L["k"].T).reshape(t, hk, d)
            v = (x @ L["v"].T).reshape(t, hk, d)
            q = _rope64(_rms64(q, L["q_norm"], c["eps"]), pos, c["theta"])
            k = _rope64(_rms64(k, L["k_norm"], c["eps"]), pos, c["theta"])
            self.keys[li] = np.concatenate([self.keys[li], k])
            self.values[li] = np.concatenate([self.values[li], v])
            K, V = self.keys[li], self.values[li]
            g = hq // hk
            att = np.empty((t, hq, d))
            for head in range(hq):
                kh, vh = K[:, head // g, :], V[:, head // g, :]
                sc = (q[:, head, :] @ kh.T) / np.sqrt(d)
                mask = np.arange(K.shape[0])[None, :] > (start + np.arange(t))[:, None]
                sc = np.where(mask, -np.inf, sc)
                sc = np.exp(sc - sc.max(axis=1, keepdims=True))
                att[:, head, :] = (sc / sc.sum(axis=1, keepdims=True)) @ vh
            h = h + att.reshape(t, hq * d) @ L["o"].T
            x = _rms64(h, L["post_norm"], c["eps"])
            gt, up = x @ L["gate"].T, x @ L["up"].T
            h = h + (gt / (1.0 + np.exp(-gt)) * up) @ L["down"].T
        return _rms64(h, self.fn, c["eps"]) @ self.head.T
