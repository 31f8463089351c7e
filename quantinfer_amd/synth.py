"""Seeded random-init Qwen3 weights (the recipe of the end-to-end config).

Every projection is f32 output rows [N, K] drawn from N(0, 0.02^2), quantized
by the reference's quantizer (Q4_K by default, the LM head Q6_K) with f16
storage rounding of the scales; the embedding is f32 N(0, 0.02^2) and the norm
weights f32 N(1, 0.05^2). Seeds: the embedding uses `seed`, then the
projections `seed + 1, seed + 2, ...` in layer order q, k, v, o, gate, up,
down, then the head; the norm weights come from numpy's default_rng(seed).

`normal(seed, n, std)` and `quantize(qtype, values)` are parameters, so that
the same recipe can be built with this library's host functions
(qi_hip_synth_normal, qi_hip_quantize; bench.py) or with the test oracle's
(tests), which produce the same values bit for bit.
"""
from __future__ import annotations

import numpy as np

OUTPUT_ROWS = 1
PROJECTIONS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")

# the Qwen3-8B architecture
QWEN3_8B = dict(vocab_size=151936, hidden_size=4096, intermediate_size=12288, num_hidden_layers=36,
                num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                max_position_embeddings=40960, rms_norm_eps=1e-6, rope_theta=1e6)
DEFAULT_SEED = 0x5EED0004
PROMPT_SEED = 7


def projection_shapes(cfg: dict) -> dict:
    """(N, K) of each projection: output rows of a logical [K, N] weight."""
    H, I, hd = cfg["hidden_size"], cfg["intermediate_size"], cfg["head_dim"]
    QS, KS = cfg["num_attention_heads"] * hd, cfg["num_key_value_heads"] * hd
    return {"q_proj": (QS, H), "k_proj": (KS, H), "v_proj": (KS, H), "o_proj": (H, QS),
            "gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I)}


def _default_fns():
    import quantinfer_amd as qa
    return (lambda seed, n, std: qa.synth_normal(seed, n, std),
            lambda qtype, v: qa.quantize(qtype, v, storage_f16=True))


def qwen3_weights(cfg: dict, seed: int = DEFAULT_SEED, qtype: int = 3, head_qtype: int = 5,
                  normal=None, quantize=None, layers: int | None = None) -> dict:
    """Weights of one random model: {"embedding", "layers" (dicts of the four
    norm vectors and the seven projections as (qtype, OUTPUT_ROWS, blocks)),
    "final_norm", "head" (head_qtype, OUTPUT_ROWS, blocks)}. `layers` builds
    only the first layers of the recipe (the head keeps its seed)."""
    if normal is None or quantize is None:
        normal, quantize = _default_fns()
    H, hd = cfg["hidden_size"], cfg["head_dim"]
    shapes = projection_shapes(cfg)
    rng = np.random.default_rng(seed)
    s = seed
    embedding = normal(s, cfg["vocab_size"] * H, 0.02).reshape(cfg["vocab_size"], H)
    out_layers = []
    nl = cfg["num_hidden_layers"]
    for li in range(nl):
        norms = {n: (1.0 + 0.05 * rng.standard_normal(d)).astype(np.float32)
                 for n, d in (("input_layernorm", H), ("q_norm", hd), ("k_norm", hd),
                              ("post_attention_layernorm", H))}
        layer = dict(norms)
        for name in PROJECTIONS:
            s += 1
            if layers is not None and li >= layers:
                continue
            n, k = shapes[name]
            layer[name] = (qtype, OUTPUT_ROWS, quantize(qtype, normal(s, n * k, 0.02)))
        if layers is None or li < layers:
            out_layers.append(layer)
    final_norm = (1.0 + 0.05 * rng.standard_normal(H)).astype(np.float32)
    s += 1
    head = (head_qtype, OUTPUT_ROWS, quantize(head_qtype, normal(s, cfg["vocab_size"] * H, 0.02)))
    return {"embedding": embedding, "layers": out_layers, "final_norm": final_norm, "head": head}


def prompt(cfg: dict, n: int, seed: int = PROMPT_SEED) -> np.ndarray:
    """Uniform random token ids."""
    return np.random.default_rng(seed).integers(0, cfg["vocab_size"], n).astype(np.int32)


def device_model(ctx, cfg: dict, weights: dict):
    """A quantinfer_amd.Qwen3 holding `weights` (from qwen3_weights)."""
    import quantinfer_amd as qa
    m = qa.Qwen3(ctx, cfg)
    m.set_embedding(weights["embedding"])
    for i, layer in enumerate(weights["layers"]):
        m.set_layer(i, layer)
    m.set_output(weights["final_norm"], weights["head"])
    return m
