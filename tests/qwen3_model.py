"""Seeded random-init Qwen3 weights for the decoder tests.

The recipe is quantinfer_amd.synth.qwen3_weights (projections N(0, 0.02^2)
quantized to Q4_K, the LM head to Q6_K; embedding N(0, 0.02^2) and norm
weights N(1, 0.05^2), f32), built here with the oracle's generator and
quantizer. The same blocks feed the device decoder; the CPU oracle gets the
dequantized rows (the bit-identical f32 values the CpuScalar matmuls multiply
by) or the blocks themselves.
"""
from __future__ import annotations

import numpy as np

from oracle import pyoracle as po
from quantinfer_amd import synth

OUTPUT_ROWS = 1
ORACLE_NAMES = {"q_proj": "q", "k_proj": "k", "v_proj": "v", "o_proj": "o",
                "gate_proj": "gate", "up_proj": "up", "down_proj": "down"}


def small_config(**kw) -> dict:
    cfg = dict(vocab_size=1000, hidden_size=512, intermediate_size=768, num_hidden_layers=2,
               num_attention_heads=8, num_key_value_heads=2, head_dim=64,
               max_position_embeddings=256, rms_norm_eps=1e-6, rope_theta=1e6)
    cfg.update(kw)
    return cfg


def oracle_config(cfg: dict) -> dict:
    return dict(vocab=cfg["vocab_size"], hidden=cfg["hidden_size"],
                intermediate=cfg["intermediate_size"], layers=cfg["num_hidden_layers"],
                heads=cfg["num_attention_heads"], kv_heads=cfg["num_key_value_heads"],
                head_dim=cfg["head_dim"], max_positions=cfg["max_position_embeddings"],
                eps=cfg["rms_norm_eps"], theta=cfg["rope_theta"])


def oracle_fns():
    """The oracle's generator and quantizer (with f16 storage rounding), for
    quantinfer_amd.synth.qwen3_weights."""
    return (lambda seed, n, std: po.fill_normal(seed, n, std),
            lambda qtype, v: po.storage_precision(qtype, po.quantize(qtype, v)))


class Qwen3Weights:
    """Weights of one random model (the recipe of quantinfer_amd.synth, built
    with the oracle's generator and quantizer): `device_layers` for
    quantinfer_amd.Qwen3, `oracle_layers` (dequantized f32 rows) for
    oracle.pyoracle.Qwen3."""

    def __init__(self, cfg: dict, seed: int = 0x5EED0004, qtype: int = po.Q4_K,
                 head_qtype: int = po.Q6_K, dequantized: bool = True):
        self.cfg = cfg
        normal, quantize = oracle_fns()
        w = synth.qwen3_weights(cfg, seed, qtype, head_qtype, normal=normal, quantize=quantize)
        self.embedding = w["embedding"]
        self.device_layers = w["layers"]
        self.final_norm = w["final_norm"]
        self.head_qtype, _, self.head_blocks = w["head"]
        shapes = synth.projection_shapes(cfg)
        self.oracle_layers = []
        for dev in self.device_layers:
            orc = {"input_norm": dev["input_layernorm"], "q_norm": dev["q_norm"],
                   "k_norm": dev["k_norm"], "post_norm": dev["post_attention_layernorm"]}
            for name, short in ORACLE_NAMES.items():
                q, _, blocks = dev[name]
                orc[short] = (po.dequantize(q, blocks).reshape(shapes[name]) if dequantized
                              else (q, blocks))
            self.oracle_layers.append(orc)
        self.head = (po.dequantize(self.head_qtype, self.head_blocks).reshape(cfg["vocab_size"], -1)
                     if dequantized else (self.head_qtype, self.head_blocks))

    def device_model(self, ctx):
        import quantinfer_amd as qa
        m = qa.Qwen3(ctx, self.cfg)
        m.set_embedding(self.embedding)
        for i, layer in enumerate(self.device_layers):
            m.set_layer(i, layer)
        m.set_output(self.final_norm, (self.head_qtype, OUTPUT_ROWS, self.head_blocks))
        return m

    def oracle_model(self, capacity: int, threads: int = 4, blocks: bool = False):
        """The oracle decoder on the dequantized f32 rows, or (blocks=True) on
        the same quantized blocks the device holds."""
        if not blocks:
            return po.Qwen3(oracle_config(self.cfg), self.embedding, self.oracle_layers,
                            self.final_norm, self.head, capacity, threads)
        layers = []
        for dev, orc in zip(self.device_layers, self.oracle_layers):
            d = {f: orc[f] for f in po.NORM_FIELDS}
            for name, short in ORACLE_NAMES.items():
                qtype, _, blk = dev[name]
                d[short] = (qtype, blk)
            layers.append(d)
        return po.Qwen3(oracle_config(self.cfg), self.embedding, layers, self.final_norm,
                        (self.head_qtype, self.head_blocks), capacity, threads)


def prompt(cfg: dict, n: int, seed: int = 7) -> np.ndarray:
    return np.random.default_rng(seed).integers(0, cfg["vocab_size"], n).astype(np.int32)
