"""Seeded random-init Qwen3 weights for the decoder tests.

Each projection is drawn from N(0, 0.02^2) as f32 output rows [N, K], quantized
with the oracle's restatement of the reference quantizer (Q4_K by default; the
LM head Q6_K, as in the end-to-end config) and dequantized again, so the same
weights feed the device decoder (as logical blocks) and the CPU oracle (as
the bit-identical f32 values the CpuScalar matmuls multiply by). Norm weights
are N(1, 0.05^2) and the embedding N(0, 0.02^2), both f32.
"""
from __future__ import annotations

import numpy as np

from oracle import pyoracle as po

OUTPUT_ROWS = 1


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


def _proj(qtype: int, n: int, k: int, seed: int):
    w = po.fill_normal(seed, n * k, 0.02)
    blocks = po.storage_precision(qtype, po.quantize(qtype, w))
    deq = po.dequantize(qtype, blocks).reshape(n, k)
    return blocks, deq


class Qwen3Weights:
    """Weights of one random model: `device_layers` for quantinfer_amd.Qwen3,
    `oracle_layers` for oracle.pyoracle.Qwen3."""

    def __init__(self, cfg: dict, seed: int = 0x5EED0004, qtype: int = po.Q4_K,
                 head_qtype: int = po.Q6_K):
        self.cfg = cfg
        H, I = cfg["hidden_size"], cfg["intermediate_size"]
        hd = cfg["head_dim"]
        QS, KS = cfg["num_attention_heads"] * hd, cfg["num_key_value_heads"] * hd
        rng = np.random.default_rng(seed)
        s = seed
        self.embedding = po.fill_normal(s, cfg["vocab_size"] * H, 0.02).reshape(cfg["vocab_size"], H)
        self.device_layers, self.oracle_layers = [], []
        shapes = {"q_proj": (QS, H), "k_proj": (KS, H), "v_proj": (KS, H), "o_proj": (H, QS),
                  "gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I)}
        oracle_names = {"q_proj": "q", "k_proj": "k", "v_proj": "v", "o_proj": "o",
                        "gate_proj": "gate", "up_proj": "up", "down_proj": "down"}
        for _ in range(cfg["num_hidden_layers"]):
            norms = {n: (1.0 + 0.05 * rng.standard_normal(d)).astype(np.float32)
                     for n, d in (("input_layernorm", H), ("q_norm", hd), ("k_norm", hd),
                                  ("post_attention_layernorm", H))}
            dev = dict(norms)
            orc = {"input_norm": norms["input_layernorm"], "q_norm": norms["q_norm"],
                   "k_norm": norms["k_norm"], "post_norm": norms["post_attention_layernorm"]}
            for name, (n, k) in shapes.items():
                s += 1
                blocks, deq = _proj(qtype, n, k, s)
                dev[name] = (qtype, OUTPUT_ROWS, blocks)
                orc[oracle_names[name]] = deq
            self.device_layers.append(dev)
            self.oracle_layers.append(orc)
        self.final_norm = (1.0 + 0.05 * rng.standard_normal(H)).astype(np.float32)
        s += 1
        self.head_blocks, self.head = _proj(head_qtype, cfg["vocab_size"], H, s)
        self.head_qtype = head_qtype

    def device_model(self, ctx):
        import quantinfer_amd as qa
        m = qa.Qwen3(ctx, self.cfg)
        m.set_embedding(self.embedding)
        for i, layer in enumerate(self.device_layers):
            m.set_layer(i, layer)
        m.set_output(self.final_norm, (self.head_qtype, OUTPUT_ROWS, self.head_blocks))
        return m

    def oracle_model(self, capacity: int, threads: int = 4):
        return po.Qwen3(oracle_config(self.cfg), self.embedding, self.oracle_layers,
                        self.final_norm, self.head, capacity, threads)


def prompt(cfg: dict, n: int, seed: int = 7) -> np.ndarray:
    return np.random.default_rng(seed).integers(0, cfg["vocab_size"], n).astype(np.int32)
