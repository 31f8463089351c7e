"""Greedy token ids of the end-to-end config, computed by the CPU oracle.

the random-init Qwen3-8B-architecture decoder (36
layers, hidden 4096, 32/8 heads of 128, SwiGLU 12288, vocab 151936; every
linear Q4_K, the head Q6_K) of quantinfer_amd.synth's recipe, a 512-token
uniform random prompt, then 128 greedy steps. The oracle (oracle/qwen3.c)
runs every linear as the CpuScalar output-row matmul on the quantized blocks
(runtime/src/qwen3/mod.rs:117-378, generation.rs:58-76, 174-201).

Writes tests/golden/qwen3_8b_greedy.json: the prompt, the 128 ids, the
top-1/top-2 logit gap at every selection (how far each choice is from a
tie), and a digest of the weights so that a test can tell that it rebuilt the
same model. Run from the repository root:

    python tests/golden/make_qwen3_8b_golden.py [--threads N]

It needs about 10 GB of memory and a few minutes on 8 cores.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import pyoracle as po  # noqa: E402
from quantinfer_amd import synth  # noqa: E402
from tests.qwen3_model import oracle_config, oracle_fns  # noqa: E402

OUT = os.path.join(ROOT, "tests", "golden", "qwen3_8b_greedy.json")
PROMPT_TOKENS = 512
NEW_TOKENS = 128


def weights_digest(w: dict) -> str:
    """blake2b over every projection's blocks (layer order), the head's blocks,
    the embedding and the norm vectors."""
    h = hashlib.blake2b(digest_size=16)
    h.update(np.ascontiguousarray(w["embedding"]).tobytes())
    for layer in w["layers"]:
        for n in ("input_layernorm", "q_norm", "k_norm", "post_attention_layernorm"):
            h.update(layer[n].tobytes())
        for p in synth.PROJECTIONS:
            h.update(layer[p][2].tobytes())
    h.update(w["final_norm"].tobytes())
    h.update(w["head"][2].tobytes())
    return h.hexdigest()


def top2_gap(logits: np.ndarray) -> float:
    part = np.partition(logits.astype(np.float64), -2)
    return float(part[-1] - part[-2])


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 1)
    args = ap.parse_args()
    cfg = dict(synth.QWEN3_8B)
    t0 = time.time()
    normal, quantize = oracle_fns()
    w = synth.qwen3_weights(cfg, synth.DEFAULT_SEED, po.Q4_K, po.Q6_K, normal=normal, quantize=quantize)
    digest = weights_digest(w)
    print(f"weights built in {time.time() - t0:.1f} s, digest {digest}", flush=True)
    layers = []
    for dev in w["layers"]:
        d = {"input_norm": dev["input_layernorm"], "q_norm": dev["q_norm"], "k_norm": dev["k_norm"],
             "post_norm": dev["post_attention_layernorm"]}
        for name, short in (("q_proj", "q"), ("k_proj", "k"), ("v_proj", "v"), ("o_proj", "o"),
                            ("gate_proj", "gate"), ("up_proj", "up"), ("down_proj", "down")):
            q, _, blocks = dev[name]
            d[short] = (q, blocks)
        layers.append(d)
    hq, _, hb = w["head"]
    model = po.Qwen3(oracle_config(cfg), w["embedding"], layers, w["final_norm"], (hq, hb),
                     PROMPT_TOKENS + NEW_TOKENS, args.threads)
    prompt = synth.prompt(cfg, PROMPT_TOKENS)
    t1 = time.time()
    logits = model.forward(prompt, last_only=True)[0]
    print(f"prompt forward {time.time() - t1:.1f} s", flush=True)
    tokens, gaps, max_abs = [], [], []
    for step in range(NEW_TOKENS):
        tok = po.argmax(logits)
        tokens.append(tok)
        gaps.append(top2_gap(logits))
        max_abs.append(float(np.max(np.abs(logits))))
        if step + 1 < NEW_TOKENS:
            logits = model.forward(np.array([tok], dtype=np.int32), last_only=True)[0]
        if step % 16 == 15:
            print(f"step {step + 1}/{NEW_TOKENS} ({time.time() - t1:.0f} s)", flush=True)
    rec = {
        "config": cfg,
        "recipe": "quantinfer_amd.synth.qwen3_weights(seed=0x5EED0004, Q4_K, head Q6_K)",
        "seed": synth.DEFAULT_SEED,
        "prompt_seed": synth.PROMPT_SEED,
        "weights_digest_blake2b128": digest,
        "prompt": [int(t) for t in prompt],
        "tokens": tokens,
        "top2_gap": gaps,
        "max_abs_logit": max_abs,
        "oracle_threads": args.threads,
        "seconds": round(time.time() - t0, 1),
    }
    with open(OUT, "w") as f:
        json.dump(rec, f)
        f.write("\n")
    print(f"wrote {OUT}: min top-2 gap {min(gaps):.3e}, {time.time() - t0:.0f} s")


if __name__ == "__main__":
    main()
