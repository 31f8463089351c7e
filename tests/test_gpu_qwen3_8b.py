"""Greedy token identity on the end-to-end config at its real size.

the random-init Qwen3-8B-architecture decoder (36
layers, hidden 4096, 32 query / 8 KV heads of 128, SwiGLU 12288, vocab
151936; every linear Q4_K, the head Q6_K; f32 embedding and norms) of
quantinfer_amd.synth's recipe, a 512-token uniform random prompt, then 128
greedy decode steps with the KV cache on the GPU. "Token ids must match the
CPU run": the CPU run is the oracle's (CpuScalar linears on the same blocks,
oracle/qwen3.c), committed as tests/golden/qwen3_8b_greedy.json by
tests/golden/make_qwen3_8b_golden.py (about 20 minutes on 8 cores, so it is
not recomputed here).

The weights are rebuilt on the box with the library's own generator and
quantizer (qi_hip_synth_normal, qi_hip_quantize), which equal the oracle's
byte for byte (tests/test_abi_cpu.py); the test first checks the rebuilt
weights' digest against the fixture's, so a mismatch in the inputs cannot
pass for a mismatch in the decoder.

F32 mode, the decoder's default (the split-half matrix-core GEMM for the
512-row prompt's Q4_K linears, f32 GEMV for the steps), must give the CPU
run's ids exactly. AUTO mode (the f16-operand GEMM for the 512-row prompt)
is run beside it: measured on MI355X it leaves the CPU run at step 1, whose
CPU top-2 gap is 5e-4 of the logit scale, inside the f16 GEMM's error; the
test holds it to that (a divergence only at such a near-tie).
"""
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "qwen3_8b_greedy.json")


@pytest.fixture(scope="module")
def golden():
    if not os.path.exists(GOLDEN):
        pytest.skip("tests/golden/qwen3_8b_greedy.json not generated")
    with open(GOLDEN) as f:
        return json.load(f)


@pytest.fixture(scope="module")
def model(golden):
    import quantinfer_amd as qa
    from quantinfer_amd import synth
    from tests.golden.make_qwen3_8b_golden import weights_digest
    cfg = dict(golden["config"])
    print("building the Qwen3-8B-shape weights (synth_normal + quantize)", flush=True)
    w = synth.qwen3_weights(cfg, golden["seed"], qa.Q4_K, qa.Q6_K)
    digest = weights_digest(w)
    print(f"weights digest {digest}", flush=True)
    assert digest == golden["weights_digest_blake2b128"]
    ctx = qa.Context(0)
    dev = synth.device_model(ctx, cfg, w)
    del w
    yield cfg, ctx, dev
    dev.free()
    ctx.close()


def _generate(qa, dev, golden, mode):
    dev.set_mode(mode)
    prompt = np.array(golden["prompt"], dtype=np.int32)
    cache = dev.kv_cache(len(prompt) + len(golden["tokens"]))
    got = dev.generate(cache, prompt, len(golden["tokens"]))
    t = dev.last_timing()
    cache.free()
    return got, t


def _report(name, got, want, gaps):
    first = next((i for i, (a, b) in enumerate(zip(got, want)) if a != b), None)
    print(f"{name}: {sum(a == b for a, b in zip(got, want))}/{len(want)} ids equal; first difference "
          f"{first}; smallest CPU top-2 gap {min(gaps):.3e} at step {int(np.argmin(gaps))}", flush=True)
    return first


def test_f32_mode_greedy_ids_equal_cpu_run(model, golden):
    import quantinfer_amd as qa
    cfg, ctx, dev = model
    got, t = _generate(qa, dev, golden, qa.MODE_F32)
    first = _report("f32", got, golden["tokens"], golden["top2_gap"])
    print(f"  prefill {t.prefill_ms:.1f} ms, decode {t.decode_ms:.1f} ms", flush=True)
    assert first is None and len(got) == len(golden["tokens"])


def test_auto_mode_diverges_only_at_a_near_tie(model, golden):
    """AUTO: the prompt's linears run on the f16-operand GEMM (normwise error
    up to 2e-3 per layer, against 1e-5 for the f32 kernels), the decode steps
    on the f32 GEMV. At this config the CPU run has near-ties (top-2 logit
    gaps down to 5e-4 of the logit scale), so AUTO's ids can leave the CPU
    run's; they must not do so before the prompt's own argmax, and the first
    difference must come at a step whose CPU top-2 gap is within the GEMM's
    error bar (2e-3 of the largest logit), i.e. a tie the f16 operands cannot
    resolve, not a defect. Token identity is F32 mode's guarantee (above)."""
    import quantinfer_amd as qa
    cfg, ctx, dev = model
    got, t = _generate(qa, dev, golden, qa.MODE_AUTO)
    first = _report("auto", got, golden["tokens"], golden["top2_gap"])
    print(f"  prefill {t.prefill_ms:.1f} ms, decode {t.decode_ms:.1f} ms", flush=True)
    assert len(got) == len(golden["tokens"])
    if first is not None:
        assert first >= 1, "the prompt's argmax differs"
        rel = golden["top2_gap"][first] / golden["max_abs_logit"][first]
        print(f"  CPU top-2 gap at step {first}: {golden['top2_gap'][first]:.3e} ({rel:.2e} of max |logit|)",
              flush=True)
        assert rel < 2e-3, rel
