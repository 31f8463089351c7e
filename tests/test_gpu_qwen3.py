"""GPU-resident Qwen3 decoder (qi_hip_qwen3_*) against the CPU oracle.

The oracle (oracle/qwen3.c) restates the reference forward pass with the
CpuScalar matmuls. The device decoder sums in other orders (MFMA GEMV,
parallel reductions), so logits are compared within a tolerance and greedy
token ids exactly: the end-to-end acceptance is "token ids must match the CPU
run". Small configurations keep the CPU side to seconds; the full
Qwen3-8B-shape run is bench.py --workload e2e.
"""
import numpy as np
import pytest

from tests.qwen3_model import Qwen3Weights, prompt, small_config

pytestmark = pytest.mark.gpu

# Normwise tolerance of the last-row logits, max|dev - cpu| / max|cpu|: f32
# GEMV / exact-order linears (1e-5 per layer) and reordered f32 reductions in
# norms and attention; f16-operand GEMM prefill (2e-3 per layer).
TOL_F32 = 1e-4
TOL_MFMA = 5e-3


def _rel(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b)) / np.max(np.abs(b)))


@pytest.fixture(scope="module")
def qa():
    import quantinfer_amd
    return quantinfer_amd


@pytest.fixture(scope="module")
def ctx(qa):
    c = qa.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def small(ctx):
    cfg = small_config(max_position_embeddings=1024)
    w = Qwen3Weights(cfg)
    dev = w.device_model(ctx)
    yield cfg, w, dev
    dev.free()


@pytest.mark.parametrize("mode", ["f32", "exact", "auto"])
def test_forward_logits_match_oracle(qa, small, mode):
    cfg, w, dev = small
    print(f"qwen3 forward mode={mode}", flush=True)
    dev.set_mode({"f32": qa.MODE_F32, "exact": qa.MODE_EXACT, "auto": qa.MODE_AUTO}[mode])
    cache = dev.kv_cache(64)
    ref = w.oracle_model(64)
    toks = prompt(cfg, 11)
    for step, chunk in enumerate([toks, [17], [901]]):
        logits, nxt = dev.forward(cache, chunk)
        want = ref.forward(chunk, last_only=True)[0]
        err = _rel(logits, want)
        print(f"  step {step}: rel err {err:.2e}", flush=True)
        assert err <= TOL_F32, (mode, step, err)
        assert nxt == int(np.argmax(logits))
        assert cache.length == ref.length
    dev.set_mode(qa.MODE_F32)  # back to the default


def test_generate_tokens_identical_to_cpu(qa, small):
    cfg, w, dev = small
    dev.set_mode(qa.MODE_F32)
    toks = prompt(cfg, 20, seed=11)
    print("qwen3 generate f32 prompt=20 new=24", flush=True)
    cache = dev.kv_cache(128)
    got = dev.generate(cache, toks, 24)
    want = w.oracle_model(128).generate(toks, 24)
    print(f"  gpu {got}\n  cpu {want}", flush=True)
    assert got == want
    assert cache.length == 20 + 24
    t = dev.last_timing()
    assert t.prompt_tokens == 20 and t.decode_steps == 24
    assert t.prefill_ms > 0 and t.decode_ms > 0
    dev.set_mode(qa.MODE_F32)  # back to the default


def test_default_mode_prompt_on_split_gemm_identical_to_cpu(qa, ctx):
    """A freshly created decoder runs in its default mode, F32: a 100-token
    prompt takes the split-half GEMM (48+ rows of Q4_K), and the greedy ids
    equal the CPU run's."""
    cfg = small_config(max_position_embeddings=256)
    w = Qwen3Weights(cfg, seed=0x5EED0011)
    dev = w.device_model(ctx)
    toks = prompt(cfg, 100, seed=17)
    print("qwen3 default mode prompt=100 new=16", flush=True)
    cache = dev.kv_cache(128)
    got = dev.generate(cache, toks, 16)
    want = w.oracle_model(128).generate(toks, 16)
    print(f"  gpu {got}\n  cpu {want}", flush=True)
    assert got == want
    dev.free()


@pytest.mark.parametrize("env", ["QI_HIP_QWEN3_UNFUSED", "QI_HIP_QWEN3_EAGER"])
def test_decode_variants_identical_to_cpu(qa, ctx, small, env, monkeypatch):
    """Decode steps with the separate element-wise kernels (instead of the
    GEMV-fused ones), and steps launched one by one (instead of the replayed
    graph), select the CPU run's tokens too."""
    cfg, w, _ = small
    monkeypatch.setenv(env, "1")
    dev = w.device_model(ctx)  # the switch is read when the model is created
    monkeypatch.delenv(env)
    dev.set_mode(qa.MODE_F32)
    toks = prompt(cfg, 20, seed=11)
    print(f"qwen3 generate {env}=1 prompt=20 new=16", flush=True)
    cache = dev.kv_cache(64)
    got = dev.generate(cache, toks, 16)
    want = w.oracle_model(64).generate(toks, 16)
    assert got == want
    dev.free()


def test_generate_matches_forward_loop(qa, small):
    """Decode steps replayed from the captured graph select the same tokens
    as step-by-step forward calls."""
    cfg, w, dev = small
    dev.set_mode(qa.MODE_F32)
    toks = prompt(cfg, 9, seed=12)
    print("qwen3 graph vs forward loop", flush=True)
    cache = dev.kv_cache(64)
    gen = dev.generate(cache, toks, 10)
    cache2 = dev.kv_cache(64)
    _, t = dev.forward(cache2, toks, logits=False)
    loop = []
    for _ in range(10):
        loop.append(t)
        _, t = dev.forward(cache2, [t], logits=False)
    assert gen == loop
    assert cache.length == cache2.length
    # a reset cache generates the same again
    cache.reset()
    assert cache.length == 0
    assert dev.generate(cache, toks, 10) == gen
    dev.set_mode(qa.MODE_F32)  # back to the default


def test_prefill_gemm_and_chunked_prompt(qa, small):
    """AUTO mode: a 600-token prompt runs as a 512-row and an 88-row chunk,
    both through the MFMA GEMM, with attention over 10 position chunks."""
    cfg, w, dev = small
    dev.set_mode(qa.MODE_AUTO)
    toks = prompt(cfg, 600, seed=13)
    print("qwen3 auto prompt=600 new=6", flush=True)
    cache = dev.kv_cache(640)
    ref = w.oracle_model(640)
    logits, nxt = dev.forward(cache, toks)
    want = ref.forward(toks, last_only=True)[0]
    err = _rel(logits, want)
    print(f"  prefill rel err {err:.2e}", flush=True)
    assert err <= TOL_MFMA
    # then decode in F32 from the same cache, against the oracle's cache
    got, exp = [nxt], [int(np.argmax(want))]
    for _ in range(5):
        lg, nxt = dev.forward(cache, [got[-1]])
        wl = ref.forward([exp[-1]], last_only=True)[0]
        got.append(nxt)
        exp.append(int(np.argmax(wl)))
    print(f"  gpu {got}\n  cpu {exp}", flush=True)
    assert got == exp
    assert cache.length == 605


def test_prompt_silu_in_gemm_epilogue(qa, ctx, monkeypatch):
    """AUTO prefill of 512 rows with intermediate 8192: the gate|up GEMM
    (K = 256, N = 16384: 64 x 4 blocks, no K split) writes SiLU(gate) * up in
    its epilogue, on the LDS-staged kernel and (QI_HIP_GEMM_REG=1, read at
    each GEMM call) on the register-weight kernel. The logits are identical
    to the run with the separate SiLU kernel (QI_HIP_QWEN3_UNFUSED=1: the same
    GEMM accumulators and the same f32 expression), and the greedy token
    matches the CPU oracle's."""
    cfg = small_config(hidden_size=256, intermediate_size=8192, num_hidden_layers=1,
                       num_attention_heads=2, num_key_value_heads=1, head_dim=128,
                       vocab_size=512, max_position_embeddings=512)
    w = Qwen3Weights(cfg, seed=0x5EED0300)
    toks = prompt(cfg, 512, seed=30)
    print("qwen3 prompt=512 intermediate=8192 fused vs unfused SiLU", flush=True)
    got = {}
    for variant in ("fused", "fused-register-kernel", "unfused"):
        if variant == "unfused":
            monkeypatch.setenv("QI_HIP_QWEN3_UNFUSED", "1")
        dev = w.device_model(ctx)
        monkeypatch.delenv("QI_HIP_QWEN3_UNFUSED", raising=False)
        dev.set_mode(qa.MODE_AUTO)
        cache = dev.kv_cache(512)
        if variant == "fused-register-kernel":
            monkeypatch.setenv("QI_HIP_GEMM_REG", "1")
        got[variant] = dev.forward(cache, toks)
        monkeypatch.delenv("QI_HIP_GEMM_REG", raising=False)
        dev.free()
    assert got["fused"][0].tobytes() == got["unfused"][0].tobytes()
    assert got["fused-register-kernel"][0].tobytes() == got["unfused"][0].tobytes()
    want = w.oracle_model(512).forward(toks, last_only=True)[0]
    err = _rel(got["fused"][0], want)
    print(f"  rel err {err:.2e}", flush=True)
    assert err <= TOL_MFMA
    assert got["fused"][1] == int(np.argmax(want))


def test_eos_stops_generation(qa, small):
    cfg, w, dev = small
    dev.set_mode(qa.MODE_F32)
    toks = prompt(cfg, 8, seed=14)
    cache = dev.kv_cache(64)
    gen = dev.generate(cache, toks, 12)
    eos = gen[3]
    first = gen.index(eos)
    cache.reset()
    print(f"qwen3 eos={eos}", flush=True)
    assert dev.generate(cache, toks, 12, eos=eos) == gen[:first + 1]
    # the EOS itself is not forwarded (generation.rs:189-195)
    assert cache.length == 8 + first
    dev.set_mode(qa.MODE_F32)  # back to the default


def test_head_dim_128_group_4(qa, ctx):
    """The Qwen3-8B attention geometry: head_dim 128, 4 query heads per KV head."""
    cfg = small_config(hidden_size=1024, intermediate_size=1024, num_hidden_layers=1,
                       num_attention_heads=8, num_key_value_heads=2, head_dim=128,
                       vocab_size=2048)
    w = Qwen3Weights(cfg, seed=0x5EED0104)
    dev = w.device_model(ctx)
    dev.set_mode(qa.MODE_F32)
    toks = prompt(cfg, 70, seed=15)
    print("qwen3 hd128 prompt=70 new=12", flush=True)
    cache = dev.kv_cache(96)
    got = dev.generate(cache, toks, 12)
    want = w.oracle_model(96).generate(toks, 12)
    print(f"  gpu {got}\n  cpu {want}", flush=True)
    assert got == want
    dev.free()


@pytest.mark.parametrize("kernel", ["mfma", "fma"])
def test_head_dim_128_prefill_row_blocks(qa, ctx, kernel, monkeypatch):
    """AUTO prefill at head_dim 128, 4 query heads per KV head, 302 rows (a
    partial last block): the prompt attention on the matrix cores (blocks of
    16 rows) and, with QI_HIP_QWEN3_ATTN_FMA=1, on the FMA kernel (blocks of 4
    rows); then decode continues from the same cache."""
    cfg = small_config(hidden_size=1024, intermediate_size=1024, num_hidden_layers=1,
                       num_attention_heads=8, num_key_value_heads=2, head_dim=128,
                       vocab_size=2048, max_position_embeddings=512)
    w = Qwen3Weights(cfg, seed=0x5EED0105)
    if kernel == "fma":
        monkeypatch.setenv("QI_HIP_QWEN3_ATTN_FMA", "1")
    dev = w.device_model(ctx)  # the switch is read when the model is created
    monkeypatch.delenv("QI_HIP_QWEN3_ATTN_FMA", raising=False)
    dev.set_mode(qa.MODE_AUTO)
    toks = prompt(cfg, 302, seed=16)
    print(f"qwen3 hd128 auto prompt=302 attention={kernel}", flush=True)
    cache = dev.kv_cache(320)
    ref = w.oracle_model(320)
    logits, nxt = dev.forward(cache, toks)
    want = ref.forward(toks, last_only=True)[0]
    err = _rel(logits, want)
    print(f"  prefill rel err {err:.2e}", flush=True)
    assert err <= TOL_MFMA
    assert nxt == int(np.argmax(want))
    lg, _ = dev.forward(cache, [nxt])
    wl = ref.forward([nxt], last_only=True)[0]
    assert _rel(lg, wl) <= TOL_MFMA
    dev.free()


@pytest.mark.parametrize("group", [1, 2, 8])
def test_head_dim_128_prompt_attention_groups(qa, ctx, group):
    """F32 mode, head_dim 128, 1/2/8 query heads per KV head: a 100-row
    prompt, then a 50-row chunk on top of the cached positions (rows of a
    block attend to up to 150 positions in 3 chunks, a partial block last)."""
    cfg = small_config(hidden_size=1024, intermediate_size=1024, num_hidden_layers=1,
                       num_attention_heads=8, num_key_value_heads=8 // group, head_dim=128,
                       vocab_size=2048, max_position_embeddings=256)
    w = Qwen3Weights(cfg, seed=0x5EED0200 + group)
    dev = w.device_model(ctx)
    dev.set_mode(qa.MODE_F32)
    toks = prompt(cfg, 150, seed=20 + group)
    print(f"qwen3 hd128 group={group} prompt=100+50", flush=True)
    cache = dev.kv_cache(192)
    ref = w.oracle_model(192)
    for chunk in (toks[:100], toks[100:]):
        logits, nxt = dev.forward(cache, chunk)
        want = ref.forward(chunk, last_only=True)[0]
        err = _rel(logits, want)
        print(f"  rel err {err:.2e}", flush=True)
        assert err <= TOL_F32
        assert nxt == int(np.argmax(logits))
    dev.free()


def test_errors(qa, ctx, small):
    cfg, w, dev = small
    cache = dev.kv_cache(16)
    with pytest.raises(qa.QiError) as e:
        dev.forward(cache, [cfg["vocab_size"]])
    assert e.value.status == qa.INVALID_INPUT
    with pytest.raises(qa.QiError) as e:
        dev.forward(cache, prompt(cfg, 17))
    assert e.value.status == qa.INVALID_INPUT and "capacity" in str(e.value)
    assert cache.length == 0
    with pytest.raises(qa.QiError) as e:
        dev.generate(cache, prompt(cfg, 10), 8)  # needs 18 positions
    assert e.value.status == qa.INVALID_INPUT
    bad = qa.KvCache(ctx, cfg["num_hidden_layers"] + 1, 16, cfg["num_key_value_heads"],
                     cfg["head_dim"])
    with pytest.raises(qa.QiError) as e:
        dev.forward(bad, [1])
    assert "layout" in str(e.value)
    bad.free()
    empty = qa.Qwen3(ctx, cfg)
    c2 = empty.kv_cache(16)
    with pytest.raises(qa.QiError) as e:
        empty.forward(c2, [1])
    assert e.value.status == qa.INVALID_INPUT
    c2.free()
    empty.free()
    with pytest.raises(qa.QiError) as e:
        qa.Qwen3(ctx, small_config(head_dim=32))
    assert e.value.status == qa.UNSUPPORTED


def test_fused_groups_must_share_format(qa, ctx, small):
    """q|k|v and gate|up are uploaded as fused projections: a layer that mixes
    formats inside a group is refused with UNSUPPORTED (such models take the
    per-linear path), while o, down and the head may differ."""
    from oracle import pyoracle as po
    cfg, w, _ = small
    m = qa.Qwen3(ctx, cfg)
    try:
        base = dict(w.device_layers[0])
        for group_member in ("v_proj", "up_proj"):
            layer = dict(base)
            qtype, layout, blocks = layer[group_member]
            values = po.dequantize(qtype, blocks)
            layer[group_member] = (qa.Q8_0, layout, qa.quantize(qa.Q8_0, values, storage_f16=True))
            with pytest.raises(qa.QiError) as e:
                m.set_layer(0, layer)
            assert e.value.status == qa.UNSUPPORTED and "fused projections" in str(e.value)
        # a different format outside the groups is accepted
        layer = dict(base)
        qtype, layout, blocks = layer["o_proj"]
        values = po.dequantize(qtype, blocks)
        layer["o_proj"] = (qa.Q8_0, layout, qa.quantize(qa.Q8_0, values, storage_f16=True))
        m.set_layer(0, layer)
    finally:
        m.free()
