"""Pins of the oracle's Qwen3 decoder restatement (oracle/qwen3.c), CPU only.

Each check is chosen so that a plausible slip (a wrong pair index in RoPE, a
missing scale, softmax over the wrong axis, a KV cache off by one position, a
transposed projection) fails: known answers transcribed from the reference's
tests, closed forms, float64 brute force, and invariants of the forward pass.
"""
import json
import os

import numpy as np
import pytest

from oracle import pyoracle as po
from tests import numpy_ref
from tests.qwen3_model import Qwen3Weights, oracle_config, prompt, small_config

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")


def _decoder_case(name):
    with open(GOLDEN) as f:
        cases = json.load(f)["decoder"]
    return next(c for c in cases if c["name"] == name)


# ------------------------------------------------------------------- ops

def test_rope_known_answer(oracle):
    # backends/cpu/src/tests.rs:136-143
    case = _decoder_case("half_split_rope_rotation")
    x = np.array(case["input"], np.float32).reshape(case["input_shape"])
    out = oracle.apply_rope(x, np.array([case["cos"]], np.float32),
                            np.array([case["sin"]], np.float32))
    assert out.ravel().tolist() == case["expected"]


def test_rope_tables_formula_and_rotation(oracle):
    d, theta = 128, 1e6
    c, s = oracle.rope_tables(theta, d, 0, 700)
    # position 0 is the identity (cos 1, sin 0 exactly)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    # the angle position * theta^(-2i/d) evaluated in float64 from the f32
    # operands: the f32 angle is within a few ulps of it
    pos = np.arange(700, dtype=np.float64)[:, None]
    expo = (2.0 * np.arange(d // 2, dtype=np.float32) / np.float32(d)).astype(np.float64)
    ang = pos * np.float64(theta) ** (-expo)[None, :]
    tol = np.abs(ang) * 4 * 2.0 ** -24 + 2e-7
    assert np.all(np.abs(c - np.cos(ang)) <= tol)
    assert np.all(np.abs(s - np.sin(ang)) <= tol)
    # rotation preserves every pair's norm; tables can start mid-sequence
    x = np.random.default_rng(1).standard_normal((700, 3, d)).astype(np.float32)
    y = oracle.apply_rope(x, c, s)
    n0 = x[..., : d // 2] ** 2 + x[..., d // 2:] ** 2
    n1 = y[..., : d // 2].astype(np.float64) ** 2 + y[..., d // 2:].astype(np.float64) ** 2
    assert np.allclose(n1, n0, rtol=1e-5)
    c2, s2 = oracle.rope_tables(theta, d, 300, 5)
    assert np.array_equal(c2, c[300:305]) and np.array_equal(s2, s[300:305])
    # one table row broadcasts to every token
    y1 = oracle.apply_rope(x[:4], c[7:8], s[7:8])
    assert np.array_equal(y1, oracle.apply_rope(x[:4], np.repeat(c[7:8], 4, 0),
                                                np.repeat(s[7:8], 4, 0)))


def test_rms_norm_softmax_silu_closed_forms(oracle):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((5, 512)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(512)).astype(np.float32)
    got = oracle.rms_norm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
    assert np.max(np.abs(got - want) / np.abs(want).max()) < 2e-6
    # a constant row c normalizes to c / sqrt(c^2 + eps)
    c = np.full((1, 8), 0.01, np.float32)
    assert np.allclose(oracle.rms_norm(c, np.ones(8, np.float32), 1e-6),
                       0.01 / np.sqrt(1e-4 + 1e-6), rtol=1e-6)
    s = oracle.softmax(x)
    assert np.allclose(s.sum(axis=1), 1.0, rtol=1e-5)
    e = np.exp(x64 - x64.max(axis=1, keepdims=True))
    assert np.allclose(s, e / e.sum(axis=1, keepdims=True), rtol=1e-5, atol=1e-9)
    g, u = x[0], x[1]
    want = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(oracle.silu_mul(g, u), want, rtol=1e-6, atol=1e-7)


def test_gqa_attention_brute_force(oracle):
    rng = np.random.default_rng(3)
    tq, hq, hk, d, start = 4, 8, 2, 64, 9
    tk = start + tq
    q = rng.standard_normal((tq, hq, d)).astype(np.float32)
    k = rng.standard_normal((tk, hk, d)).astype(np.float32)
    v = rng.standard_normal((tk, hk, d)).astype(np.float32)
    got = oracle.gqa_attention(q, k, v, start)
    for t in range(tq):
        last = start + t
        for h in range(hq):
            g = h // (hq // hk)
            sc = k[: last + 1, g].astype(np.float64) @ q[t, h].astype(np.float64) / np.sqrt(d)
            p = np.exp(sc - sc.max())
            want = (p / p.sum()) @ v[: last + 1, g].astype(np.float64)
            assert np.allclose(got[t, h], want, rtol=1e-5, atol=1e-6), (t, h)
    # causality: keys after a query's position do not change its output
    k2, v2 = k.copy(), v.copy()
    k2[start + 1:] = 7.0
    v2[start + 1:] = -3.0
    got2 = oracle.gqa_attention(q[:1], k2, v2, start)
    assert np.array_equal(got2[0], got[0])
    # a single key returns its value exactly (softmax weight exp(0)/1 = 1)
    one = oracle.gqa_attention(q[:1], k[:1], v[:1], 0)
    assert np.array_equal(one[0, 0], v[0, 0])


def test_embedding_and_argmax(oracle):
    table = np.arange(12, dtype=np.float32).reshape(4, 3)
    assert oracle.embedding(table, [2, 0]).tolist() == [[6, 7, 8], [0, 1, 2]]
    with pytest.raises(oracle.OracleError):
        oracle.embedding(table, [4])
    # generation.rs:58-76: first index of the maximum, non-finite rejected
    assert oracle.argmax(np.array([1.0, 3.0, 3.0, 2.0], np.float32)) == 1
    with pytest.raises(oracle.OracleError):
        oracle.argmax(np.array([1.0, np.nan], np.float32))
    with pytest.raises(oracle.OracleError):
        oracle.argmax(np.array([1.0, np.inf], np.float32))


def test_linear_rows_is_the_cpu_scalar_matmul(oracle):
    """The decoder's linear equals CpuScalar's output-row matmul on the blocks
    bit for bit (matmul.rs:319-330 with the dequantized values), for one row
    and many, on 1 and 3 threads."""
    rng = np.random.default_rng(4)
    k, n = 512, 37
    blocks = oracle.quantize(oracle.Q4_K, oracle.fill_normal(11, n * k, 0.02))
    w = oracle.dequantize(oracle.Q4_K, blocks).reshape(n, k)
    for m in (1, 3, 9, 17):
        x = rng.standard_normal((m, k)).astype(np.float32)
        ref = oracle.matmul_output_rows(oracle.Q4_K, x, blocks, n)
        for threads in (1, 3):
            assert np.array_equal(oracle.linear_rows(x, w, threads), ref), (m, threads)
        assert np.array_equal(oracle.matmul_f32(x, np.ascontiguousarray(w.T)), ref)


# ------------------------------------------------------------- decoder

def test_filled_model_closed_form(oracle):
    """runtime/src/qwen3/tests.rs:22-99: with constant weights the value rows
    are constant, so attention returns them whatever the scores are, and every
    logit of every row has a closed form (evaluated here in float64)."""
    case = _decoder_case("qwen3_filled_prefill_decode")
    c, f = case["config"], case["fill"]
    H, I, V, hd = c["hidden"], c["intermediate"], c["vocab"], c["head_dim"]
    QS, KS = c["heads"] * hd, c["kv_heads"] * hd
    P = f["projections"]
    layer = {"input_norm": np.ones(H), "q_norm": np.ones(hd), "k_norm": np.ones(hd),
             "post_norm": np.ones(H), "q": np.full((QS, H), P), "k": np.full((KS, H), P),
             "v": np.full((KS, H), P), "o": np.full((H, QS), P), "gate": np.full((I, H), P),
             "up": np.full((I, H), P), "down": np.full((H, I), P)}
    m = oracle.Qwen3(c, np.full((V, H), f["embedding"]), [layer], np.ones(H),
                     np.full((V, H), f["lm_head"]), c["max_positions"], 1)
    pre = m.forward(case["prefill_tokens"])
    assert list(pre.shape) == case["expected_prefill_logits_shape"]
    assert m.length == case["expected_length_after_prefill"]
    dec = m.forward(case["decode_tokens"])
    assert list(dec.shape) == case["expected_decode_logits_shape"]
    assert m.length == case["expected_length_after_decode"]

    eps = c["eps"]
    nrm = lambda v: v / np.sqrt(v * v + eps)  # noqa: E731  (RMSNorm of a constant row)
    a = nrm(f["embedding"])
    v = H * a * P                      # every q/k/v element; attention returns v
    h1 = f["embedding"] + QS * v * P   # o projection of the constant attention output
    g = H * nrm(h1) * P                # gate == up
    h2 = h1 + I * (g / (1 + np.exp(-g)) * g) * P
    logit = H * nrm(h2) * f["lm_head"]
    for row in np.vstack([pre, dec]):
        assert np.all(row == row[0])
        assert abs(row[0] - logit) <= 1e-6 * abs(logit)
    assert oracle.argmax(dec[0]) == 0


@pytest.fixture(scope="module")
def small():
    cfg = small_config(num_hidden_layers=2)
    return cfg, Qwen3Weights(cfg)


def test_decoder_matches_float64_restatement(oracle, small):
    cfg, w = small
    m = w.oracle_model(64, threads=2)
    ref = numpy_ref.Qwen3F64(oracle_config(cfg), w.embedding, w.oracle_layers, w.final_norm,
                             w.head)
    toks = prompt(cfg, 11)
    got = m.forward(toks)
    want = ref.forward(toks)
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1e-4
    # decode rows too, through the cache of both
    for t in (5, 77, 3):
        got = m.forward([t])
        want = ref.forward([t])
        assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1e-4


def test_decoder_kv_cache_invariant(oracle, small):
    """Prompt then one token through the cache equals the whole sequence at
    once, bit for bit: every row's arithmetic is independent of how the rows
    are batched (qwen3/mod.rs forward over DecodeBatchItem)."""
    cfg, w = small
    toks = prompt(cfg, 9)
    one = w.oracle_model(32)
    full = one.forward(toks)
    two = w.oracle_model(32)
    head = two.forward(toks[:6])
    assert np.array_equal(head, full[:6])
    for i in range(6, 9):
        assert np.array_equal(two.forward(toks[i:i + 1])[0], full[i])
    assert two.length == one.length == 9
    # last-row-only projection equals the last row of the full projection
    three = w.oracle_model(32)
    assert np.array_equal(three.forward(toks, last_only=True)[0], full[-1])


def test_generate_is_forward_then_argmax_loop(oracle, small):
    cfg, w = small
    toks = prompt(cfg, 7)
    m = w.oracle_model(32)
    gen = m.generate(toks, 6)
    assert m.length == 7 + 6  # the last selected token is forwarded too (generation.rs:189-199)
    m2 = w.oracle_model(32)
    logits = m2.forward(toks, last_only=True)[0]
    manual = []
    for _ in range(6):
        t = oracle.argmax(logits)
        manual.append(t)
        logits = m2.forward([t])[0]
    assert gen == manual
    # EOS stops before forwarding it
    m3 = w.oracle_model(32)
    assert m3.generate(toks, 6, eos=gen[2]) == gen[:3]
    assert m3.length == 7 + 2
    # capacity is enforced like KvCache::append (cache.rs:113-118)
    m4 = w.oracle_model(8)
    with pytest.raises(oracle.OracleError):
        m4.forward(prompt(cfg, 9))


@pytest.mark.parametrize("qtype", [po.Q8_0, po.Q4_0, po.Q4_K, po.Q5_K, po.Q6_K])
def test_linear_on_blocks_is_the_output_row_matmul(oracle, qtype):
    """qo_linear on quantized blocks equals the CpuScalar output-row matmul
    (matmul.rs:119-160, 282-332) bit for bit, for any row count and thread
    count, and equals qo_linear_rows on the dequantized rows."""
    k, n = 512, 40
    blocks = po.quantize(qtype, po.fill_normal(21 + qtype, n * k, 0.02, 0.005, 0.2))
    deq = po.dequantize(qtype, blocks).reshape(n, k)
    for m in (1, 5, 9):
        x = po.fill_normal(m, m * k)
        ref = po.matmul_output_rows(qtype, x.reshape(m, k), blocks, n)
        for threads in (1, 3):
            y = po.linear(x.reshape(m, k), (qtype, blocks), n, threads)
            assert y.tobytes() == ref.tobytes(), (m, threads)
        assert po.linear_rows(x.reshape(m, k), deq, threads=2).tobytes() == ref.tobytes()


def test_decoder_on_blocks_equals_decoder_on_dequantized_rows(oracle, small):
    cfg, w = small
    p = prompt(cfg, 11)
    a = w.oracle_model(32, threads=3).forward(p)
    b = w.oracle_model(32, threads=2, blocks=True).forward(p)
    assert a.tobytes() == b.tobytes()
    ga = w.oracle_model(32, threads=1).generate(p, 6)
    gb = w.oracle_model(32, threads=4, blocks=True).generate(p, 6)
    assert ga == gb
