"""Pin the oracle's binary16 conversions (the `half` 2.7.1 arithmetic the
reference uses for every f16 scale) against numpy's IEEE binary16."""
import numpy as np

from tests.helpers import load_golden


def test_f16_to_f32_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = oracle.f16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(ours[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    assert np.array_equal(np.isinf(ours), np.isinf(ref))


def test_f32_to_f16_round_to_nearest_even_at_every_boundary(oracle):
    # every half value, the midpoints between neighbours and one ulp (f32) on
    # each side of every midpoint: exactly where a rounding mistake shows
    h = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16)
    v = h.view(np.float16).astype(np.float64)
    nxt = np.append(v[1:], 65520.0)  # 65520 = first value that rounds to inf
    mid = ((v + nxt) / 2).astype(np.float32)
    cand = np.concatenate([
        v.astype(np.float32), mid,
        np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(0)),
    ])
    cand = np.concatenate([cand, -cand, np.array([1e-9, 3e-8, 2.98e-8, 2.9802322e-8, 7e4, 1e38],
                                                 dtype=np.float32)])
    ours = oracle.f32_to_f16(cand)
    ref = cand.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


def test_f32_to_f16_random(oracle):
    rng = np.random.default_rng(7)
    raw = rng.integers(0, 2 ** 32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    x = raw.view(np.float32)
    x = x[np.isfinite(x)]
    assert np.array_equal(oracle.f32_to_f16(x), x.astype(np.float16).view(np.uint16))


def test_reference_half_vector(oracle):
    # format/src/gguf/tests.rs:191: 0.5 is stored as [0x00, 0x38]
    case = [w for w in load_golden()["wire"] if w["name"] == "f16_half_is_0x3800"][0]
    h = int(oracle.f32_to_f16([case["f32"]])[0])
    assert [h & 0xFF, h >> 8] == case["f16_le_bytes"]


def test_stored_f16_scale_subnormal_rule(oracle):
    # quant schemes/mod.rs:27-40: a positive value that rounds to zero becomes
    # the smallest subnormal; everything else is plain round-to-nearest.
    assert oracle.stored_f16_scale(1e-9) == 2.0 ** -24
    assert oracle.stored_f16_scale(0.0) == 0.0
    assert oracle.stored_f16_scale(5e-5) == float(np.float32(np.float16(5e-5)))
    import pytest
    with pytest.raises(oracle.OracleError):
        oracle.stored_f16_scale(1e6)
