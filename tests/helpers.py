"""Shared test helpers: block arrays from fixture dicts, error metrics."""
import json
import os

import numpy as np

from oracle import pyoracle as po

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_golden(name="reference_known_answers.json"):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def blocks_from_dicts(qtype, dicts):
    arr = np.zeros(len(dicts), dtype=po.BLOCK_DTYPES[qtype])
    for i, d in enumerate(dicts):
        for key, value in d.items():
            arr[i][key] = value
    return arr


def lhs_from_case(case):
    shape = case["lhs_shape"]
    if "lhs_fill" in case:
        return np.full(shape, case["lhs_fill"], dtype=np.float32)
    return np.asarray(case["lhs"], dtype=np.float32).reshape(shape)


def guarded_rel_err(actual, exact, x, w_deq):
    """max_i |a_i - e_i| / max(|e_i|, 2^-10 * sum_k |x_k w_ik|).

    `exact` is the f64 product of x and the dequantized weights; the floor keeps
    the ratio meaningful for outputs that cancel to near zero."""
    absdot = np.abs(x.astype(np.float64)) @ np.abs(w_deq.astype(np.float64)).T
    denom = np.maximum(np.abs(exact), absdot * 2.0 ** -10)
    denom = np.where(denom == 0, 1.0, denom)
    return float(np.max(np.abs(actual.astype(np.float64) - exact) / denom))


def reference_bound_ok(actual, exact):
    """runtime/src/linear/tests.rs:152: |a - e| < 1e-4 + 1e-5 |e|."""
    return bool(np.all(np.abs(actual.astype(np.float64) - exact) < 1e-4 + 1e-5 * np.abs(exact)))
