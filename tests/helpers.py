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


KAPPA_CAP = 64.0


def guarded_rel_err(actual, exact, x, w_deq, kappa=KAPPA_CAP):
    """max_i |a_i - e_i| / max(|e_i|, sum_k |x_k w_ik| / 64).

    `exact` is the f64 product of x and the dequantized weights. Relative error
    for outputs whose dot-product condition number sum|x w| / |e| is at most 64;
    beyond that the error is measured against sum|x w| / 64, because no f32
    summation order (the CPU reference's included) is accurate to 1e-5
    relative on an output that cancels further."""
    absdot = np.abs(x.astype(np.float64)) @ np.abs(w_deq.astype(np.float64)).T
    denom = np.maximum(np.abs(exact), absdot / kappa)
    denom = np.where(denom == 0, 1.0, denom)
    return float(np.max(np.abs(actual.astype(np.float64) - exact) / denom))


def normwise_rel_err(actual, reference):
    """max_i |a_i - r_i| / max_i |r_i| (r: the CPU reference's f32 result)."""
    r = reference.astype(np.float64)
    return float(np.max(np.abs(actual.astype(np.float64) - r)) / max(np.max(np.abs(r)), 1e-300))


def reference_bound_ok(actual, exact):
    """runtime/src/linear/tests.rs:152: |a - e| < 1e-4 + 1e-5 |e|."""
    return bool(np.all(np.abs(actual.astype(np.float64) - exact) < 1e-4 + 1e-5 * np.abs(exact)))
