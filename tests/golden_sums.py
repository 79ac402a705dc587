"""The reference's causal_sum_lookup outputs (tests/golden/sum_vectors.json,
written by tests/golden/make_sum_vectors.py) as tensors, and the bound on how
far the reference's own arithmetic may lie from the exact sums.

The reference (ravel_lm/ravel_memory.py:216-224) takes a global cumulative
sum over the sorted tape in the payload dtype and subtracts the prefix before
each segment.  Each of the two prefixes and the difference are rounded once,
so with u the dtype's unit roundoff and S_d the sum of |payload[..., d]| over
the valid records (a bound on every prefix), the reference result r of an exact
sum x satisfies |r - x| <= 2u (2 S_d + |x|) (the factor 2 covers the
accumulation inside the cumulative sum).  Integer cases keep every prefix
exactly representable, so there r == x.
"""
import json
import math
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
VEC = json.load(open(os.path.join(HERE, "golden", "sum_vectors.json")))
CASES = VEC["cases"]

DTYPES = {"float32": torch.float32, "float64": torch.float64, "bfloat16": torch.bfloat16,
          "float16": torch.float16}
UNIT = {torch.float32: 2.0 ** -24, torch.float64: 2.0 ** -53, torch.bfloat16: 2.0 ** -9,
        torch.float16: 2.0 ** -12}


def _decode(values):
    special = {"nan": math.nan, "inf": math.inf, "-inf": -math.inf, "-0": -0.0}
    return [special[v] if isinstance(v, str) else float(v) for v in values]


def tensors(case):
    """(write, read or None, payload, A, write_mask or None, ref_sum, ref_mask)."""
    dt = DTYPES[case["dtype"]]
    shape = case["shape"]
    p = torch.tensor(_decode(case["payload"]), dtype=torch.float64).view(shape).to(dt)
    w = torch.tensor(case["write"], dtype=torch.long)
    r = None if case["read"] is None else torch.tensor(case["read"], dtype=torch.long)
    m = None if case["write_mask"] is None else torch.tensor(case["write_mask"], dtype=torch.bool)
    s = torch.tensor(_decode(case["sum"]), dtype=torch.float64).view(shape).to(dt)
    mask = torch.tensor(case["mask"], dtype=torch.bool)
    return w, r, p, case["address_space"], m, s, mask


def reference_bound(payload, truth, write_mask=None):
    """Per-element bound on |reference - exact| (float64, shape of truth)."""
    p = payload.double().abs()
    if write_mask is not None:
        p = p * write_mask.view(*write_mask.shape, 1, 1).double()
    S = p.sum(dim=(0, 1, 2))  # [D]
    u = UNIT[payload.dtype]
    return 2 * u * (2 * S.view(1, 1, 1, -1) + truth.abs())
