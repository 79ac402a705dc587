"""The fp64 sum oracle against the reference's own causal_sum_lookup outputs
(tests/golden/sum_vectors.json): masks bit-exact; integer cases, where the
reference's arithmetic is exact, bit-exact; every other case within the
rounding bound of the reference's cumsum-minus-prefix arithmetic.  Planted
mistakes in a copy of the oracle's result (a dropped record, the read at t
instead of before t) fail those checks."""
import pytest
import torch

import oracle
from golden_sums import CASES, reference_bound, tensors


def _check(case, truth, tmask):
    w, r, p, A, m, ref, rmask = tensors(case)
    if not torch.equal(tmask, rmask):
        return False
    if case["name"].startswith("int_") or case["name"] in ("all_masked", "single_address"):
        return torch.equal(truth.to(ref.dtype), ref)
    err = (ref.double() - truth).abs()
    return bool((err <= reference_bound(p, truth, m)).all())


@pytest.mark.parametrize("case", CASES, ids=lambda c: c["name"])
def test_sum_oracle_matches_reference_outputs(case):
    w, r, p, A, m, ref, rmask = tensors(case)
    truth, tmask = oracle.seg_sum(w, p, r, address_space=A, write_mask=m)
    assert _check(case, truth, tmask), case["name"]


def test_sum_vectors_cover_the_interface():
    names = {c["name"] for c in CASES}
    assert {c["dtype"] for c in CASES} == {"float32", "float64", "bfloat16", "float16"}
    assert any(c["read"] is not None for c in CASES) and any(c["write_mask"] for c in CASES)
    assert "all_masked" in names and any(n.startswith("int_") for n in names)
    wrap = next(c for c in CASES if c["name"] == "int_f64_wrap")
    flat = [a for row in wrap["write"] for t in row for a in t]
    assert min(flat) < 0 and max(flat) >= wrap["address_space"]


@pytest.mark.parametrize("name", ["int_f32", "int_f32_reads_mask", "int_bf16", "int_f16", "normal_f32",
                                  "normal_f32_reads_mask", "normal_f64"])
def test_planted_mistakes_fail_the_sum_vectors(name):
    case = next(c for c in CASES if c["name"] == name)
    w, r, p, A, m, ref, rmask = tensors(case)
    truth, tmask = oracle.seg_sum(w, p, r, address_space=A, write_mask=m)
    assert _check(case, truth, tmask)
    # One record dropped from the tape: the first valid write of (b=0, c=0).
    t0 = 0 if m is None else int(torch.nonzero(m[0])[0])
    p2 = p.clone()
    p2[0, t0, 0] = 0
    dropped, dmask = oracle.seg_sum(w, p2, r, address_space=A, write_mask=m)
    assert not _check(case, dropped, dmask)
    # Non-strict causality: reads also see the write at their own time.
    B, T, C = w.shape
    rd = w if r is None else r
    same = (rd % A) == (w % A)
    if m is not None:
        same = same & m.view(B, T, 1)
    incl = truth + p.double() * same.unsqueeze(-1)
    assert not _check(case, incl, tmask)
