"""Non-finite payloads (inf, -inf, NaN, -0.0) through the lookups.

Latest-k: a slot with a source is a bit-exact copy of the source row (NaN
payload bits, infinities and -0.0 included); a slot without one is +0.0.  The
reference's generic path multiplies a clamped neighbour's row by the validity
mask (ravel_lm/ravel_memory.py:173-175), so its empty slots are +0.0, -0.0 or
NaN depending on an unrelated record; its GPU arm writes +0.0
(ravel_lm/triton_latest1.py:67-68), which is what this library does.

Segmented sum: sums are per stream, so a non-finite payload reaches only the
later outputs of its own (b, c, a) stream, with IEEE semantics (inf + -inf =
NaN), exactly as the oracle's per-stream fp64 sums.  The reference's global
cumsum-minus-prefix (ravel_memory.py:216-229) would spread it to every later
output of the whole tape; that is a property of its arithmetic, not of the
operator, and is not reproduced.
"""
import pytest
import torch

import oracle
from ravel_em import causal_last_k_lookup, causal_sum_lookup
from test_gpu_sum import oracle_terms, sum_bound, sum_depth

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.view({2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()])


def _poisoned(B, T, C, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    p = torch.randn(B, T, C, D, generator=g)
    flat = p.view(-1, D)
    n = flat.shape[0]
    idx = torch.randperm(n, generator=g)[: max(4, n // 50)]
    specials = torch.tensor([float("inf"), float("-inf"), float("nan"), -0.0])
    flat[idx] = specials[torch.arange(idx.numel()) % 4].view(-1, 1)
    return p.to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("sep,k", [(False, 1), (False, 3), (True, 2)])
def test_latest_k_non_finite_rows_copy_bits_and_empty_slots_are_positive_zero(device, dtype, sep, k):
    B, T, C, D, A = 2, 300, 3, 16, 7
    g = torch.Generator().manual_seed(5 + k)
    w = torch.randint(0, A, (B, T, C), generator=g)
    r = torch.randint(0, A, (B, T, C), generator=g) if sep else None
    p = _poisoned(B, T, C, D, dtype, 17 + k)
    vals, mask = causal_last_k_lookup(w.to(device), p.to(device), None if r is None else r.to(device),
                                      address_space=A, k=k)
    ov, om, _ = oracle.latest_k(w, p, r, address_space=A, k=k)
    assert torch.equal(mask.cpu(), om)
    assert torch.equal(_bits(vals.cpu()), _bits(ov))  # NaN bits, -0.0, inf and +0.0 alike
    empty = vals.cpu()[~om]
    assert empty.numel() > 0 and (_bits(empty) == 0).all(), "empty slots must be +0.0"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("sep", [False, True])
def test_sum_non_finite_stays_in_its_stream(device, dtype, sep):
    B, T, C, D, A = 2, 3000, 3, 8, 5
    g = torch.Generator().manual_seed(41)
    w = torch.randint(0, A, (B, T, C), generator=g)
    r = torch.randint(0, A, (B, T, C), generator=g) if sep else None
    p = torch.randn(B, T, C, D, generator=g)
    p[0, 100, 1, 2] = float("nan")   # one NaN, one inf and one -inf in one stream's column
    p[1, 200, 0, :] = float("inf")
    p[1, 1200, 0, :] = float("-inf")
    p = p.to(dtype)
    out, omask = causal_sum_lookup(w.to(device), p.to(device), None if r is None else r.to(device),
                                   address_space=A)
    truth, tmask = oracle.seg_sum(w, p, r, address_space=A)
    got = out.cpu().double()
    assert torch.equal(omask.cpu(), tmask)
    assert torch.equal(torch.isnan(got), torch.isnan(truth))
    assert torch.equal(torch.isposinf(got), torch.isposinf(truth))
    assert torch.equal(torch.isneginf(got), torch.isneginf(truth))
    assert torch.isnan(truth).any() and torch.isinf(truth).any()
    fin = torch.isfinite(truth)
    # the finite outputs, within the accumulation bound of tests/test_gpu_sum.py:
    # other streams are untouched by the non-finite records
    scale, _ = oracle.seg_sum(w, p.abs(), r, address_space=A)
    n = oracle_terms(w, r, A, None, w.shape)
    lim = sum_bound(truth, scale, n, dtype, sum_depth(T, D, dtype))
    assert ((got - truth).abs()[fin] <= lim[fin]).all()
    assert fin.float().mean() > 0.5
