"""GPU parity of causal_sum_lookup against the fp64 oracle.

Tolerances (the reference's own cumsum-minus-prefix arithmetic is far less
accurate, so the ground truth is fp64 per-stream sums):
  fp32 / fp64 payloads: |gpu - truth| <= 1e-5 |truth| + 1e-7 * sum|x|
  bf16 / fp16 payloads: |gpu - truth| <= 1e-2 |truth| + 1e-4 * sum|x|
where sum|x| is the per-output sum of absolute payload values (the scale of the
accumulation).  Masks are exact.  The reference's own outputs on small inputs
(tests/golden/sum_vectors.json) are matched bit-exactly where its arithmetic is
exact and within its rounding bound elsewhere.
"""
import pytest
import torch

import golden_sums
import oracle
from ravel_em import causal_sum_lookup, workloads

pytestmark = pytest.mark.gpu

TOL = {torch.float32: (1e-5, 1e-7), torch.float64: (1e-5, 1e-7), torch.bfloat16: (1e-2, 1e-4),
       torch.float16: (1e-2, 1e-4)}


def check_sum(write, payload, read=None, *, A, mask=None):
    out, omask = causal_sum_lookup(write, payload, read, address_space=A, write_mask=mask)
    truth, tmask = oracle.seg_sum(write, payload, read, address_space=A, write_mask=mask)
    scale, _ = oracle.seg_sum(write, payload.abs(), read, address_space=A, write_mask=mask)
    assert torch.equal(omask.cpu(), tmask)
    rtol, atol = TOL[payload.dtype]
    got = out.cpu().double()
    err = (got - truth).abs()
    lim = rtol * truth.abs() + atol * scale
    worst = (err - lim).max().item() if err.numel() else 0.0
    assert worst <= 0, f"sum tolerance exceeded by {worst}"
    assert not got[~tmask].any(), "reads without an earlier record must be zero"


def test_causal_sum_exact(device):
    # tests/test_memory.py:61-67 of the reference
    addr = torch.tensor([[[1], [2], [1], [1]]], device=device)
    payload = torch.tensor([1.0, 10.0, 3.0, 7.0], device=device).view(1, 4, 1, 1)
    vals, mask = causal_sum_lookup(addr, payload, address_space=8)
    assert vals[0, 0, 0, 0].item() == 0.0
    assert vals[0, 2, 0, 0].item() == 1.0
    assert vals[0, 3, 0, 0].item() == 4.0
    assert mask.cpu().view(-1).tolist() == [False, False, True, True]


CASES = [
    (2, 17, 3, 11, False, False),
    (2, 17, 3, 11, False, True),
    (3, 40, 2, 5, True, False),
    (2, 33, 4, 7, True, True),
    (2, 25, 2, 1, False, False),
    (3, 5000, 2, 300, False, False),
    (1, 70000, 1, 2, False, False),  # runs spanning hundreds of chunks
    (1, 70000, 1, 3, True, True),
    (2, 3000, 3, 1 << 21, False, True),
]


@pytest.mark.parametrize("case", CASES, ids=[str(i) for i in range(len(CASES))])
@pytest.mark.parametrize("dtype,D", [(torch.float32, 5), (torch.bfloat16, 64), (torch.float16, 3),
                                     (torch.float64, 70)])
def test_sum_parity(device, case, dtype, D):
    B, T, C, A, masked, sep = case
    g = torch.Generator().manual_seed(T + D)
    w = torch.randint(0, A, (B, T, C), generator=g)
    r = torch.randint(0, A, (B, T, C), generator=g) if sep else None
    m = (torch.rand(B, T, generator=g) < 0.6) if masked else None
    p = torch.randn(B, T, C, D, generator=g).to(dtype)
    check_sum(w.to(device), p.to(device), None if r is None else r.to(device), A=A,
              mask=None if m is None else m.to(device))


def test_sum_integer_payloads_are_exact(device):
    """Small integers sum exactly in every dtype: compare bit-for-bit."""
    g = torch.Generator().manual_seed(4)
    B, T, C, A, D = 2, 3000, 3, 5, 4
    w = torch.randint(0, A, (B, T, C), generator=g)
    p = torch.randint(-3, 4, (B, T, C, D), generator=g).float()
    out, mask = causal_sum_lookup(w.to(device), p.to(device), address_space=A)
    truth, tmask = oracle.seg_sum(w, p, address_space=A)
    assert torch.equal(out.cpu().double(), truth) and torch.equal(mask.cpu(), tmask)


@pytest.mark.parametrize("name", ["cfg1", "cfg2_f32", "cfg2_bf16", "cfg3", "cfg4", "cfg4_adv"])
def test_sum_baseline_configs(device, name):
    print(f"[sum parity] {name}", flush=True)
    w = {
        "cfg1": lambda: workloads.cfg1(device),
        "cfg2_f32": lambda: workloads.cfg2(device, torch.float32),
        "cfg2_bf16": lambda: workloads.cfg2(device, torch.bfloat16),
        "cfg3": lambda: workloads.cfg3(device, B=8),
        "cfg4": lambda: workloads.cfg4(device, B=1),
        "cfg4_adv": lambda: workloads.cfg4(device, adversarial=True, B=1),
    }[name]()
    check_sum(w.write, w.payload, w.read, A=w.address_space)


@pytest.mark.parametrize("case", golden_sums.CASES, ids=lambda c: c["name"])
def test_sum_matches_reference_outputs(device, case):
    """The reference's own outputs (tests/golden/sum_vectors.json): masks bit-exact;
    integer cases, exact in the reference's arithmetic, bit-exact; otherwise
    |gpu - reference| <= (the reference's rounding bound) + (this kernel's tolerance
    against the exact sum above)."""
    w, r, p, A, m, ref, rmask = golden_sums.tensors(case)
    out, omask = causal_sum_lookup(w.to(device), p.to(device), None if r is None else r.to(device),
                                   address_space=A, write_mask=None if m is None else m.to(device))
    out, omask = out.cpu(), omask.cpu()
    assert out.dtype == ref.dtype and torch.equal(omask, rmask)
    if case["name"].startswith("int_") or case["name"] in ("all_masked", "single_address"):
        assert torch.equal(out, ref)
        return
    truth, _ = oracle.seg_sum(w, p, r, address_space=A, write_mask=m)
    scale, _ = oracle.seg_sum(w, p.abs(), r, address_space=A, write_mask=m)
    rtol, atol = TOL[p.dtype]
    lim = golden_sums.reference_bound(p, truth, m) + rtol * truth.abs() + atol * scale
    assert ((out.double() - ref.double()).abs() <= lim).all()
