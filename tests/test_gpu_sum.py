"""GPU parity of causal_sum_lookup against the fp64 oracle.

The reference's own cumsum-minus-prefix arithmetic is far less accurate than
these kernels (it rounds global prefixes), so the ground truth is the oracle's
fp64 per-stream sum, and the bound is the accumulation error these kernels
can make plus one rounding of the result:

  fp32 / fp64 payloads (accumulated in fp64, rounded once):
      |gpu - truth| <= 1e-5 |truth| + (n-1) 2^-52 S
  bf16 / fp16 payloads (accumulated in fp32, rounded once):
      |gpu - truth| <= 1e-2 |truth| + min(n-1, depth) 2^-24 S

n is the number of terms of the output, S their sum of absolute values, and
depth the longest chain of additions one term passes through in the kernel's
summation tree (sum_depth below): a walker's own positions, the fold over the
walkers of a part and the look-back over earlier parts (walker kernel), or a
64-position chunk and the carry scan over chunks (chunk kernels).  A sum of n
terms formed by any tree has first-order error <= min(n-1, depth) u S, so these
bounds follow from the kernels' structure; 1e-5 and 1e-2 are the relative
tolerances the benchmark statement sets.  Every check prints the largest
relative error it saw and its largest fraction of the bound.  Masks are exact.
The reference's own outputs on small inputs (tests/golden/sum_vectors.json)
are matched bit-exactly where its arithmetic is exact and within its rounding
bound elsewhere.
"""
import math

import pytest
import torch

import golden_sums
import oracle
from ravel_em import causal_sum_lookup, workloads

pytestmark = pytest.mark.gpu

RTOL = {torch.float32: 1e-5, torch.float64: 1e-5, torch.bfloat16: 1e-2, torch.float16: 1e-2}
# the smallest subnormal of the output dtype: a floor for rounding near zero
TINY = {torch.float32: 2.0 ** -149, torch.float64: 2.0 ** -1074, torch.bfloat16: 2.0 ** -133,
        torch.float16: 2.0 ** -24}


def sum_depth(T: int, D: int, dtype: torch.dtype, walker: bool = True) -> int:
    """Longest addition chain of one term in the GPU summation (em_sum.hip).

    Merged kernel (2T <= 8192, the same rows): see the comment in the body.
    Walker kernel (rows of 1..64 whole 16-byte units, 16-byte aligned): a part
    of 1024 positions is split over NW = 256 / G walkers of L = 1024 / NW
    positions; a term is added along its walker's tail (<= L), the part's fold
    over walkers (<= NW), the look-back over earlier parts (<= ceil(T / 1024)),
    the carry fold into its walker (<= NW) and the final walk (<= L).  Chunk
    kernels: a 64-position chunk, the carry scan (<= 2 ceil(nch / 16) + 16 over
    nch = ceil(T / 64) chunks) and the fix-up walk (<= 64)."""
    row = D * torch.empty((), dtype=dtype).element_size()
    G = row // 16
    if walker and row % 16 == 0 and 1 <= G <= 64 and G & (G - 1) == 0:
        nw = 256 // G
        depth = 2 * (1024 // nw) + 2 * nw + math.ceil(T / 1024)
        if 2 * T <= 8192:
            # short tapes may take the one-block merged kernel: 2T items over
            # NW = 512 / G walkers of L items (a multiple of 16), the walkers'
            # tails folded in NG groups of NW / NG (NG = min(64, 512 / D))
            nw = 512 // G
            n2r = -(-2 * T // 16) * 16
            L = -(-(-(-n2r // nw)) // 16) * 16
            ng = min(64, 512 // D)
            depth = max(depth, 2 * L + 2 * (nw // ng) + ng)
        return depth
    nch = math.ceil(T / 64)
    return 64 + 2 * math.ceil(nch / 16) + 16 + 64


def sum_bound(truth, scale, n, dtype, depth):
    """Allowed |gpu - truth| per element (see the module docstring)."""
    terms = (n - 1).clamp_min(0)
    if dtype in (torch.float32, torch.float64):
        acc = terms * 2.0 ** -52 * scale
    else:
        acc = terms.clamp_max(depth) * 2.0 ** -24 * scale
    return RTOL[dtype] * truth.abs() + 1.01 * acc + TINY[dtype]


def compare_sums(got, truth, scale, n, dtype, depth, label=""):
    """Assert got is within sum_bound of truth; print the largest errors."""
    got = got.double()
    err = (got - truth).abs()
    lim = sum_bound(truth, scale, n, dtype, depth)
    frac = (err / lim).max().item() if err.numel() else 0.0
    nz = truth != 0
    rel = (err[nz] / truth[nz].abs()).max().item() if nz.any() else 0.0
    # outputs whose terms do not cancel much (|truth| >= S / 100)
    wc = nz & (truth.abs() * 100 >= scale)
    rel_wc = (err[wc] / truth[wc].abs()).max().item() if wc.any() else 0.0
    print(f"[sum parity] {label} max rel err {rel:.3e} (where |sum| >= S/100: {rel_wc:.3e}), "
          f"max err/bound {frac:.3f}", flush=True)
    assert frac <= 1.0, f"sum bound exceeded: max err/bound {frac}"


def oracle_terms(write, read, A, mask, shape):
    """Per output: the number of terms n (from an all-ones payload)."""
    B, T, C = shape
    ones = torch.ones(B, T, C, 1, dtype=torch.float64)
    n, _ = oracle.seg_sum(write, ones, read, address_space=A, write_mask=mask)
    return n


def check_sum(write, payload, read=None, *, A, mask=None, walker=True, label=""):
    out, omask = causal_sum_lookup(write, payload, read, address_space=A, write_mask=mask)
    truth, tmask = oracle.seg_sum(write, payload, read, address_space=A, write_mask=mask)
    scale, _ = oracle.seg_sum(write, payload.abs(), read, address_space=A, write_mask=mask)
    n = oracle_terms(write, read, A, mask, write.shape)
    assert torch.equal(omask.cpu(), tmask)
    B, T, C, D = payload.shape
    got = out.cpu()
    compare_sums(got, truth, scale, n, payload.dtype, sum_depth(T, D, payload.dtype, walker),
                 label or f"{tuple(payload.shape)} {payload.dtype}")
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
    (40, 300, 8, 37, False, False),  # more segments than CUs: 512-thread blocks
    (40, 300, 8, 3, True, True),
    (8, 512, 4, 2, False, False),  # runs across walkers: every block folds, one iteration a walker
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


@pytest.mark.parametrize("G", [1, 2, 4, 8, 16, 32, 64])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_sum_fold_every_row_width(device, G, dtype):
    """Two addresses a segment make runs longer than two walker ranges, so every block of the
    short-tape kernel folds its walkers' tails; the fold's groups and the pads between them
    depend on the 16-byte units of a row, G = 1 .. 64."""
    D = G * 16 // torch.empty((), dtype=dtype).element_size()
    B, T, C, A = 3, 512, 2, 2
    g = torch.Generator().manual_seed(G)
    w = torch.randint(0, A, (B, T, C), generator=g)
    p = torch.randn(B, T, C, D, generator=g).to(dtype)
    print(f"[fold sum] G={G} D={D} {dtype}", flush=True)
    check_sum(w.to(device), p.to(device), A=A)


def test_sum_integer_payloads_are_exact(device):
    """Small integers sum exactly in every dtype: compare bit-for-bit."""
    g = torch.Generator().manual_seed(4)
    B, T, C, A, D = 2, 3000, 3, 5, 4
    w = torch.randint(0, A, (B, T, C), generator=g)
    p = torch.randint(-3, 4, (B, T, C, D), generator=g).float()
    out, mask = causal_sum_lookup(w.to(device), p.to(device), address_space=A)
    truth, tmask = oracle.seg_sum(w, p, address_space=A)
    assert torch.equal(out.cpu().double(), truth) and torch.equal(mask.cpu(), tmask)


@pytest.mark.parametrize("name", ["cfg1", "cfg1b", "cfg2_f32", "cfg2_bf16", "cfg3", "cfg4",
                                  "cfg4_adv"])
def test_sum_baseline_configs(device, name):
    print(f"[sum parity] {name}", flush=True)
    w = {
        "cfg1": lambda: workloads.cfg1(device),
        "cfg1b": lambda: workloads.cfg1(device, variant="1b"),
        "cfg2_f32": lambda: workloads.cfg2(device, torch.float32),
        "cfg2_bf16": lambda: workloads.cfg2(device, torch.bfloat16),
        "cfg3": lambda: workloads.cfg3(device),
        "cfg4": lambda: workloads.cfg4(device),
        "cfg4_adv": lambda: workloads.cfg4(device, adversarial=True),
    }[name]()
    check_sum(w.write, w.payload, w.read, A=w.address_space, label=name)


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
    n = oracle_terms(w, r, A, m, w.shape)
    depth = sum_depth(w.shape[1], p.shape[-1], p.dtype)
    lim = golden_sums.reference_bound(p, truth, m) + sum_bound(truth, scale, n, p.dtype, depth)
    assert ((out.double() - ref.double()).abs() <= lim).all()


# Separate reads without a write mask: rows of 1 to 8 16-byte units in every
# payload dtype, over the short-tape sort's sizes and one step past them.
SEP_ROWS = [(torch.float32, 4), (torch.float32, 16), (torch.bfloat16, 64), (torch.float16, 8),
            (torch.float64, 2), (torch.float64, 16)]
SEP_SHAPES = [
    (2, 1, 3, 5),      # one step: every read sees nothing
    (2, 17, 3, 11),
    (3, 1000, 2, 7),   # long runs spanning every walker of a segment
    (1, 4096, 2, 1),   # one address; the longest short tape
    (2, 4096, 2, 4096),
    (2, 1025, 1, 300),
    (1, 2049, 3, 40),
    (1, 4097, 1, 50),  # one step over: the global sort
]


@pytest.mark.parametrize("shape", SEP_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("dtype,D", SEP_ROWS, ids=lambda x: str(x).replace("torch.", ""))
def test_sum_separate_reads(device, shape, dtype, D):
    B, T, C, A = shape
    print(f"[separate-read sum] {shape} {dtype} D={D}", flush=True)
    g = torch.Generator().manual_seed(T * 7 + D)
    w = torch.randint(-A, 2 * A, (B, T, C), generator=g)  # out-of-range ids wrap (Python %)
    r = torch.randint(-A, 2 * A, (B, T, C), generator=g)
    p = torch.randn(B, T, C, D, generator=g).to(dtype)
    check_sum(w.to(device), p.to(device), r.to(device), A=A)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 64), (torch.float32, 4)])
def test_sum_reads_equal_to_writes_match_direct(device, dtype, D):
    """The same addresses passed as separate reads give the direct sum (integer
    payloads, so the two paths' different summation orders agree exactly)."""
    g = torch.Generator().manual_seed(11)
    w = torch.randint(0, 9, (2, 3000, 4), generator=g).to(device)
    p = torch.randint(-3, 4, (2, 3000, 4, D), generator=g).to(dtype).to(device)
    direct, dmask = causal_sum_lookup(w, p, address_space=9)
    sep, smask = causal_sum_lookup(w, p, w.clone(), address_space=9)
    assert torch.equal(dmask, smask) and torch.equal(direct, sep)


def test_sum_reads_disjoint_from_writes(device):
    g = torch.Generator().manual_seed(12)
    w = torch.randint(0, 50, (2, 2000, 3), generator=g).to(device)
    r = torch.randint(50, 100, (2, 2000, 3), generator=g).to(device)
    p = torch.randn(2, 2000, 3, 8, generator=g).to(device)
    out, mask = causal_sum_lookup(w, p, r, address_space=100)
    assert not mask.any() and not out.any()



@pytest.mark.parametrize("sep", [False, True])
def test_sum_unaligned_payload(device, sep):
    """A payload view 2 bytes into its storage (16-byte rows that are not
    16-byte aligned) takes the chunk kernels instead of the walker."""
    g = torch.Generator().manual_seed(31)
    B, T, C, D, A = 2, 700, 3, 8, 13
    w = torch.randint(0, A, (B, T, C), generator=g)
    r = torch.randint(0, A, (B, T, C), generator=g) if sep else None
    base = torch.randn(B * T * C * D + 1, generator=g).to(torch.bfloat16)
    p = base.to(device)[1:].view(B, T, C, D)
    assert p.data_ptr() % 16 != 0 and p.is_contiguous()
    check_sum(w.to(device), p, None if r is None else r.to(device), A=A, walker=False)


# Rows of 64 16-byte units (the walker's widest): 512 bf16/fp16 columns, two per
# thread in the part fold, 256 fp32 and 128 fp64 columns.  Long runs (few
# addresses) cross the 1024-position parts, so every carry and look-back path
# is exercised, forward and backward.
WIDE_ROWS = [(torch.bfloat16, 512), (torch.float16, 512), (torch.float32, 256),
             (torch.float64, 128)]
WIDE_SHAPES = [(1, 3000, 2, 3, False, False), (2, 5000, 1, 40, False, False),
               (1, 3000, 2, 3, False, True), (2, 2500, 2, 5, True, False)]


@pytest.mark.parametrize("shape", WIDE_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("dtype,D", WIDE_ROWS, ids=lambda x: str(x).replace("torch.", ""))
def test_sum_wide_rows(device, shape, dtype, D):
    B, T, C, A, masked, sep = shape
    print(f"[wide-row sum] {shape} {dtype} D={D}", flush=True)
    g = torch.Generator().manual_seed(T + D + 5)
    w = torch.randint(0, A, (B, T, C), generator=g)
    r = torch.randint(0, A, (B, T, C), generator=g) if sep else None
    m = (torch.rand(B, T, generator=g) < 0.7) if masked else None
    p = torch.randn(B, T, C, D, generator=g).to(dtype)
    check_sum(w.to(device), p.to(device), None if r is None else r.to(device), A=A,
              mask=None if m is None else m.to(device), label=f"wide {shape} {dtype}")


@pytest.mark.parametrize("shape", WIDE_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("dtype,D", WIDE_ROWS, ids=lambda x: str(x).replace("torch.", ""))
def test_sum_wide_rows_backward(device, shape, dtype, D):
    B, T, C, A, masked, sep = shape
    print(f"[wide-row sum backward] {shape} {dtype} D={D}", flush=True)
    g = torch.Generator().manual_seed(T + D + 6)
    w = torch.randint(0, A, (B, T, C), generator=g)
    r = torch.randint(0, A, (B, T, C), generator=g) if sep else None
    m = (torch.rand(B, T, generator=g) < 0.7) if masked else None
    p = torch.randn(B, T, C, D, generator=g).to(dtype)
    gy = torch.randn(B, T, C, D, generator=g).to(dtype)
    pg = p.to(device).requires_grad_(True)
    out, _ = causal_sum_lookup(w.to(device), pg, None if r is None else r.to(device), address_space=A,
                               write_mask=None if m is None else m.to(device))
    (grad,) = torch.autograd.grad(out, pg, gy.to(device))
    want, scale, n = oracle.seg_sum_grad(w, gy, r, address_space=A, write_mask=m)
    # Reads = writes: the reverse walk of the forward's kernels.  Separate reads
    # or a mask: the read gradients are first added per sorted write position
    # with atomics (fp64 for fp32/fp64 payloads, fp32 for 16-bit ones), in no
    # fixed order, so the chain is bounded by n only.
    depth = sum_depth(T, D, dtype) if r is None and m is None else T
    compare_sums(grad.cpu(), want, scale, n, dtype, depth, f"wide backward {shape} {dtype}")
