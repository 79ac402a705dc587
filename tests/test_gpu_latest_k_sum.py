"""GPU parity of causal_last_k_and_sum_lookup: the latest-k lookup and the
segmented sum of one tape in one call (the pair that the reference memory layer
makes with use_sum_read, ravel_lm/model.py:366-386).

Bar, on every case:
  * sources bit-exact to the oracle's history replay (and to the sources that
    causal_last_k_sources returns);
  * values and latest-k masks bit-exact (copies of the oracle's source rows;
    the same tensors causal_last_k_lookup returns);
  * sums within the accumulation bound of tests/test_gpu_sum.py against the
    oracle's fp64 per-stream sums, and bit-identical to causal_sum_lookup's
    (the joint kernels add in the same order); sum masks exact.
The cases reach each of the call's three forms: the merged short-tape kernel
with sources (T <= 4096, k <= 8, rows of whole 16-byte units), the long-tape
walker with latest-1 values (reads = writes, no mask, k = 1), and the two
operators back to back (everything else).
"""
import numpy as np
import pytest
import torch

import oracle
from ravel_em import (LayerAddresses, causal_last_k_and_sum_lookup, causal_last_k_lookup,
                      causal_last_k_sources, causal_sum_lookup, workloads)
from ravel_em import _native as nat
from ravel_em import _ops
from test_gpu_latest_k import expected_values
from test_gpu_sum import compare_sums, oracle_terms, sum_depth

pytestmark = pytest.mark.gpu


def joint_sources(write, payload, read, A, k, mask):
    """The joint call through its op body with sources wanted."""
    w = write.contiguous()
    r = None if read is None else read.contiguous()
    m = None if mask is None else mask.bool().contiguous()
    return _ops.latest_k_sum_impl(w, payload.contiguous(), r, m, int(A), int(k), True)


def check_joint(write, payload, read=None, *, A, k, mask=None, label="", against_separate=True):
    label = label or f"{tuple(payload.shape)} {payload.dtype} A={A} k={k}"
    print(f"[joint parity] {label}", flush=True)
    vals, vmask, summ, smask = causal_last_k_and_sum_lookup(write, payload, read, address_space=A,
                                                            k=k, write_mask=mask)
    svals, svmask, src, ssum, ssmask = joint_sources(write, payload, read, A, k, mask)
    torch.cuda.synchronize()
    osrc = oracle.latest_k_src(write, read, address_space=A, k=k, write_mask=mask)
    gsrc = src.cpu().numpy()
    bad = np.argwhere(gsrc != osrc)
    assert bad.size == 0, f"{len(bad)} source mismatches, first at {bad[:3].tolist()}"
    assert torch.equal(vmask.cpu(), torch.from_numpy(osrc >= 0))
    assert torch.equal(vals, expected_values(payload, osrc))
    assert torch.equal(svals, vals) and torch.equal(svmask, vmask)
    truth, tmask = oracle.seg_sum(write, payload, read, address_space=A, write_mask=mask)
    assert torch.equal(smask.cpu(), tmask) and torch.equal(ssmask, smask)
    scale, _ = oracle.seg_sum(write, payload.abs(), read, address_space=A, write_mask=mask)
    n = oracle_terms(write, read, A, mask, write.shape)
    B, T, C, D = payload.shape
    got = summ.cpu()
    compare_sums(got, truth, scale, n, payload.dtype, sum_depth(T, D, payload.dtype), label)
    assert not got[~tmask].any(), "reads without an earlier record must be zero"
    assert torch.equal(ssum, summ)
    if against_separate:
        _, _, src1 = causal_last_k_sources(write, payload, read, address_space=A, k=k,
                                           write_mask=mask)
        sum1, _ = causal_sum_lookup(write, payload, read, address_space=A, write_mask=mask)
        assert torch.equal(src1, src)
        assert torch.equal(sum1, summ), "joint sums differ from causal_sum_lookup's"


def test_joint_exact(device):
    # the reference's KATs (tests/test_memory.py:16-23, :61-67) in one call
    addr = torch.tensor([[[1], [2], [1], [1]]], device=device)
    payload = torch.tensor([1.0, 10.0, 3.0, 7.0], device=device).view(1, 4, 1, 1)
    vals, vmask, summ, smask = causal_last_k_and_sum_lookup(addr, payload, address_space=8, k=2)
    assert vals[0, 3, 0, :, 0].cpu().tolist() == [3.0, 1.0]
    assert vmask[0, 3, 0].cpu().tolist() == [True, True]
    assert vals[0, 2, 0, :, 0].cpu().tolist() == [1.0, 0.0]
    assert summ.cpu().view(-1).tolist() == [0.0, 0.0, 1.0, 4.0]
    assert smask.cpu().view(-1).tolist() == [False, False, True, True]


CASES = [
    # B, T, C, A, masked, separate reads, k
    (2, 17, 3, 11, False, False, 1),
    (2, 17, 3, 11, False, True, 1),
    (3, 40, 2, 5, True, False, 3),
    (2, 33, 4, 7, True, True, 4),
    (2, 25, 2, 1, False, False, 2),     # one address: every run is the whole segment
    (2, 9, 2, 4, False, False, 8),
    (2, 300, 3, 2, False, True, 5),     # long runs over many walkers, per-slot stores
    (40, 300, 8, 37, False, False, 4),  # more segments than CUs: 512-thread blocks
    (2, 1000, 3, 2, False, False, 8),   # reads at the writes, k = 8: long runs, carried ring
    (1, 4096, 2, 3, False, False, 6),   # the same at T = 4096, k = 6 of a ring of 8
    (3, 700, 2, 5, False, False, 3),    # k = 3 of a ring of 4, long runs
    (40, 300, 8, 3, True, True, 8),
    (1, 3000, 2, 2, True, False, 8),    # runs far longer than two walker ranges
    (3, 4096, 2, 300, False, True, 4),  # the longest merged tape
    (2, 4096, 1, 1, False, False, 1),   # one run of 8192 items
    (2, 700, 3, 23, False, False, 12),  # k > 8: the two operators
    (3, 5000, 2, 300, False, False, 1),  # long tape: the walker writes the values
    (1, 70000, 1, 2, False, False, 1),  # long runs across many walker parts
    (1, 70000, 1, 3, True, True, 2),    # long tape with mask and reads: the pair
    (2, 3000, 3, 1 << 21, False, False, 1),  # 64-bit packed keys
    (2, 9000, 3, 1 << 17, False, False, 1),  # 3 digit passes, long tape
]


@pytest.mark.parametrize("case", CASES, ids=[str(i) for i in range(len(CASES))])
@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 64), (torch.float32, 8), (torch.float16, 24),
                                     (torch.float64, 6)])
def test_joint_parity(device, case, dtype, D):
    B, T, C, A, masked, sep, k = case
    g = torch.Generator().manual_seed(7 * T + D + k)
    w = torch.randint(0, A, (B, T, C), generator=g)
    r = torch.randint(0, A, (B, T, C), generator=g) if sep else None
    m = (torch.rand(B, T, generator=g) < 0.6) if masked else None
    p = torch.randn(B, T, C, D, generator=g).to(dtype)
    check_joint(w.to(device), p.to(device), None if r is None else r.to(device), A=A, k=k,
                mask=None if m is None else m.to(device))


@pytest.mark.parametrize("G", [1, 2, 4, 8, 16, 32, 64])
@pytest.mark.parametrize("k", [3, 8])
def test_joint_fold_every_row_width(device, G, k):
    """Runs longer than two walker ranges (two addresses a segment) at every row width of the
    short-tape kernel: every block folds its walkers' tails and carries their rings."""
    D = G * 8  # bf16: G 16-byte units a row
    B, T, C, A = 3, 512, 2, 2
    g = torch.Generator().manual_seed(G + k)
    w = torch.randint(0, A, (B, T, C), generator=g)
    p = torch.randn(B, T, C, D, generator=g).to(torch.bfloat16)
    check_joint(w.to(device), p.to(device), None, A=A, k=k)


@pytest.mark.parametrize("D,dtype", [(5, torch.float32), (3, torch.float16), (1, torch.float64),
                                     (128, torch.bfloat16), (64, torch.float16),
                                     (8, torch.float64)])
def test_joint_row_shapes(device, D, dtype):
    """Rows that are not whole 16-byte units (the pair), wide rows, and fp16 and
    fp64 rows of whole units (the long tape's walker writes their values)."""
    g = torch.Generator().manual_seed(D)
    for (B, T, C, A, k) in [(2, 300, 3, 17, 3), (2, 6000, 2, 40, 1)]:
        w = torch.randint(0, A, (B, T, C), generator=g)
        p = torch.randn(B, T, C, D, generator=g).to(dtype)
        check_joint(w.to(device), p.to(device), None, A=A, k=k)


def test_joint_int32_addresses_and_wrap(device):
    g = torch.Generator().manual_seed(11)
    B, T, C, A = 2, 500, 3, 13
    w = torch.randint(-40, 40, (B, T, C), generator=g).to(torch.int32)
    r = torch.randint(-40, 40, (B, T, C), generator=g).to(torch.int32)
    p = torch.randn(B, T, C, 16, generator=g).to(torch.bfloat16)
    check_joint(w.to(device), p.to(device), r.to(device), A=A, k=4)
    check_joint(w.to(device), p.to(device), None, A=A, k=1)


def test_joint_all_masked_and_empty(device):
    w = torch.randint(0, 5, (2, 8, 3), device=device)
    p = torch.randn(2, 8, 3, 4, device=device)
    m = torch.zeros(2, 8, dtype=torch.bool, device=device)
    vals, vmask, summ, smask = causal_last_k_and_sum_lookup(w, p, address_space=5, k=2, write_mask=m)
    assert not vmask.any() and not vals.any() and not smask.any() and not summ.any()
    w0 = torch.zeros(0, 8, 3, dtype=torch.long, device=device)
    p0 = torch.zeros(0, 8, 3, 4, device=device)
    vals, vmask, summ, smask = causal_last_k_and_sum_lookup(w0, p0, address_space=5, k=2)
    assert vals.shape == (0, 8, 3, 2, 4) and vmask.shape == (0, 8, 3, 2)
    assert summ.shape == (0, 8, 3, 4) and smask.shape == (0, 8, 3)


def test_joint_argument_errors(device):
    w = torch.zeros(1, 4, 2, dtype=torch.long, device=device)
    p = torch.zeros(1, 4, 2, 3, device=device)
    with pytest.raises(ValueError, match="k must be positive"):
        causal_last_k_and_sum_lookup(w, p, address_space=4, k=0)
    with pytest.raises(ValueError, match="write_mask must have shape"):
        causal_last_k_and_sum_lookup(w, p, address_space=4,
                                     write_mask=torch.ones(2, 4, dtype=torch.bool, device=device))


@pytest.mark.parametrize("sep,masked,k,T", [(False, False, 1, 300), (True, True, 3, 300),
                                            (False, False, 1, 5000), (False, True, 2, 5000)])
def test_joint_gradients(device, sep, masked, k, T):
    """Gradients of values and sums together equal those of the two separate ops."""
    g = torch.Generator().manual_seed(T + k)
    B, C, A, D = 2, 3, 17, 16
    w = torch.randint(0, A, (B, T, C), generator=g).to(device)
    r = torch.randint(0, A, (B, T, C), generator=g).to(device) if sep else None
    m = (torch.rand(B, T, generator=g) < 0.6).to(device) if masked else None
    p = torch.randn(B, T, C, D, generator=g).to(device).requires_grad_(True)
    gv = torch.randn(B, T, C, k, D, generator=g).to(device)
    gs = torch.randn(B, T, C, D, generator=g).to(device)
    vals, _, summ, _ = causal_last_k_and_sum_lookup(w, p, r, address_space=A, k=k, write_mask=m)
    (vals * gv).sum().add((summ * gs).sum()).backward()
    got = p.grad.clone()
    p.grad = None
    v1, _ = causal_last_k_lookup(w, p, r, address_space=A, k=k, write_mask=m)
    s1, _ = causal_sum_lookup(w, p, r, address_space=A, write_mask=m)
    (v1 * gv).sum().add((s1 * gs).sum()).backward()
    torch.testing.assert_close(got, p.grad, rtol=1e-5, atol=1e-5)


def test_joint_split_ranges(device):
    """Calls split into row ranges give the unsplit results (sources bit for bit)."""
    lib = nat.library()
    g = torch.Generator().manual_seed(5)
    for (B, T, C, A, k, sep) in [(5, 300, 3, 11, 4, True), (4, 5000, 2, 37, 1, False)]:
        w = torch.randint(0, A, (B, T, C), generator=g).to(device)
        r = torch.randint(0, A, (B, T, C), generator=g).to(device) if sep else None
        p = torch.randn(B, T, C, 16, generator=g).to(device, torch.bfloat16)
        full = joint_sources(w, p, r, A, k, None)
        lib.ravel_em_set_split_slots(T * C * k)  # one batch row per range
        try:
            split = joint_sources(w, p, r, A, k, None)
        finally:
            lib.ravel_em_set_split_slots(0)
        for a, b in zip(full, split):
            assert torch.equal(a, b)


@pytest.mark.parametrize("offs", [(1, 3, 0), (5, 5, 0), (0, 7, 0), (2, 9, 1)])
def test_joint_walker_masks_at_byte_offsets(device, offs):
    """The long-tape joint form (reads = writes, no mask, k = 1) writes the sum
    mask at random records and copies it into the latest-1 mask: through the C
    entry point, masks that start at any byte offset (alike or unlike modulo 16,
    so the copy takes its byte path or its head, 16-byte body and tail) equal
    the aligned call's, and the bytes around them stay untouched.  With the
    values and sums one element off 16-byte alignment the call takes its
    two-operator form, whose kernels store in units the pointers allow."""
    lib = nat.library()
    g = torch.Generator().manual_seed(11)
    B, T, C, D, A = 2, 6000, 3, 64, 700  # T > 4096: the sorted walker path
    w = torch.randint(0, A, (B, T, C), generator=g).to(device)
    p = torch.randn(B, T, C, D, generator=g).to(device, torch.bfloat16)
    want = joint_sources(w, p, None, A, 1, None)
    n = B * T * C
    vbuf = torch.full((n + 32,), 0xA5, dtype=torch.uint8, device=device)
    sbuf = torch.full((n + 32,), 0x5A, dtype=torch.uint8, device=device)
    o1, o2, e = offs
    values = p.new_empty(n * D + 8)[e:e + n * D].view(B, T, C, 1, D)
    out = p.new_empty(n * D + 8)[e:e + n * D].view(B, T, C, D)
    code = nat.payload_code(p.dtype)
    nbytes = lib.ravel_em_latest_k_sum_workspace(B, T, C, D, A, 1, 0, 0, 0, code)
    ws = nat.workspace(nbytes, device)
    print(f"[joint masks] offsets {offs}", flush=True)
    nat.check(lib.ravel_em_latest_k_sum_fwd(
        nat.ptr(w), None, nat.addr_code(w.dtype), None, nat.ptr(p), code, B, T, C, D, A, 1,
        nat.ptr(values), vbuf.data_ptr() + o1, None, nat.ptr(out), sbuf.data_ptr() + o2,
        nat.ptr(ws), ws.numel(), nat.stream_of(p)))
    nat.after_call(ws)
    torch.cuda.synchronize()
    assert torch.equal(values, want[0])
    if e == 0:
        assert torch.equal(out, want[3])
    else:  # another kernel's order of additions: within the sum bound of the fp64 truth
        truth, _ = oracle.seg_sum(w, p, None, address_space=A)
        scale, _ = oracle.seg_sum(w, p.abs(), None, address_space=A)
        compare_sums(out.cpu(), truth, scale, oracle_terms(w, None, A, None, w.shape), p.dtype,
                     sum_depth(T, D, p.dtype, walker=False), f"offsets {offs}")
    assert torch.equal(vbuf[o1:o1 + n].bool(), want[1].reshape(-1))
    assert torch.equal(sbuf[o2:o2 + n].bool(), want[4].reshape(-1))
    assert torch.equal(vbuf[o1:o1 + n], sbuf[o2:o2 + n])  # 0/1 bytes, the same in both
    assert bool((vbuf[:o1] == 0xA5).all()) and bool((vbuf[o1 + n:] == 0xA5).all())
    assert bool((sbuf[:o2] == 0x5A).all()) and bool((sbuf[o2 + n:] == 0x5A).all())


def test_joint_produced_addresses(device):
    """LayerAddresses: addresses produced in the call give the tensor call's results."""
    g = torch.Generator().manual_seed(3)
    B, T, A = 2, 600, 64
    tokens = torch.randint(0, 300, (B, T), generator=g).to(device)
    logits = torch.randn(B, T, 2 * 2 * 8, generator=g).to(device)
    rlogits = torch.randn(B, T, 2 * 2 * 8, generator=g).to(device)
    p = torch.randn(B, T, 5, 16, generator=g).to(device, torch.bfloat16)
    for rl in (None, rlogits):
        src = LayerAddresses(token_ids=tokens, n_literal_heads=3, bos_token_id=257,
                             write_logits=logits, read_logits=rl, n_learned_heads=2,
                             n_codebooks=2, codebook_size=8)
        wa, ra = src.materialize(address_space=A)
        got = causal_last_k_and_sum_lookup(src, p, address_space=A, k=2)
        want = causal_last_k_and_sum_lookup(wa, p, None if rl is None else ra, address_space=A, k=2)
        for a, b in zip(got, want):
            assert torch.equal(a, b)


@pytest.mark.parametrize("name", ["cfg1", "cfg1b", "cfg2_f32", "cfg2_bf16", "cfg3", "cfg4",
                                  "cfg4_adv"])
def test_joint_baseline_configs(device, name):
    w = {
        "cfg1": lambda: workloads.cfg1(device),
        "cfg1b": lambda: workloads.cfg1(device, variant="1b"),
        "cfg2_f32": lambda: workloads.cfg2(device, torch.float32),
        "cfg2_bf16": lambda: workloads.cfg2(device, torch.bfloat16),
        "cfg3": lambda: workloads.cfg3(device),
        "cfg4": lambda: workloads.cfg4(device),
        "cfg4_adv": lambda: workloads.cfg4(device, adversarial=True),
    }[name]()
    check_joint(w.write, w.payload, w.read, A=w.address_space, k=w.k, label=name,
                against_separate=name in ("cfg1", "cfg2_bf16", "cfg4"))
