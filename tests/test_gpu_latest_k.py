"""GPU parity of causal_last_k_lookup and the sort order.

Bar: sorted keys/order and latest-k source indices bit-exact to the oracle;
values are copies, so bit-exact too (missing slots are +0.0; the reference's
payload*0 can give -0.0, which compares equal).
"""
import json
import os

import numpy as np
import pytest
import torch

import oracle
from ravel_em import causal_last_k_lookup, causal_last_k_sources, causal_sum_lookup, sort_order, workloads

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))


def expected_values(payload: torch.Tensor, src: np.ndarray) -> torch.Tensor:
    """Gather on the device from the oracle's source indices (exact copies)."""
    B, T, C, D = payload.shape
    s = torch.from_numpy(src.astype(np.int64)).to(payload.device).view(-1)
    rows = payload.reshape(-1, D).index_select(0, s.clamp_min(0))
    rows = torch.where((s >= 0).view(-1, 1), rows, torch.zeros((), dtype=rows.dtype, device=rows.device))
    return rows.view(B, T, C, src.shape[-1], D)


def check_against_oracle(write, payload, read=None, *, A, k, mask=None):
    vals, vmask, src = causal_last_k_sources(write, payload, read, address_space=A, k=k, write_mask=mask)
    vals2, vmask2 = causal_last_k_lookup(write, payload, read, address_space=A, k=k, write_mask=mask)
    torch.cuda.synchronize()
    osrc = oracle.latest_k_src(write, read, address_space=A, k=k, write_mask=mask)
    gsrc = src.cpu().numpy()
    bad = np.argwhere(gsrc != osrc)
    assert bad.size == 0, f"{len(bad)} source mismatches, first at {bad[:3].tolist()}"
    assert torch.equal(vmask.cpu(), torch.from_numpy(osrc >= 0))
    assert torch.equal(vals, expected_values(payload, osrc))
    assert torch.equal(vals2, vals) and torch.equal(vmask2, vmask)


# --------------------------------------------- reference tests on the GPU --


def test_causal_latest_exact(device):
    case = KATS["latest_exact"]
    addr = torch.tensor(case["write"], device=device)
    payload = torch.tensor(case["payload"], device=device)
    vals, mask = causal_last_k_lookup(addr, payload, address_space=case["address_space"], k=case["k"])
    assert not mask[0, 0, 0, 0]
    assert vals[0, 2, 0, 0, 0].item() == 0.0
    assert vals[0, 4, 0, 0, 0].item() == 2.0
    assert vals[0, 4, 0, 1, 0].item() == 0.0
    _, _, src = causal_last_k_sources(addr, payload, address_space=8, k=2)
    assert src.cpu().tolist() == case["full_src"]


def test_causal_latest_separate_reads_mask_and_payload_gradient(device):
    # tests/test_memory.py:26-58 of the reference, on the device
    write = torch.tensor([[[1], [2], [1], [3], [2], [1]]], device=device)
    read = torch.tensor([[[1], [1], [2], [1], [2], [3]]], device=device)
    write_mask = torch.tensor([[True, True, False, True, True, True]], device=device)
    payload = torch.randn(1, 6, 1, 3, device=device, requires_grad=True)
    actual, actual_mask = causal_last_k_lookup(write, payload, read, address_space=8, k=2, write_mask=write_mask)
    expected = torch.zeros_like(actual)
    expected_mask = torch.zeros_like(actual_mask)
    history = {}
    for t in range(write.shape[1]):
        prior = history.get(int(read[0, t, 0]), [])
        for j, source_t in enumerate(reversed(prior[-2:])):
            expected[0, t, 0, j] = payload[0, source_t, 0]
            expected_mask[0, t, 0, j] = True
        if write_mask[0, t]:
            history.setdefault(int(write[0, t, 0]), []).append(t)
    torch.testing.assert_close(actual, expected)
    assert torch.equal(actual_mask, expected_mask)
    weights = torch.randn_like(actual)
    actual_grad = torch.autograd.grad((actual * weights).sum(), payload, retain_graph=True)[0]
    expected_grad = torch.autograd.grad((expected * weights).sum(), payload)[0]
    torch.testing.assert_close(actual_grad, expected_grad)


def test_bench_forced_repeat(device):
    case = KATS["bench_forced_repeat"]
    torch.manual_seed(case["torch_manual_seed"])
    B, T, C, D, A = case["B"], case["T"], case["C"], case["D"], case["address_space"]
    addr = torch.randint(0, max(1, A - 1), (B, T, C))
    payload = torch.randn(B, T, C, D)
    for t in case["forced_times"]:
        addr[:, t, :] = A - 1
    payload[:, case["forced_times"][0]] = case["forced_value"]
    vals, mask = causal_last_k_lookup(addr.to(device), payload.to(device), address_space=A, k=1)
    t1 = case["forced_times"][1]
    assert torch.equal(vals[:, t1, :, 0, :].cpu(), torch.full((B, C, D), case["forced_value"]))
    assert bool(mask[:, t1, :, 0].all())


# --------------------------------------------------------- random parity --

SMALL = [
    # B, T, C, A, lo, hi, masked, separate reads, k
    (2, 17, 3, 11, None, None, False, False, 1),
    (2, 17, 3, 11, None, None, False, True, 1),
    (3, 40, 2, 5, None, None, True, False, 3),
    (2, 33, 4, 7, None, None, True, True, 4),
    (1, 64, 1, 3, -20, 20, False, True, 5),
    (2, 25, 2, 1, None, None, False, False, 2),
    (2, 9, 2, 4, None, None, False, False, 12),
    (1, 30, 3, 6, 2**31 - 10, 2**31 + 10, False, True, 2),
    (3, 5000, 2, 300, None, None, False, False, 2),  # several sort tiles per segment
    (1, 70000, 1, 2, None, None, True, False, 3),  # long runs across many tiles
    (2, 3000, 3, 1 << 21, None, None, False, True, 2),  # 64-bit packed keys (21+12 bits)
    (2, 257, 5, 100003, None, None, True, True, 1),  # odd sizes, 3 digit passes
    (1, 3000, 40, 1 << 20, None, None, False, False, 2),  # 3 passes x 40 heads: generic sort
    (1, 300, 200, 50, None, None, False, True, 1),  # 200 heads: pack tile over the LDS budget
    (2, 9000, 3, 1 << 17, None, None, True, False, 2),  # masked, 3 passes, 2 look-back sweeps
    (1, 65536, 2, 3, None, None, False, False, 1),  # one-chunk link at its longest segment
    (1, 70000, 2, 50, None, None, False, False, 1),  # link in 16384-step chunks (T > 65536)
    (2, 2048, 4, 5000, None, None, False, False, 8),  # batch-row link at its LDS limit (C*T = 8192)
    (3, 1000, 8, 1024, None, None, False, False, 5),  # batch-row link, ragged time chunks
    (2, 1000, 4, (1 << 23) + 5, None, None, False, False, 3),  # batch-row link over 64-bit keys
    (2, 333, 3, 7, None, None, False, False, 1),  # batch-row link, k = 1, scalar stores
    (3, 1, 2, 5, None, None, False, False, 2),  # one step: every slot missing
    (2, 1, 3, 5, None, None, True, True, 1),  # one step, masked, separate reads
    (1, 4096, 2, 70000, None, None, False, False, 4),  # per-segment LDS sort at its longest, 3 passes
    (1, 4097, 2, 70000, None, None, True, False, 4),  # one step over it: the global sort, masked
    (2, 1025, 3, 1 << 16, None, None, True, True, 3),  # short sort, masked, 2 keys per thread
]


# k == 1 self-links: the link's segment-major sources go through the
# vectorized transpose when the head count is a power of two (up to 16) and
# through the generic one otherwise; the gather then picks its unit from the
# row width and alignment.  Cover several head counts and row widths, ragged
# time tiles, and an unaligned payload view (2-byte units).
LINK1_SHAPES = [
    # B, T, C, D, dtype
    (2, 37, 2, 8, torch.bfloat16),    # 16-byte rows
    (1, 300, 4, 16, torch.float32),   # 64-byte rows
    (3, 129, 8, 64, torch.bfloat16),  # 128-byte rows (the headline shape's rows)
    (2, 50, 16, 128, torch.float32),  # 512-byte rows
    (1, 1000, 16, 4, torch.float32),  # 16-byte rows, 16 heads
    (2, 70, 4, 8, torch.float64),     # 64-byte rows of float64
    (2, 90, 3, 8, torch.bfloat16),    # 3 heads: the generic transpose
    (1, 80, 32, 8, torch.bfloat16),   # 32 heads: the generic transpose
]


@pytest.mark.parametrize("case", LINK1_SHAPES, ids=[str(i) for i in range(len(LINK1_SHAPES))])
def test_latest_1_shapes(device, case):
    B, T, C, D, dtype = case
    g = torch.Generator().manual_seed(T * 7 + C)
    w = torch.randint(0, 40, (B, T, C), generator=g)
    p = torch.randn(B, T, C, D, generator=g).to(dtype)
    check_against_oracle(w.to(device), p.to(device), A=40, k=1)


# Self-links with k == 1, no mask, 32-bit keys and two or more digit passes
# (A > 256) are linked inside the sort's last pass: cover one and many tiles
# per segment, three passes, long runs of one hot address, and the sources.
FUSED_LINK = [
    # B, T, C, A, hot fraction
    (2, 300, 3, 257, 0.0),
    (2, 5000, 4, 1000, 0.0),
    (1, 65536, 2, 65536, 0.0),
    (1, 30000, 3, 1 << 17, 0.0),   # 3 passes (17 + 15 bits)
    (2, 20000, 2, 4096, 0.9),      # one hot address: runs across all tiles
    (1, 9000, 16, 70000, 0.5),
]


@pytest.mark.parametrize("case", FUSED_LINK, ids=[str(i) for i in range(len(FUSED_LINK))])
def test_latest_1_link_in_sort(device, case):
    B, T, C, A, hot = case
    g = torch.Generator().manual_seed(B * 131 + T + C)
    w = torch.randint(0, A, (B, T, C), generator=g)
    if hot > 0:
        w = torch.where(torch.rand(B, T, C, generator=g) < hot, torch.full_like(w, 7), w)
    p = torch.randn(B, T, C, 8, generator=g).to(torch.bfloat16)
    check_against_oracle(w.to(device), p.to(device), A=A, k=1)


def test_latest_1_unaligned_payload_view(device):
    g = torch.Generator().manual_seed(5)
    w = torch.randint(0, 9, (2, 33, 4), generator=g)
    base = torch.randn(2 * 33 * 4 * 8 + 1, generator=g).to(torch.bfloat16).to(device)
    p = base[1:].view(2, 33, 4, 8)  # 2-byte offset: 16-byte rows, unaligned on the device
    assert p.data_ptr() % 16 != 0
    check_against_oracle(w.to(device), p, A=9, k=1)


@pytest.mark.parametrize("case", SMALL, ids=[str(i) for i in range(len(SMALL))])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_latest_k_parity(device, case, dtype):
    B, T, C, A, lo, hi, masked, sep, k = case
    g = torch.Generator().manual_seed(B * 1000 + T + k)
    lo = 0 if lo is None else lo
    hi = A if hi is None else hi
    w = torch.randint(lo, hi, (B, T, C), generator=g)
    r = torch.randint(lo, hi, (B, T, C), generator=g) if sep else None
    m = (torch.rand(B, T, generator=g) < 0.6) if masked else None
    p = torch.randn(B, T, C, 5, generator=g).to(dtype)
    check_against_oracle(w.to(device), p.to(device), None if r is None else r.to(device),
                         A=A, k=k, mask=None if m is None else m.to(device))


@pytest.mark.parametrize("addr_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("D,dtype", [(1, torch.float32), (3, torch.float16), (8, torch.bfloat16), (33, torch.float64)])
def test_latest_k_dtypes_and_row_widths(device, addr_dtype, D, dtype):
    g = torch.Generator().manual_seed(D)
    B, T, C, A = 2, 300, 3, 17
    w = torch.randint(0, A, (B, T, C), generator=g).to(addr_dtype)
    r = torch.randint(0, A, (B, T, C), generator=g).to(addr_dtype)
    p = torch.randn(B, T, C, D, generator=g).to(dtype)
    check_against_oracle(w.to(device), p.to(device), r.to(device), A=A, k=3)
    check_against_oracle(w.to(device), p.to(device), None, A=A, k=2)


def test_sort_order_bit_exact(device):
    for (B, T, C, A, masked) in [(2, 17, 3, 11, False), (3, 40, 2, 5, True), (2, 3000, 3, 1 << 21, False),
                                 (2, 257, 5, 100003, True), (4, 4096, 8, 4096, False)]:
        g = torch.Generator().manual_seed(T)
        w = torch.randint(-A, 2 * A, (B, T, C), generator=g)
        m = (torch.rand(B, T, generator=g) < 0.5) if masked else None
        keys, order = sort_order(w.to(device), address_space=A, write_mask=None if m is None else m.to(device))
        okeys, oorder = oracle.sort_order(w, address_space=A, write_mask=m)
        assert keys.dtype == (torch.int32 if oracle.key_bits(B, T, C, A) == 32 else torch.int64)
        assert np.array_equal(keys.cpu().numpy().astype(np.int64), okeys)
        assert np.array_equal(order.cpu().numpy(), oorder)


def test_all_writes_masked_gives_zeros(device):
    w = torch.randint(0, 5, (2, 8, 3), device=device)
    p = torch.randn(2, 8, 3, 4, device=device)
    m = torch.zeros(2, 8, dtype=torch.bool, device=device)
    vals, mask = causal_last_k_lookup(w, p, address_space=5, k=2, write_mask=m)
    assert not mask.any() and not vals.any()
    keys, order = sort_order(w, address_space=5, write_mask=m)
    assert keys.numel() == 0 and order.numel() == 0


def test_empty_tape(device):
    w = torch.zeros(0, 8, 3, dtype=torch.long, device=device)
    p = torch.zeros(0, 8, 3, 4, device=device)
    vals, mask = causal_last_k_lookup(w, p, address_space=5, k=2)
    assert vals.shape == (0, 8, 3, 2, 4) and mask.shape == (0, 8, 3, 2)


# ---------------------------------------------- benchmark configurations --


@pytest.mark.parametrize("name", ["cfg1", "cfg1b", "cfg2_f32", "cfg2_bf16", "cfg3", "cfg4", "cfg4_adv"])
def test_baseline_config_parity(device, name):
    print(f"[parity] {name}", flush=True)
    if name == "cfg1":
        w = workloads.cfg1(device)
    elif name == "cfg1b":
        w = workloads.cfg1(device, variant="1b")
    elif name == "cfg2_f32":
        w = workloads.cfg2(device, torch.float32)
    elif name == "cfg2_bf16":
        w = workloads.cfg2(device, torch.bfloat16)
    elif name == "cfg3":
        w = workloads.cfg3(device)
    elif name == "cfg4":
        w = workloads.cfg4(device)
    else:
        w = workloads.cfg4(device, adversarial=True)
    check_against_oracle(w.write, w.payload, w.read, A=w.address_space, k=w.k)
    if name in ("cfg2_f32", "cfg4"):
        keys, order = sort_order(w.write, address_space=w.address_space)
        okeys, oorder = oracle.sort_order(w.write, address_space=w.address_space)
        assert np.array_equal(keys.cpu().numpy().astype(np.int64), okeys)
        assert np.array_equal(order.cpu().numpy(), oorder)


def test_resolve_and_gather_stage_entry_points(device):
    """ravel_em_latest_k_resolve + ravel_em_gather_rows reproduce the fused call."""
    from ravel_em import _native as nat

    lib = nat.library()
    for sep, masked in [(False, False), (True, False), (False, True)]:
        g = torch.Generator().manual_seed(int(sep) * 2 + int(masked))
        B, T, C, A, D, k = 2, 700, 3, 23, 12, 3
        w = torch.randint(0, A, (B, T, C), generator=g).to(device)
        r = torch.randint(0, A, (B, T, C), generator=g).to(device) if sep else None
        m = (torch.rand(B, T, generator=g) < 0.5).to(device) if masked else None
        p = torch.randn(B, T, C, D, generator=g).to(device, torch.bfloat16)
        src = torch.empty(B, T, C, k, dtype=torch.int32, device=device)
        ws = nat.workspace(lib.ravel_em_latest_k_resolve_workspace(B, T, C, A, k, int(sep), int(masked)), device)
        stream = torch.cuda.current_stream(device).cuda_stream
        nat.check(lib.ravel_em_latest_k_resolve(w.data_ptr(), None if r is None else r.data_ptr(), nat.INT64,
                                                None if m is None else m.data_ptr(), B, T, C, A, k,
                                                src.data_ptr(), ws.data_ptr(), ws.numel(), stream))
        vals = torch.empty(B, T, C, k, D, dtype=torch.bfloat16, device=device)
        mask = torch.empty(B, T, C, k, dtype=torch.bool, device=device)
        nat.check(lib.ravel_em_gather_rows(p.data_ptr(), B * T * C, D * 2, src.data_ptr(), B * T * C * k,
                                           vals.data_ptr(), mask.data_ptr(), stream))
        want_v, want_m, want_s = causal_last_k_sources(w, p, r, address_space=A, k=k, write_mask=m)
        assert torch.equal(src, want_s) and torch.equal(vals, want_v) and torch.equal(mask, want_m)
        osrc = oracle.latest_k_src(w, r, address_space=A, k=k, write_mask=m)
        assert np.array_equal(src.cpu().numpy(), osrc)


def test_stage_timer_reports_each_stage(device):
    import ctypes

    from ravel_em import _native as nat

    lib = nat.library()
    # a tape longer than 4096 steps, so the global sort, the resolve and the gather all run
    w = torch.randint(0, 50, (2, 5000, 4), device=device)
    p = torch.randn(2, 5000, 4, 8, device=device)
    nat.check(lib.ravel_em_profile_start())
    for _ in range(3):
        causal_last_k_lookup(w, p, address_space=50, k=2)
    ms = (ctypes.c_double * 5)()
    calls = (ctypes.c_int * 5)()
    nat.check(lib.ravel_em_profile_stop(ms, calls, 5))
    assert list(calls)[:3] == [3, 3, 3] and all(ms[i] > 0 for i in range(3))
    causal_last_k_lookup(w, p, address_space=50, k=2)  # timer off again: nothing recorded
    nat.check(lib.ravel_em_profile_stop(ms, calls, 5))
    assert list(calls) == [0] * 5


@pytest.mark.parametrize("shape", [(4, 65536, 16, 65536, False), (2, 5000, 3, 300, True), (3, 2000, 8, 1 << 20, False),
                                   (1, 70000, 2, 3, True)])
def test_fused_and_generic_sorts_agree(device, shape):
    from ravel_em import _native as nat

    B, T, C, A, masked = shape
    g = torch.Generator().manual_seed(T)
    w = torch.randint(0, A, (B, T, C), generator=g).to(device)
    m = (torch.rand(B, T, generator=g) < 0.5).to(device) if masked else None
    lib = nat.library()
    outs = []
    for path in (0, 1):
        nat.check(lib.ravel_em_set_sort_path(path))
        try:
            outs.append(sort_order(w, address_space=A, write_mask=m))
        finally:
            nat.check(lib.ravel_em_set_sort_path(0))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    if B * T * C <= 1 << 20:
        okeys, oorder = oracle.sort_order(w, address_space=A, write_mask=m)
        assert np.array_equal(outs[0][1].cpu().numpy(), oorder)


# ------------------------------------------ buckets that span many pieces --
# With two 8-bit address digits, k = 1 and reads = writes, the link groups each
# stream's records by the high address digit (a bucket): one wave walks a
# bucket of up to 1024 records, a block of 8 waves a bucket of up to 8192, and
# a larger bucket goes in parts of 8192 records to separate blocks, whose
# last one to finish carries each low digit's last time from part to part.
# These cases put many records into few buckets, at those boundaries, with
# digits missing from whole parts, and several large buckets per stream.

def _hot_case(name, T, A, C=2, B=2):
    g = torch.Generator().manual_seed(T + A + len(name))
    if name == "one_address":
        w = torch.full((B, T, C), 7, dtype=torch.long)
    elif name == "two_digits_one_bucket":  # same high digit, low digits 3 and 200
        w = torch.where(torch.rand(B, T, C, generator=g) < 0.5, 3, 200)
    elif name == "rare_digit":  # a low digit seen once early and once late in a hot bucket
        w = torch.full((B, T, C), 5, dtype=torch.long)
        w[:, 3, :] = 9
        w[:, T - 2, :] = 9
    elif name == "skewed":  # 90% of records at one address, the rest spread
        w = torch.randint(0, A, (B, T, C), generator=g)
        w = torch.where(torch.rand(B, T, C, generator=g) < 0.9, torch.zeros_like(w), w)
    elif name == "few_buckets":  # A = 512: two buckets of ~T/2 records
        w = torch.randint(0, A, (B, T, C), generator=g)
    elif name == "mixed_modes":  # head 0 one hot address, head 1 uniform
        w = torch.randint(0, A, (B, T, C), generator=g)
        w[:, :, 0] = 11
    elif name == "two_hot_groups":  # hot buckets 0 and 200 (different owner blocks), some spread
        w = torch.where(torch.rand(B, T, C, generator=g) < 0.5, 7, 200 * 256 + 9)
        r = torch.randint(0, A, (B, T, C), generator=g)
        w = torch.where(torch.rand(B, T, C, generator=g) < 0.05, r, w)
    else:
        raise ValueError(name)
    return w


HOT = [("one_address", 1024, 4096), ("one_address", 1025, 4096), ("one_address", 2048, 4096),
       ("one_address", 8192, 4096), ("one_address", 8193, 4096), ("one_address", 16385, 4096),
       ("one_address", 70000 // 2, 65536), ("two_digits_one_bucket", 5000, 256 * 256),
       ("rare_digit", 20000, 4096), ("skewed", 30000, 65536), ("few_buckets", 40000, 512),
       ("few_buckets", 3000, 300), ("mixed_modes", 30000, 65536),
       ("two_hot_groups", 40000, 65536)]


@pytest.mark.parametrize("case", HOT, ids=[f"{n}-{T}-{A}" for n, T, A in HOT])
def test_multi_piece_buckets(device, case):
    name, T, A = case
    print(f"[hot buckets] {name} T={T} A={A}", flush=True)
    w = _hot_case(name, T, A)
    p = torch.randn(*w.shape, 8).to(torch.bfloat16)
    check_against_oracle(w.to(device), p.to(device), A=A, k=1)


@pytest.mark.parametrize("case", HOT, ids=[f"{n}-{T}-{A}" for n, T, A in HOT])
def test_sort_order_hot_buckets(device, case):
    """The full sort of the same tapes: with two address digits it scatters by
    the high digit, then sorts each bucket by the low digit (a wave, a block,
    or the parts of a large bucket, placed from the parts' histograms); the
    keys and the order are the oracle's, and so is the segmented sum walked
    over them."""
    name, T, A = case
    print(f"[hot sort] {name} T={T} A={A}", flush=True)
    w = _hot_case(name, T, A)
    keys, order = sort_order(w.to(device), address_space=A)
    okeys, oorder = oracle.sort_order(w, address_space=A)
    assert np.array_equal(keys.cpu().numpy().astype(np.int64), okeys)
    assert np.array_equal(order.cpu().numpy(), oorder)
    p = torch.randint(-3, 4, (*w.shape, 8)).float()  # small integers: exact sums
    out, mask = causal_sum_lookup(w.to(device), p.to(device), address_space=A)
    truth, tmask = oracle.seg_sum(w, p, address_space=A)
    assert torch.equal(out.cpu().double(), truth) and torch.equal(mask.cpu(), tmask)


def test_eager_fast_path_matches_the_registered_op(device):
    """The public calls without autograd run the ops' bodies directly; the
    registered ops (the autograd and torch.compile route) give the same bits."""
    from ravel_em import _ops

    g = torch.Generator().manual_seed(21)
    w = torch.randint(0, 40, (2, 300, 3), generator=g).to(device)
    p = torch.randn(2, 300, 3, 8, generator=g).to(device)
    vals, mask = causal_last_k_lookup(w, p, address_space=40, k=3)
    v2, m2, _ = _ops.latest_k(w, p, None, None, 40, 3, False)
    assert torch.equal(vals, v2) and torch.equal(mask, m2)
    s, sm = causal_sum_lookup(w, p, address_space=40)
    s2, sm2 = _ops.seg_sum(w, p, None, None, 40)
    assert torch.equal(s, s2) and torch.equal(sm, sm2)


def test_launch_stream_is_torch_current_stream(device):
    from ravel_em import _native as nat

    t = torch.zeros(4, device=device)
    assert nat.stream_of(t) == torch.cuda.current_stream(device).cuda_stream
    side = torch.cuda.Stream(device)
    with torch.cuda.stream(side):
        assert nat.stream_of(t) == side.cuda_stream
        w = torch.randint(0, 9, (1, 64, 2), device=device)
        p = torch.randn(1, 64, 2, 4, device=device)
        vals, mask = causal_last_k_lookup(w, p, address_space=9)
    side.synchronize()
    ref, rmask = causal_last_k_lookup(w, p, address_space=9)
    assert torch.equal(vals, ref) and torch.equal(mask, rmask)
