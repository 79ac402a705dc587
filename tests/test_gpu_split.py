"""Tapes split by batch rows (the entry points' row ranges).

A call whose slots B*T*C*k (records, for the sums, the prefill and the
addresses) pass 2^26 runs as consecutive ranges of whole batch rows of at most
2^26 slots.  Two kinds of check:

* small tapes with the range size lowered by ravel_em_set_split_slots, so every
  entry point splits at sizes the oracle checks: latest-k values, masks,
  sources, the prefill and produced addresses are bit-identical to the unsplit
  call and to the oracle; sums and gradients are within the accumulation
  bounds of tests/test_gpu_sum.py (the split moves part boundaries, so the
  summation order may change);
* full-size tapes past 2^31, which the kernels' 32-bit indices could not take
  in one piece: latest-k with k = 4 over 2^29 records (2^31 slots, int32
  sources still valid) and latest-1 and the segmented sum over 2^31 records;
  rows at range boundaries and the ends are checked against the oracle run on
  those rows alone (each row is an independent tape).
"""
import contextlib

import numpy as np
import pytest
import torch

import oracle
from ravel_em import (LayerAddresses, RavelLayerCache, causal_last_k_lookup,
                      causal_last_k_sources, causal_sum_lookup, fused_latest1_linear,
                      literal_addresses_from_tokens, sort_order)
from ravel_em import _native as nat
from test_gpu_sum import compare_sums, oracle_terms, sum_depth

pytestmark = pytest.mark.gpu


@contextlib.contextmanager
def split_slots(n):
    lib = nat.library()
    nat.check(lib.ravel_em_set_split_slots(int(n)))
    try:
        yield
    finally:
        nat.check(lib.ravel_em_set_split_slots(0))


def tape(device, B, T, C, A, *, read=False, mask=False, D=5, dtype=torch.float32, seed=0):
    g = torch.Generator().manual_seed(seed)
    w = torch.randint(0, A, (B, T, C), generator=g)
    r = torch.randint(0, A, (B, T, C), generator=g) if read else None
    m = torch.rand(B, T, generator=g) < 0.7 if mask else None
    p = torch.randn(B, T, C, D, generator=g).to(dtype)
    dev = lambda x: None if x is None else x.to(device)
    return dev(w), dev(p), dev(r), dev(m), (w, p, r, m)


LK_CASES = [
    # B, T, C, A, k, separate reads, masked, dtype
    (5, 37, 3, 11, 1, False, False, torch.float32),
    (5, 37, 3, 11, 4, False, False, torch.bfloat16),
    (5, 300, 2, 7, 2, True, False, torch.float32),
    (4, 50, 3, 5, 3, False, True, torch.float32),
    (3, 5000, 2, 300, 1, False, False, torch.bfloat16),
    (3, 5000, 2, 300, 2, True, True, torch.bfloat16),
    (2, 70000, 1, 3, 1, False, False, torch.float32),
]


@pytest.mark.parametrize("B,T,C,A,k,sep,masked,dtype", LK_CASES)
@pytest.mark.parametrize("rows", [1, 2])
def test_latest_k_split_matches_unsplit_and_oracle(device, B, T, C, A, k, sep, masked, dtype, rows):
    w, p, r, m, host = tape(device, B, T, C, A, read=sep, mask=masked, dtype=dtype)
    print(f"[split] latest-k B={B} T={T} C={C} A={A} k={k} sep={sep} mask={masked} rows={rows}",
          flush=True)
    base = causal_last_k_sources(w, p, r, address_space=A, k=k, write_mask=m)
    with split_slots(rows * T * C * k):
        got = causal_last_k_sources(w, p, r, address_space=A, k=k, write_mask=m)
        vals, vmask = causal_last_k_lookup(w, p, r, address_space=A, k=k, write_mask=m)
    for a, b in zip(got, base):
        assert torch.equal(a, b)
    assert torch.equal(vals, base[0]) and torch.equal(vmask, base[1])
    want = oracle.latest_k_src(host[0], host[2], address_space=A, k=k, write_mask=host[3])
    assert np.array_equal(got[2].cpu().numpy().astype(np.int64), want)


SUM_CASES = [
    # B, T, C, A, separate reads, masked, D, dtype
    (5, 37, 3, 11, False, False, 8, torch.float32),
    (4, 300, 2, 7, True, False, 64, torch.bfloat16),
    (4, 50, 3, 5, False, True, 16, torch.float32),
    (3, 5000, 2, 300, False, False, 64, torch.bfloat16),
    (2, 70000, 1, 3, True, True, 8, torch.float32),
]


@pytest.mark.parametrize("B,T,C,A,sep,masked,D,dtype", SUM_CASES)
def test_seg_sum_split_within_bound(device, B, T, C, A, sep, masked, D, dtype):
    w, p, r, m, host = tape(device, B, T, C, A, read=sep, mask=masked, D=D, dtype=dtype, seed=3)
    print(f"[split] sum B={B} T={T} C={C} A={A} D={D} {dtype} sep={sep} mask={masked}", flush=True)
    with split_slots(T * C):  # one row per range
        out, omask = causal_sum_lookup(w, p, r, address_space=A, write_mask=m)
    hw, hp, hr, hm = host
    truth, tmask = oracle.seg_sum(hw, hp, hr, address_space=A, write_mask=hm)
    scale, _ = oracle.seg_sum(hw, hp.abs(), hr, address_space=A, write_mask=hm)
    n = oracle_terms(hw, hr, A, hm, (B, T, C))
    assert torch.equal(omask.cpu(), tmask)
    compare_sums(out.cpu(), truth, scale, n, dtype, sum_depth(T, D, dtype), "split rows")


@pytest.mark.parametrize("sep,masked", [(False, False), (True, False), (False, True)])
def test_gradients_split(device, sep, masked):
    B, T, C, A, k, D = 5, 300, 2, 7, 3, 8
    w, p, r, m, host = tape(device, B, T, C, A, read=sep, mask=masked, D=D, seed=4)
    print(f"[split] gradients sep={sep} mask={masked}", flush=True)
    gv = torch.randn(B, T, C, k, D, generator=torch.Generator().manual_seed(9)).to(device)
    gs = torch.randn(B, T, C, D, generator=torch.Generator().manual_seed(10)).to(device)

    def grads():
        x = p.clone().requires_grad_(True)
        vals, _ = causal_last_k_lookup(w, x, r, address_space=A, k=k, write_mask=m)
        (g_lk,) = torch.autograd.grad(vals, x, gv)
        sums, _ = causal_sum_lookup(w, x, r, address_space=A, write_mask=m)
        (g_sum,) = torch.autograd.grad(sums, x, gs)
        return g_lk, g_sum

    # the forward calls split; the backward nodes run on autograd's worker
    # thread, outside this thread's range size (test_backward_entry_points_split
    # splits those)
    with split_slots(2 * T * C * k):  # latest-k: two rows per range; sums: six
        g_lk, g_sum = grads()
    with split_slots(T * C):  # one row per range for both
        g_lk1, g_sum1 = grads()
    # latest-k: grad_payload[s] = sum of the slots that copied s, in fp64
    src = oracle.latest_k_src(host[0], host[2], address_space=A, k=k, write_mask=host[3])
    want = torch.zeros(B * T * C, D, dtype=torch.float64)
    sel = src.reshape(-1) >= 0
    want.index_add_(0, torch.from_numpy(src.reshape(-1)[sel]),
                    gv.cpu().double().reshape(-1, D)[torch.from_numpy(sel)])
    for g in (g_lk, g_lk1):
        assert torch.allclose(g.cpu().double().reshape(-1, D), want, rtol=1e-5, atol=1e-5)
    truth, _, _ = oracle.seg_sum_grad(host[0], gs.cpu().double(), host[2], address_space=A,
                                   write_mask=host[3])
    for g in (g_sum, g_sum1):
        assert torch.allclose(g.cpu().double(), truth, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("sep,masked", [(False, False), (True, False), (False, True)])
def test_backward_entry_points_split(device, sep, masked):
    """The two backward entry points split into ranges.  The range size is set
    per thread and autograd runs backward nodes on its own worker thread, so
    test_gradients_split splits the forward calls only; here the backward C
    entry points are called on this thread, unsplit and in one-row ranges, and
    checked against each other and the oracle (latest-k: the sorted form, whose
    sources are made range-local and back; sums: the reverse walk)."""
    B, T, C, A, k, D = 5, 300, 2, 7, 3, 8
    w, p, r, m, host = tape(device, B, T, C, A, read=sep, mask=masked, D=D, seed=14)
    print(f"[split] backward entry points sep={sep} mask={masked}", flush=True)
    lib = nat.library()
    code = nat.FLOAT32
    stream = nat.stream_of(p)
    _, _, src = causal_last_k_sources(w, p, r, address_space=A, k=k, write_mask=m)
    gv = torch.randn(B, T, C, k, D, generator=torch.Generator().manual_seed(15)).to(device)
    gs = torch.randn(B, T, C, D, generator=torch.Generator().manual_seed(16)).to(device)

    def lk_bwd():
        out = torch.empty(B, T, C, D, device=device)
        ws = nat.workspace(lib.ravel_em_latest_k_bwd_workspace(B, T, C, D, k, code, 0), device)
        nat.check(lib.ravel_em_latest_k_bwd(src.data_ptr(), gv.data_ptr(), code, B, T, C, D, k, 0,
                                            out.data_ptr(), ws.data_ptr(), ws.numel(), stream))
        assert nat.status_word(ws) == 0
        return out

    def sum_bwd():
        out = torch.empty(B, T, C, D, device=device)
        ws = nat.workspace(lib.ravel_em_seg_sum_bwd_workspace(B, T, C, D, A, int(sep), int(masked),
                                                              code), device)
        nat.check(lib.ravel_em_seg_sum_bwd(w.data_ptr(), nat.ptr(r), nat.INT64, nat.ptr(m),
                                           gs.data_ptr(), code, B, T, C, D, A, out.data_ptr(),
                                           ws.data_ptr(), ws.numel(), stream))
        assert nat.status_word(ws) == 0
        return out

    base_lk, base_sum = lk_bwd(), sum_bwd()
    with split_slots(T * C * k):  # one batch row per range
        lk1 = lk_bwd()
    with split_slots(T * C):
        sum1 = sum_bwd()
    # each source's slots lie in its own row, so the slot-order sums are unchanged
    assert torch.equal(lk1, base_lk)
    want = torch.zeros(B * T * C, D, dtype=torch.float64)
    osrc = oracle.latest_k_src(host[0], host[2], address_space=A, k=k, write_mask=host[3])
    sel = osrc.reshape(-1) >= 0
    want.index_add_(0, torch.from_numpy(osrc.reshape(-1)[sel]),
                    gv.cpu().double().reshape(-1, D)[torch.from_numpy(sel)])
    assert torch.allclose(lk1.cpu().double().reshape(-1, D), want, rtol=1e-5, atol=1e-5)
    truth, _, _ = oracle.seg_sum_grad(host[0], gs.cpu().double(), host[2], address_space=A,
                                      write_mask=host[3])
    for g in (base_sum, sum1):
        assert torch.allclose(g.cpu().double(), truth, rtol=1e-5, atol=1e-5)


def test_fused_linear_split(device):
    B, T, C, A, P, M = 5, 300, 2, 7, 8, 24
    w, p, r, _, _ = tape(device, B, T, C, A, read=True, D=P, seed=6)
    wt = torch.randn(M, C * P, generator=torch.Generator().manual_seed(2)).to(device)
    print("[split] fused latest-1 linear", flush=True)
    x = p.clone().requires_grad_(True)
    base = fused_latest1_linear(w, x, r, wt, address_space=A)
    gb = torch.autograd.grad(base.sum(), x)[0]
    with split_slots(2 * T * C):
        x2 = p.clone().requires_grad_(True)
        got = fused_latest1_linear(w, x2, r, wt, address_space=A)
        g2 = torch.autograd.grad(got.sum(), x2)[0]
        plain = fused_latest1_linear(w, p, r, wt, address_space=A)
    assert torch.allclose(got, base, rtol=1e-5, atol=1e-5)
    assert torch.allclose(plain, base, rtol=1e-5, atol=1e-5)
    assert torch.allclose(g2, gb, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("B,T,C,A,masked", [(5, 37, 3, 11, False), (5, 37, 3, 11, True),
                                             (3, 5000, 2, 300, True), (4, 3000, 3, 1 << 20, False)])
def test_sort_order_split(device, B, T, C, A, masked):
    w, _, _, m, host = tape(device, B, T, C, A, mask=masked, seed=11)
    print(f"[split] sort order B={B} T={T} C={C} A={A} mask={masked}", flush=True)
    base = sort_order(w, address_space=A, write_mask=m)
    with split_slots(2 * T * C):
        got = sort_order(w, address_space=A, write_mask=m)
    assert torch.equal(got[0], base[0]) and torch.equal(got[1], base[1])
    keys, order = oracle.sort_order(host[0], address_space=A, write_mask=host[3])
    assert np.array_equal(got[0].cpu().numpy().astype(np.int64), keys)
    assert np.array_equal(got[1].cpu().numpy(), order)


@pytest.mark.parametrize("masked", [False, True])
def test_prefill_split(device, masked):
    B, T, C, A, k, D = 6, 200, 3, 13, 4, 8
    w, p, _, m, host = tape(device, B, T, C, A, mask=masked, D=D, dtype=torch.bfloat16, seed=8)
    print(f"[split] prefill mask={masked}", flush=True)
    base = RavelLayerCache.prefill(w, p, address_space=A, k=k, write_mask=m)
    with split_slots(2 * T * C):
        got = RavelLayerCache.prefill(w, p, address_space=A, k=k, write_mask=m)
    assert torch.equal(got.values, base.values) and torch.equal(got.filled, base.filled)
    vals, filled = oracle.cache_prefill(host[0], host[1], address_space=A, k=k, write_mask=host[3])
    assert torch.equal(got.filled.cpu(), filled)
    assert torch.equal(got.values.cpu()[filled], vals[filled])


def test_produced_addresses_split(device):
    B, T, n_lit, H, Q, S, A, k = 5, 120, 3, 2, 2, 8, 61, 2
    g = torch.Generator().manual_seed(12)
    toks = torch.randint(0, 40, (B, T), generator=g).to(device)
    n = H * Q * S
    packed = torch.randn(B, T, 4 + 2 * n, generator=g).to(torch.bfloat16).to(device)
    src = LayerAddresses(toks, n_lit, 257, packed[..., 4:4 + n], packed[..., 4 + n:], H, Q, S)
    p = torch.randn(B, T, n_lit + H, 8, generator=g).to(device)
    print("[split] produced addresses", flush=True)
    base = causal_last_k_sources(src, p, address_space=A, k=k)
    base_lit = literal_addresses_from_tokens(toks, address_space=A, n_heads=n_lit, bos_token_id=257)
    with split_slots(2 * T * (n_lit + H) * k):
        got = causal_last_k_sources(src, p, address_space=A, k=k)
        sums = causal_sum_lookup(src, p, address_space=A)
    with split_slots(T * n_lit):
        lit = literal_addresses_from_tokens(toks, address_space=A, n_heads=n_lit, bos_token_id=257)
    for a, b in zip(got, base):
        assert torch.equal(a, b)
    assert torch.equal(lit, base_lit)
    wa, ra = src.materialize(address_space=A)
    want = causal_sum_lookup(wa, p, ra, address_space=A)
    assert torch.equal(sums[1], want[1])
    assert torch.allclose(sums[0], want[0], rtol=1e-5, atol=1e-5)


def test_gather_rows_split(device):
    lib = nat.library()
    rows = torch.randn(50, 3, device=device)
    src = torch.randint(-1, 50, (1000,), dtype=torch.int32, device=device)
    print("[split] gather rows", flush=True)

    def gather():
        out = torch.empty(1000, 3, device=device)
        mask = torch.empty(1000, dtype=torch.bool, device=device)
        nat.check(lib.ravel_em_gather_rows(rows.data_ptr(), 50, 12, src.data_ptr(), 1000,
                                           out.data_ptr(), mask.data_ptr(), nat.stream_of(rows)))
        return out, mask

    base = gather()
    with split_slots(97):
        got = gather()
    assert torch.equal(got[0], base[0]) and torch.equal(got[1], base[1])
    valid = src.long() >= 0
    assert torch.equal(base[1], valid)
    assert torch.equal(base[0][valid], rows[src.long()[valid]])


# ------------------------------------------------------ past 2^31 --


def _row_sources(w_row, A, k):
    """Oracle sources of one batch row alone (record ids local to the row)."""
    return oracle.latest_k_src(w_row, address_space=A, k=k)


def test_latest_k_past_2p31_slots(device):
    # 8192 rows x 32768 steps x 2 heads = 2^29 records, k = 4: 2^31 slots,
    # run as 32 ranges of 256 rows; int32 sources still valid
    B, T, C, A, k = 8192, 32768, 2, 4096, 4
    N = B * T * C
    print(f"[split] latest-k past 2^31 slots B={B} T={T} C={C} k={k}", flush=True)
    gen = torch.Generator(device=device).manual_seed(21)
    w = torch.randint(0, A, (B, T, C), generator=gen, device=device, dtype=torch.int32)
    p = torch.randn(B, T, C, 1, generator=gen, device=device)
    vals, vmask, src = causal_last_k_sources(w, p, address_space=A, k=k)
    torch.cuda.synchronize()
    assert vals.shape == (B, T, C, k, 1) and src.shape == (B, T, C, k)
    flat_p = p.reshape(-1)
    for b in (0, 255, 256, 4097, 8191):
        want = _row_sources(w[b:b + 1].cpu(), A, k).reshape(T, C, k)
        got = src[b].cpu().numpy().astype(np.int64)
        loc = np.where(got >= 0, got - b * T * C, -1)
        assert np.array_equal(loc, want), f"row {b}"
        s = src[b].long()
        ok = s >= 0
        assert torch.equal(vmask[b], ok)
        assert torch.equal(vals[b, ..., 0][ok], flat_p[s[ok]])
        assert not vals[b, ..., 0][~ok].any()
    assert int(src.max()) < N


def test_latest1_and_sum_past_2p31_records(device):
    # 32768 rows x 65536 steps = 2^31 records: 32 ranges of 1024 rows
    B, T, C, A = 32768, 65536, 1, 4096
    print(f"[split] latest-1 and sum past 2^31 records B={B} T={T}", flush=True)
    gen = torch.Generator(device=device).manual_seed(22)
    w = torch.randint(0, A, (B, T, C), generator=gen, device=device, dtype=torch.int32)
    p = torch.randn(B, T, C, 1, generator=gen, device=device)
    check_rows = (0, 1023, 1024, 32767)
    host_w = {b: w[b:b + 1].cpu() for b in check_rows}
    host_p = {b: p[b:b + 1].cpu() for b in check_rows}
    vals, vmask = causal_last_k_lookup(w, p, address_space=A, k=1)
    torch.cuda.synchronize()
    for b in check_rows:
        want = _row_sources(host_w[b], A, 1).reshape(T, C)
        ok = torch.from_numpy(want >= 0)
        assert torch.equal(vmask[b, :, :, 0].cpu(), ok), f"row {b}"
        got = vals[b, :, :, 0, 0].cpu()
        exp = host_p[b].reshape(-1)[torch.from_numpy(np.maximum(want, 0)).reshape(-1)].reshape(T, C)
        assert torch.equal(got[ok], exp[ok]) and not got[~ok].any(), f"row {b}"
    del vals, vmask
    out, omask = causal_sum_lookup(w, p, address_space=A)
    torch.cuda.synchronize()
    for b in check_rows:
        truth, tmask = oracle.seg_sum(host_w[b], host_p[b], address_space=A)
        scale, _ = oracle.seg_sum(host_w[b], host_p[b].abs(), address_space=A)
        n = oracle_terms(host_w[b], None, A, None, (1, T, C))
        assert torch.equal(omask[b:b + 1].cpu(), tmask), f"row {b}"
        compare_sums(out[b:b + 1].cpu(), truth, scale, n, torch.float32,
                     sum_depth(T, 1, torch.float32), f"row {b} of 2^31 records")
    del out, omask
    keys, order = sort_order(w, address_space=A)
    torch.cuda.synchronize()
    assert keys.dtype == torch.int64 and keys.numel() == B * T * C
    for b in check_rows:
        wk, wo = oracle.sort_order(host_w[b], address_space=A)
        sl = slice(b * T * C, (b + 1) * T * C)
        # row b alone: its keys without the row's base, its order from 0
        assert np.array_equal(keys[sl].cpu().numpy() - b * C * A * (T + 1), wk), f"row {b}"
        assert np.array_equal(order[sl].cpu().numpy() - b * T * C, wo), f"row {b}"


@pytest.mark.parametrize("sep,masked", [(False, False), (True, True)])
def test_static_entry_split(device, sep, masked):
    """The entry point without a workspace runs split calls out of its static
    scratch: same results as the workspace call, status word zero (folded over
    the ranges)."""
    lib = nat.library()
    B, T, C, A, k, D = 5, 300, 2, 7, 2, 8
    w, p, r, m, _ = tape(device, B, T, C, A, read=sep, mask=masked, D=D, seed=13)
    print(f"[split] static entry sep={sep} mask={masked}", flush=True)
    base = causal_last_k_sources(w, p, r, address_space=A, k=k, write_mask=m)
    vals = torch.full((B, T, C, k, D), 7.0, device=device)
    mask = torch.ones(B, T, C, k, dtype=torch.bool, device=device)
    src = torch.full((B, T, C, k), -5, dtype=torch.int32, device=device)
    status = torch.full((1,), 0xFFFF, dtype=torch.int32, device=device)
    with split_slots(2 * T * C * k):
        nat.check(lib.ravel_em_latest_k_fwd_static(
            nat.ptr(w), nat.ptr(r), nat.addr_code(w.dtype), nat.ptr(m), nat.ptr(p),
            nat.payload_code(p.dtype), B, T, C, D, A, k, nat.ptr(vals), nat.ptr(mask), nat.ptr(src),
            nat.ptr(status), nat.stream_of(p)))
    torch.cuda.synchronize()
    assert status.item() == 0
    assert torch.equal(vals, base[0]) and torch.equal(mask, base[1]) and torch.equal(src, base[2])
