"""Pin the CPU oracle before trusting it.

Each oracle function is checked against (1) the known-answer cases of the
reference's own tests (tests/golden/reference_kats.json), (2) the other,
independently written restatements (C history replay, torch restatement of the
reference algorithm, pure-Python brute force), and (3) closed forms and
invariants, chosen so that plausible mistakes (off-by-one causality, a wrong
slot order, dropped masking, wrong remainder sign, missing int32 conversion)
fail at least one check.  test_planted_mistakes_are_caught shows that.
"""
import json
import os

import numpy as np
import pytest
import torch

import oracle
from oracle import brute, torch_ref

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))


def _t(x, dtype=torch.long):
    return torch.tensor(x, dtype=dtype)


# ------------------------------------------------------------------ KATs --


def test_key_dtype_kat():
    for case in KATS["key_dtype"]["cases"]:
        want = getattr(torch, case["dtype"])
        args = (case["B"], case["T"], case["C"], case["A"])
        assert torch_ref.key_dtype(*args) == want
        assert oracle.key_bits(*args) == (32 if want == torch.int32 else 64)
        assert brute.key_is_int32(*args) == (want == torch.int32)


def _check_latest_exact(vals, mask, case):
    for a in case["asserted"]:
        idx = tuple(a["index"])
        if "mask" in a:
            assert bool(mask[idx]) == a["mask"]
        else:
            assert vals[idx].item() == a["value"]


def test_latest_exact_kat_all_oracles():
    case = KATS["latest_exact"]
    w, p = _t(case["write"]), _t(case["payload"], torch.float32)
    A, k = case["address_space"], case["k"]
    vals, mask, src = oracle.latest_k(w, p, address_space=A, k=k)
    _check_latest_exact(vals, mask, case)
    assert src.tolist() == case["full_src"]
    tv, tm = torch_ref.latest_k(w, p, address_space=A, k=k)
    _check_latest_exact(tv, tm, case)
    assert torch.equal(tm, mask)
    assert brute.latest_k_src(case["write"], None, A, k) == case["full_src"]


def test_latest_separate_reads_mask_kat_all_oracles():
    case = KATS["latest_separate_reads_masked"]
    w, r = _t(case["write"]), _t(case["read"])
    m = torch.tensor(case["write_mask"])
    A, k = case["address_space"], case["k"]
    src = oracle.latest_k_src(w, r, address_space=A, k=k, write_mask=m)
    assert src.tolist() == case["full_src"]
    assert brute.latest_k_src(case["write"], case["read"], A, k, case["write_mask"]) == case["full_src"]
    p = torch.randn(1, 6, 1, 3, generator=torch.Generator().manual_seed(3))
    ov, om = oracle.gather_slots(p, src)
    tv, tm = torch_ref.latest_k(w, p, r, address_space=A, k=k, write_mask=m)
    assert torch.equal(om, tm)
    assert torch.equal(ov, tv)


def test_sum_exact_kat_all_oracles():
    case = KATS["sum_exact"]
    w, p = _t(case["write"]), _t(case["payload"], torch.float32)
    A = case["address_space"]
    out, mask = oracle.seg_sum(w, p, address_space=A)
    for a in case["asserted"]:
        assert out[tuple(a["index"])].item() == a["value"]
    assert out.tolist() == case["full_sum"]
    assert mask.tolist() == case["full_mask"]
    tv, tm = torch_ref.seg_sum(w, p, address_space=A)
    assert tv.tolist() == case["full_sum"]
    assert tm.tolist() == case["full_mask"]
    bv, bm = brute.seg_sum(case["write"], None, case["payload"], A)
    assert bv == case["full_sum"] and bm == case["full_mask"]


def test_decode_cache_kat():
    case = KATS["decode_cache"]
    B, C, A, D = case["batch_size"], case["n_heads"], case["address_space"], case["payload_dim"]
    values = torch.zeros(B, C, A, D)
    filled = torch.zeros(B, C, A, dtype=torch.bool)
    addr = _t(case["addresses"])
    _, mask = torch_ref.cache_read(values, filled, addr)
    assert mask.tolist() == case["mask_before_write"]
    payload = _t(case["payload"], torch.float32)
    torch_ref.cache_write(values, filled, addr, payload)
    vals, mask = torch_ref.cache_read(values, filled, addr)
    assert mask.tolist() == case["mask_after_write"]
    assert torch.equal(vals, payload)
    # The C oracle's one-write prefill is the same state.
    cv, cf = oracle.cache_prefill(addr.view(B, 1, C), payload.view(B, 1, C, D), address_space=A, k=1)
    assert torch.equal(cv[..., 0, :], values) and torch.equal(cf[..., 0], filled)


def test_bench_forced_repeat_kat():
    case = KATS["bench_forced_repeat"]
    torch.manual_seed(case["torch_manual_seed"])
    B, T, C, D, A = case["B"], case["T"], case["C"], case["D"], case["address_space"]
    addr = torch.randint(0, max(1, A - 1), (B, T, C))
    payload = torch.randn(B, T, C, D)
    for t in case["forced_times"]:
        addr[:, t, :] = A - 1
    payload[:, case["forced_times"][0], :, :] = case["forced_value"]
    vals, mask, _ = oracle.latest_k(addr, payload, address_space=A, k=1)
    t1 = case["forced_times"][1]
    assert bool(mask[:, t1, :, 0].all())
    assert torch.equal(vals[:, t1, :, 0, :], torch.full((B, C, D), case["forced_value"]))
    tv, _ = torch_ref.latest_k(addr, payload, address_space=A, k=1)
    assert torch.equal(tv[:, t1, :, 0, :], vals[:, t1, :, 0, :])


# ------------------------------------------------- cross-restatement --


def _rand_case(seed, B, T, C, A, lo=None, hi=None, masked=False, sep_read=False):
    g = torch.Generator().manual_seed(seed)
    lo = 0 if lo is None else lo
    hi = A if hi is None else hi
    w = torch.randint(lo, hi, (B, T, C), generator=g)
    r = torch.randint(lo, hi, (B, T, C), generator=g) if sep_read else None
    m = (torch.rand(B, T, generator=g) < 0.7) if masked else None
    return w, r, m


CASES = [
    # seed, B, T, C, A, lo, hi, masked, sep_read, k
    (1, 2, 17, 3, 11, None, None, False, False, 1),
    (2, 2, 17, 3, 11, None, None, False, True, 2),
    (3, 3, 40, 2, 5, None, None, True, False, 3),
    (4, 2, 33, 4, 7, None, None, True, True, 4),
    (5, 1, 64, 1, 3, -20, 20, False, True, 5),  # negative addresses wrap
    (6, 2, 25, 2, 1, None, None, False, False, 2),  # A = 1: one stream per (b,c)
    (7, 2, 9, 2, 4, None, None, False, False, 12),  # k > T
    (8, 1, 30, 3, 6, 2**31 - 10, 2**31 + 10, False, True, 2),  # int32 truncation
]


@pytest.mark.parametrize("seed,B,T,C,A,lo,hi,masked,sep,k", CASES)
def test_latest_k_three_way(seed, B, T, C, A, lo, hi, masked, sep, k):
    w, r, m = _rand_case(seed, B, T, C, A, lo, hi, masked, sep)
    src = oracle.latest_k_src(w, r, address_space=A, k=k, write_mask=m)
    bsrc = brute.latest_k_src(w.tolist(), None if r is None else r.tolist(), A, k,
                              None if m is None else m.tolist())
    assert src.tolist() == bsrc
    p = torch.randn(B, T, C, 3, generator=torch.Generator().manual_seed(seed + 100))
    ov, om = oracle.gather_slots(p, src)
    tv, tm = torch_ref.latest_k(w, p, r, address_space=A, k=k, write_mask=m)
    assert torch.equal(om, tm)
    assert torch.equal(ov, tv)  # pure copies; invalid slots are +0 here and 0*x there


@pytest.mark.parametrize("seed,B,T,C,A,lo,hi,masked,sep,k", CASES)
def test_sort_order_three_way(seed, B, T, C, A, lo, hi, masked, sep, k):
    w, _, m = _rand_case(seed, B, T, C, A, lo, hi, masked, sep)
    keys, order = oracle.sort_order(w, address_space=A, write_mask=m)
    bkeys, border = brute.sorted_keys(w.tolist(), A, None if m is None else m.tolist())
    assert keys.tolist() == bkeys and order.tolist() == border
    # the same keys sorted by torch (what the reference runs)
    kd = torch_ref.key_dtype(B, T, C, A)
    _, flat = torch_ref._flat_keys(torch_ref._reduced(w, kd, A), A, 0)
    if m is not None:
        flat = flat[m.view(B, T, 1).expand(B, T, C).reshape(-1)]
    sk, so = torch.sort(flat)
    assert sk.tolist() == bkeys and so.tolist() == border


@pytest.mark.parametrize("seed,B,T,C,A,lo,hi,masked,sep,k", CASES)
def test_seg_sum_three_way(seed, B, T, C, A, lo, hi, masked, sep, k):
    w, r, m = _rand_case(seed, B, T, C, A, lo, hi, masked, sep)
    p = torch.randn(B, T, C, 4, generator=torch.Generator().manual_seed(seed + 200), dtype=torch.float64)
    out, mask = oracle.seg_sum(w, p, r, address_space=A, write_mask=m)
    bo, bm = brute.seg_sum(w.tolist(), None if r is None else r.tolist(), p.tolist(), A,
                           None if m is None else m.tolist())
    assert out.tolist() == bo  # same summation order in fp64: identical
    assert mask.tolist() == bm
    tv, tm = torch_ref.seg_sum(w, p, r, address_space=A, write_mask=m)
    assert torch.equal(tm, mask)
    torch.testing.assert_close(tv, out, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("seed,B,T,C,A,lo,hi,masked,sep,k", CASES)
def test_seg_sum_grad_matches_autograd(seed, B, T, C, A, lo, hi, masked, sep, k):
    """oracle.seg_sum_grad against autograd of the torch restatement of the
    reference's sum (an independent, differentiable formulation); n against
    the same autograd with unit gradients."""
    w, r, m = _rand_case(seed, B, T, C, A, lo, hi, masked, sep)
    gen = torch.Generator().manual_seed(seed + 300)
    p = torch.randn(B, T, C, 3, generator=gen, dtype=torch.float64).requires_grad_(True)
    gy = torch.randn(B, T, C, 3, generator=gen, dtype=torch.float64)
    tv, _ = torch_ref.seg_sum(w, p, r, address_space=A, write_mask=m)
    (want,) = torch.autograd.grad(tv, p, gy)
    g, s, n = oracle.seg_sum_grad(w, gy, r, address_space=A, write_mask=m)
    torch.testing.assert_close(g, want, rtol=1e-12, atol=1e-12)
    (want_s,) = torch.autograd.grad(torch_ref.seg_sum(w, p, r, address_space=A, write_mask=m)[0],
                                    p, gy.abs())
    torch.testing.assert_close(s, want_s, rtol=1e-12, atol=1e-12)
    (want_n,) = torch.autograd.grad(torch_ref.seg_sum(w, p, r, address_space=A, write_mask=m)[0],
                                    p, torch.ones_like(gy))
    assert torch.equal(n.expand_as(want_n), want_n)


def test_cache_prefill_matches_replay():
    g = torch.Generator().manual_seed(11)
    B, T, C, A, k, D = 2, 30, 3, 6, 3, 2
    w = torch.randint(-2, A + 2, (B, T, C), generator=g)  # out of range clamps
    m = torch.rand(B, T, generator=g) < 0.8
    p = torch.randn(B, T, C, D, generator=g)
    vals, filled = oracle.cache_prefill(w, p, address_space=A, k=k, write_mask=m)
    steps = [("write", w[:, t].tolist(), p[:, t].tolist()) for t in range(T) if bool(m[0, t]) and bool(m[1, t])]
    # replay per batch row to honour a per-row mask
    for b in range(B):
        st = [("write", [w[b, t].tolist()], [p[b, t].tolist()]) for t in range(T) if bool(m[b, t])]
        state, _ = brute.cache_replay(st, 1, C, A, k)
        for c in range(C):
            for a in range(A):
                hist = state.get((0, c, a), [])
                for j in range(k):
                    assert bool(filled[b, c, a, j]) == (j < len(hist))
                    want = hist[j] if j < len(hist) else [0.0] * D
                    assert vals[b, c, a, j].tolist() == want
    del steps


# ---------------------------------------------------------- closed forms --


def test_single_stream_closed_form():
    """One address per (b,c): slot j of time t is t-1-j; sum is the exclusive
    prefix sum (numpy cumsum in fp64)."""
    B, T, C, A, k = 2, 50, 3, 9, 4
    w = torch.full((B, T, C), 7)
    src = oracle.latest_k_src(w, address_space=A, k=k)
    for b in range(B):
        for t in range(T):
            for c in range(C):
                want = [(b * T + t - 1 - j) * C + c if t - 1 - j >= 0 else -1 for j in range(k)]
                assert src[b, t, c].tolist() == want
    p = torch.randn(B, T, C, 5, dtype=torch.float64, generator=torch.Generator().manual_seed(5))
    out, mask = oracle.seg_sum(w, p, address_space=A)
    excl = np.cumsum(p.numpy(), axis=1) - p.numpy()
    np.testing.assert_allclose(out.numpy(), excl, rtol=1e-12, atol=1e-12)
    assert mask[:, 0].sum() == 0 and bool(mask[:, 1:].all())


def test_previous_occurrence_closed_form():
    """k=1, read == write: the source is the previous occurrence of the same
    reduced address in the (b,c) row (numpy brute force, independent code)."""
    g = np.random.default_rng(9)
    B, T, C, A = 3, 200, 4, 13
    w = g.integers(-40, 40, size=(B, T, C))
    src = oracle.latest_k_src(torch.from_numpy(w), address_space=A, k=1)[..., 0]
    red = np.mod(w, A)
    for b in range(B):
        for c in range(C):
            last = {}
            for t in range(T):
                a = red[b, t, c]
                want = (b * T + last[a]) * C + c if a in last else -1
                assert src[b, t, c] == want
                last[a] = t


def test_int32_key_truncation_matches_reference_conversion():
    """With an int32 key dtype the reference converts addresses with
    .to(int32) before the remainder: 2^32 + 5 behaves as 5."""
    B, T, C, A = 1, 6, 1, 10
    assert torch_ref.key_dtype(B, T, C, A) == torch.int32
    w = torch.tensor([[[5], [2**32 + 5], [3], [2**32 + 3], [-5], [5]]])
    src = oracle.latest_k_src(w, address_space=A, k=1)[..., 0].reshape(-1).tolist()
    # 2^32+5 -> 5 (matches t=0); 2^32+3 -> 3 (matches t=2); -5 -> 5 (matches t=1)
    assert src == [-1, 0, -1, 2, 1, 4]
    p = torch.arange(T, dtype=torch.float32).view(1, T, 1, 1)
    tv, tm = torch_ref.latest_k(w, p, address_space=A, k=1)
    assert tv.reshape(-1).tolist() == [0.0, 0.0, 0.0, 2.0, 1.0, 4.0]


def test_all_masked_gives_empty():
    w = torch.randint(0, 5, (2, 8, 3))
    m = torch.zeros(2, 8, dtype=torch.bool)
    src = oracle.latest_k_src(w, address_space=5, k=2, write_mask=m)
    assert (src == -1).all()
    keys, order = oracle.sort_order(w, address_space=5, write_mask=m)
    assert keys.size == 0 and order.size == 0
    tv, tm = torch_ref.latest_k(w, torch.randn(2, 8, 3, 2), address_space=5, k=2, write_mask=m)
    assert not tm.any() and not tv.any()


# ------------------------------------------------------ planted mistakes --


def test_planted_mistakes_are_caught(monkeypatch):
    """Each plausible mistake, planted in a restatement, fails a check above."""
    case = KATS["latest_exact"]
    w, p = _t(case["write"]), _t(case["payload"], torch.float32)

    # 1. non-strict causality (read key at t instead of t-1)
    orig = torch_ref._flat_keys
    monkeypatch.setattr(torch_ref, "_flat_keys", lambda addr, A, shift: orig(addr, A, 0))
    vals, mask = torch_ref.latest_k(w, p, address_space=8, k=2)
    with pytest.raises(AssertionError):
        _check_latest_exact(vals, mask, case)
    monkeypatch.setattr(torch_ref, "_flat_keys", orig)

    # 2. slot order reversed (oldest first)
    src = oracle.latest_k_src(w, address_space=8, k=2)
    assert src[..., ::-1].tolist() != case["full_src"]

    # 3. write_mask ignored
    cm = KATS["latest_separate_reads_masked"]
    got = brute.latest_k_src(cm["write"], cm["read"], 8, 2, None)
    assert got != cm["full_src"]

    # 4. C-style remainder (sign of the dividend) instead of Python's
    # (-3 mod 8 is 5 in Python, -3 with C's fmod: t=1 must see t=0)
    w2 = [[[-3], [5], [-3]]]
    assert oracle.latest_k_src(torch.tensor(w2), address_space=8, k=1).reshape(-1).tolist() == [-1, 0, 1]
    monkeypatch.setattr(brute, "wrap", lambda a, A, v: int(np.fmod(a, A)))
    assert brute.latest_k_src(w2, None, 8, 1) != [[[[-1]], [[0]], [[1]]]]
