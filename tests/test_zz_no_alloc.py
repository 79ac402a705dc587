"""ravel_em_latest_k_fwd_static (the entry point that allocates nothing)
against ravel_em_latest_k_fwd with a caller workspace, both through the C ABI:
two calls in a row, the second smaller, so the second runs on scratch the
first left behind.  Values, masks and sources must be bit-identical, and both
calls' status words zero."""
import pytest
import torch

from ravel_em import _native as nat

pytestmark = pytest.mark.gpu

STATIC_BYTES = 128 << 20  # RAVEL_EM_STATIC_SCRATCH_BYTES


def _inputs(device, seed, B, T, C, A, D, dtype, sep, masked):
    g = torch.Generator().manual_seed(seed)
    w = torch.randint(0, A, (B, T, C), generator=g)
    r = torch.randint(0, A, (B, T, C), generator=g) if sep else None
    m = (torch.rand(B, T, generator=g) < 0.7) if masked else None
    p = torch.randn(B, T, C, D, generator=g).to(dtype)
    mv = lambda t: None if t is None else t.to(device)
    return mv(w), mv(r), mv(m), mv(p)


def _outputs(p, k, want_src):
    B, T, C, D = p.shape
    vals = torch.full((B, T, C, k, D), 7, dtype=p.dtype, device=p.device)
    mask = torch.ones(B, T, C, k, dtype=torch.bool, device=p.device)
    src = torch.full((B, T, C, k), -5, dtype=torch.int32, device=p.device) if want_src else None
    return vals, mask, src


def _bits(t):
    return t.view({1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()])


def _run_both(w, r, m, p, A, k, want_src):
    lib = nat.library()
    B, T, C, D = p.shape
    stream = nat.stream_of(p)
    code = nat.payload_code(p.dtype)
    need = lib.ravel_em_latest_k_workspace(B, T, C, A, k, int(r is not None), int(m is not None),
                                           int(want_src))
    assert 0 < need <= STATIC_BYTES
    ws = nat.workspace(need, p.device)
    v1, m1, s1 = _outputs(p, k, want_src)
    nat.check(lib.ravel_em_latest_k_fwd(
        nat.ptr(w), nat.ptr(r), nat.addr_code(w.dtype), nat.ptr(m), nat.ptr(p), code,
        B, T, C, D, A, k, nat.ptr(v1), nat.ptr(m1), nat.ptr(s1), nat.ptr(ws), ws.numel(), stream))
    st1 = nat.status_word(ws)
    v2, m2, s2 = _outputs(p, k, want_src)
    status = torch.full((1,), 0xFFFF, dtype=torch.int32, device=p.device)
    nat.check(lib.ravel_em_latest_k_fwd_static(
        nat.ptr(w), nat.ptr(r), nat.addr_code(w.dtype), nat.ptr(m), nat.ptr(p), code,
        B, T, C, D, A, k, nat.ptr(v2), nat.ptr(m2), nat.ptr(s2), nat.ptr(status), stream))
    torch.cuda.synchronize()
    assert st1 == 0 and status.item() == 0, (st1, status.item())
    # bit-identical: compare the raw bits (±0 and NaN included)
    assert torch.equal(_bits(v1), _bits(v2))
    assert torch.equal(m1, m2)
    if want_src:
        assert torch.equal(s1, s2)


@pytest.mark.parametrize("order", ["large_then_small", "small_then_large_then_small"])
def test_static_scratch_matches_workspace_entry_point(device, order):
    big = dict(seed=1, B=4, T=65536, C=16, A=65536, D=64, dtype=torch.bfloat16, sep=False,
               masked=False, k=1, want_src=False)  # the cfg4 headline shape
    small = dict(seed=2, B=3, T=1000, C=3, A=50, D=8, dtype=torch.float32, sep=True, masked=True,
                 k=4, want_src=True)
    mid = dict(seed=3, B=2, T=70000, C=4, A=3, D=16, dtype=torch.float16, sep=False, masked=False,
               k=2, want_src=True)
    plan = [big, small] if order == "large_then_small" else [small, mid, small]
    for case in plan:
        print(f"[no-alloc] {case}", flush=True)
        w, r, m, p = _inputs(device, case["seed"], case["B"], case["T"], case["C"], case["A"],
                             case["D"], case["dtype"], case["sep"], case["masked"])
        _run_both(w, r, m, p, case["A"], case["k"], case["want_src"])
