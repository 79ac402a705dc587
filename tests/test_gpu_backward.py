"""GPU gradients of the lookups against autograd of an independent dense
formulation (fp64, CPU): the latest-k values are a linear gather from the
oracle's source indices, the sums a linear map by per-stream masks."""
import numpy as np
import pytest
import torch

import oracle
from ravel_em import causal_last_k_lookup, causal_sum_lookup

pytestmark = pytest.mark.gpu


def dense_latest_k(payload64: torch.Tensor, src: np.ndarray) -> torch.Tensor:
    B, T, C, D = payload64.shape
    s = torch.from_numpy(src.astype(np.int64)).view(-1)
    rows = payload64.reshape(-1, D).index_select(0, s.clamp_min(0))
    rows = rows * (s >= 0).view(-1, 1).to(rows.dtype)
    return rows.view(B, T, C, src.shape[-1], D)


CASES = [
    # B, T, C, A, masked, separate reads, k
    (2, 50, 3, 7, False, False, 1),
    (2, 50, 3, 7, False, False, 3),
    (2, 50, 3, 7, True, False, 2),
    (2, 50, 3, 7, False, True, 2),
    (1, 5000, 2, 3, False, False, 4),
]


@pytest.mark.parametrize("case", CASES, ids=[str(i) for i in range(len(CASES))])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_latest_k_gradient(device, case, dtype):
    B, T, C, A, masked, sep, k = case
    g = torch.Generator().manual_seed(T + k)
    w = torch.randint(0, A, (B, T, C), generator=g)
    r = torch.randint(0, A, (B, T, C), generator=g) if sep else None
    m = (torch.rand(B, T, generator=g) < 0.6) if masked else None
    p = torch.randn(B, T, C, 4, generator=g).to(dtype)
    gy = torch.randn(B, T, C, k, 4, generator=g).to(dtype)
    pg = p.to(device).requires_grad_(True)
    vals, _ = causal_last_k_lookup(w.to(device), pg, None if r is None else r.to(device), address_space=A, k=k,
                                   write_mask=None if m is None else m.to(device))
    (grad,) = torch.autograd.grad(vals, pg, gy.to(device))
    src = oracle.latest_k_src(w, r, address_space=A, k=k, write_mask=m)
    p64 = p.double().requires_grad_(True)
    (want,) = torch.autograd.grad(dense_latest_k(p64, src), p64, gy.double())
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    torch.testing.assert_close(grad.cpu().double(), want, rtol=tol, atol=tol)


# Separate reads and masked writes take the sorted backward (a stable sort of
# the slots' source ids, then each source's slots summed in slot order): the
# gradient must be bit-identical from run to run, and match fp64 autograd of
# the dense formulation.  Few addresses make long runs of slots per source,
# which cross the summing kernels' parts (walker: 16-byte rows) and chunks
# (other rows).
DET_CASES = [
    # B, T, C, A, kept share of writes (1 = no mask), separate reads, k, D, dtype
    (2, 3000, 3, 4, 1.0, True, 4, 64, torch.bfloat16),
    (1, 5000, 2, 2, 0.7, False, 3, 5, torch.float32),
    (2, 2000, 2, 7, 0.7, True, 8, 16, torch.float16),
    (1, 6000, 1, 1, 1.0, True, 2, 8, torch.float64),
    (2, 500, 4, 300, 0.7, True, 1, 24, torch.bfloat16),
    # one write in 500 kept: ~1500 slots name each source, runs cross parts
    (1, 8000, 2, 1, 0.002, True, 3, 64, torch.bfloat16),
    (1, 8000, 2, 1, 0.002, False, 3, 6, torch.float32),
]


@pytest.mark.parametrize("case", DET_CASES, ids=[str(i) for i in range(len(DET_CASES))])
def test_latest_k_backward_sorted_is_deterministic(device, case):
    B, T, C, A, keep, sep, k, D, dtype = case
    print(f"[sorted backward] {case}", flush=True)
    g = torch.Generator().manual_seed(T + k + D)
    w = torch.randint(0, A, (B, T, C), generator=g)
    r = torch.randint(0, A, (B, T, C), generator=g) if sep else None
    m = (torch.rand(B, T, generator=g) < keep) if keep < 1 else None
    p = torch.randn(B, T, C, D, generator=g).to(dtype)
    gy = torch.randn(B, T, C, k, D, generator=g).to(dtype)
    grads = []
    for _ in range(2):
        pg = p.to(device).requires_grad_(True)
        vals, _ = causal_last_k_lookup(w.to(device), pg, None if r is None else r.to(device),
                                       address_space=A, k=k,
                                       write_mask=None if m is None else m.to(device))
        (grad,) = torch.autograd.grad(vals, pg, gy.to(device))
        grads.append(grad.cpu())
    bits = {2: torch.int16, 4: torch.int32, 8: torch.int64}[grads[0].element_size()]
    assert torch.equal(grads[0].view(bits), grads[1].view(bits)), "two runs differ"
    src = oracle.latest_k_src(w, r, address_space=A, k=k, write_mask=m)
    p64 = p.double().requires_grad_(True)
    (want,) = torch.autograd.grad(dense_latest_k(p64, src), p64, gy.double())
    # a source's slots summed in fp32 (16-bit rows) or fp64, rounded once
    acc_u = 2.0 ** -24 if dtype in (torch.bfloat16, torch.float16) else 2.0 ** -52
    rtol = {torch.bfloat16: 1e-2, torch.float16: 1e-2, torch.float32: 1e-5, torch.float64: 1e-5}[dtype]
    (scale,) = torch.autograd.grad(dense_latest_k(p64, src), p64, gy.double().abs())
    (nterm,) = torch.autograd.grad(dense_latest_k(p64, src), p64, torch.ones_like(gy, dtype=torch.float64))
    err = (grads[0].double() - want).abs()
    bound = rtol * want.abs() + 1.01 * nterm * acc_u * scale + 1e-30
    print(f"[sorted backward] max err/bound {(err / bound).max().item():.3f}, "
          f"longest run {int(nterm.max().item())}", flush=True)
    assert (err <= bound).all()


def dense_sum(payload64, write, read, A, mask):
    """out[r] = sum over earlier same-stream writes, as an explicit masked matmul."""
    B, T, C, D = payload64.shape
    rd = write if read is None else read
    wa = torch.remainder(write, A)
    ra = torch.remainder(rd, A)
    tt = torch.arange(T)
    earlier = tt.view(T, 1) > tt.view(1, T)  # [t_read, t_write]
    outs = []
    for b in range(B):
        heads = []
        for c in range(C):
            same = ra[b, :, c].view(T, 1) == wa[b, :, c].view(1, T)
            M = (same & earlier).double()
            if mask is not None:
                M = M * mask[b].double().view(1, T)
            heads.append(M @ payload64[b, :, c])
        outs.append(torch.stack(heads, dim=1))
    return torch.stack(outs)


@pytest.mark.parametrize("case", CASES[:4], ids=[str(i) for i in range(4)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sum_gradient(device, case, dtype):
    B, T, C, A, masked, sep, _ = case
    g = torch.Generator().manual_seed(T + 99)
    w = torch.randint(0, A, (B, T, C), generator=g)
    r = torch.randint(0, A, (B, T, C), generator=g) if sep else None
    m = (torch.rand(B, T, generator=g) < 0.6) if masked else None
    p = torch.randn(B, T, C, 4, generator=g).to(dtype)
    gy = torch.randn(B, T, C, 4, generator=g).to(dtype)
    pg = p.to(device).requires_grad_(True)
    out, _ = causal_sum_lookup(w.to(device), pg, None if r is None else r.to(device), address_space=A,
                               write_mask=None if m is None else m.to(device))
    (grad,) = torch.autograd.grad(out, pg, gy.to(device))
    p64 = p.double().requires_grad_(True)
    (want,) = torch.autograd.grad(dense_sum(p64, w, r, A, m), p64, gy.double())
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    torch.testing.assert_close(grad.cpu().double(), want, rtol=tol, atol=tol)
