"""GPU parity of the fused latest-1 lookup + linear map (the reference's
triton_fused_latest1_linear, ravel_lm/triton_memory.py:378-485) against an
fp64 CPU formulation built on the oracle's sources: out = A @ W^T with A the
rows gathered through oracle.latest_k_src, and its autograd for the gradients.

Tolerance: the device forms exact products and accumulates them in fp32, then
rounds once to the output dtype, so per element
  |out - ref| <= rtol |ref| + K 2^-24 (|A| @ |W|^T)
with K = C*P the length of the sum (fp32 accumulation of K products) and rtol
1e-2 for bf16/f16 outputs (bf16 rounding is 2^-8 relative), 1e-5 for fp32."""
import numpy as np
import pytest
import torch

import oracle
from ravel_em import fused_latest1_linear

pytestmark = pytest.mark.gpu


def dense_ref(write, payload, read, weight, A):
    src = oracle.latest_k_src(write, read, address_space=A, k=1)[..., 0]
    B, T, C, P = payload.shape
    s = torch.from_numpy(src.astype(np.int64)).view(-1)
    p64 = payload.double().reshape(-1, P)
    rows = p64.index_select(0, s.clamp_min(0)) * (s >= 0).view(-1, 1).double()
    a = rows.view(B * T, C * P)
    w = weight.double()
    return (a @ w.t()).view(B, T, -1), (a.abs() @ w.abs().t()).view(B, T, -1), src


def check_close(out, ref, scale, K, dtype):
    rel = 1e-5 if dtype in (torch.float32, torch.float64) else 1e-2
    err = (out.double().cpu() - ref).abs()
    bound = rel * ref.abs() + 1.01 * K * 2.0 ** -24 * scale + 1e-30
    frac = (err / bound).max().item()
    print(f"[fused] max err/bound {frac:.3f}", flush=True)
    bad = (err > bound).nonzero()
    assert bad.numel() == 0, f"{bad.shape[0]} elements out of tolerance, first {bad[:3].tolist()}"


CASES = [
    # B, T, C, P, M, A, dtype, separate reads
    (2, 300, 16, 64, 192, 97, torch.bfloat16, False),   # the headline shapes' head/row layout
    (1, 257, 3, 8, 8, 11, torch.bfloat16, False),       # K = 24: one partial chunk
    (2, 130, 4, 16, 256, 13, torch.float16, False),     # f16, M = 256 (all four column waves)
    (1, 1000, 2, 32, 64, 5, torch.bfloat16, True),      # separate reads
    (3, 45, 1, 128, 120, 7, torch.bfloat16, False),     # one head, K = 128
    (2, 200, 8, 64, 128, 31, torch.bfloat16, False),    # two column tiles per wave
    (1, 150, 5, 24, 200, 9, torch.float16, False),      # four column tiles, M not a multiple of 64
    (1, 90, 2, 8, 40, 3, torch.bfloat16, False),        # one column tile, K = 16
    (2, 256, 3, 24, 68, 260, torch.bfloat16, False),    # M = 68 (d_model of ravel_200k_byte)
    (2, 256, 3, 24, 68, 260, torch.float32, False),     # the same in fp32 (autocast off)
    (2, 300, 16, 64, 192, 97, torch.float32, False),    # fp32, 16 heads, K = 1024
    (1, 500, 2, 32, 128, 5, torch.float32, True),       # fp32, separate reads
    (1, 200, 3, 8, 300, 13, torch.bfloat16, False),     # M > 256: two column blocks
    (1, 130, 2, 16, 520, 7, torch.float16, False),      # three column blocks, last partial
    (1, 120, 2, 4, 77, 5, torch.float32, False),        # fp32 P = 4, odd M
]


@pytest.mark.parametrize("case", CASES, ids=[str(i) for i in range(len(CASES))])
def test_fused_latest1_linear_forward(device, case):
    B, T, C, P, M, A, dtype, sep = case
    g = torch.Generator().manual_seed(T + M)
    w = torch.randint(0, A, (B, T, C), generator=g)
    r = torch.randint(0, A, (B, T, C), generator=g) if sep else None
    p = torch.randn(B, T, C, P, generator=g).to(dtype)
    W = (torch.randn(M, C * P, generator=g) / (C * P) ** 0.5).to(dtype)
    out = fused_latest1_linear(w.to(device), p.to(device), None if r is None else r.to(device),
                               W.to(device), address_space=A)
    torch.cuda.synchronize()
    assert out.shape == (B, T, M) and out.dtype == dtype
    ref, scale, _ = dense_ref(w, p, r, W, A)
    check_close(out, ref, scale, C * P, dtype)


def test_fused_latest1_linear_deterministic(device):
    g = torch.Generator().manual_seed(3)
    w = torch.randint(0, 50, (2, 700, 16), generator=g).to(device)
    p = torch.randn(2, 700, 16, 64, generator=g).to(torch.bfloat16).to(device)
    W = torch.randn(192, 1024, generator=g).to(torch.bfloat16).to(device)
    a = fused_latest1_linear(w, p, None, W, address_space=50)
    b = fused_latest1_linear(w, p, None, W, address_space=50)
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype,P,M", [(torch.float64, 16, 64), (torch.bfloat16, 12, 64),
                                       (torch.float32, 6, 68)])
def test_fused_latest1_linear_other_shapes_use_the_lookup_and_a_library_gemm(device, dtype, P, M):
    B, T, C, A = 2, 80, 3, 9
    g = torch.Generator().manual_seed(P * M)
    w = torch.randint(0, A, (B, T, C), generator=g)
    p = torch.randn(B, T, C, P, generator=g).to(dtype)
    W = (torch.randn(M, C * P, generator=g) / (C * P) ** 0.5).to(dtype)
    out = fused_latest1_linear(w.to(device), p.to(device), None, W.to(device), address_space=A)
    ref, scale, _ = dense_ref(w, p, None, W, A)
    check_close(out, ref, scale, C * P, dtype)


@pytest.mark.parametrize("dtype,M", [(torch.bfloat16, 32), (torch.float32, 68)])
def test_fused_latest1_linear_gradients(device, dtype, M):
    B, T, C, P, A = 2, 60, 3, 16, 7
    g = torch.Generator().manual_seed(11)
    w = torch.randint(0, A, (B, T, C), generator=g)
    p = torch.randn(B, T, C, P, generator=g).to(dtype)
    W = (torch.randn(M, C * P, generator=g) / (C * P) ** 0.5).to(dtype)
    gout = torch.randn(B, T, M, generator=g).to(dtype)
    pd = p.to(device).requires_grad_(True)
    Wd = W.to(device).requires_grad_(True)
    out = fused_latest1_linear(w.to(device), pd, None, Wd, address_space=A)
    out.backward(gout.to(device))
    # fp64 autograd of the dense formulation on the CPU
    src = oracle.latest_k_src(w, None, address_space=A, k=1)[..., 0]
    s = torch.from_numpy(src.astype(np.int64)).view(-1)
    p64 = p.double().requires_grad_(True)
    W64 = W.double().requires_grad_(True)
    rows = p64.reshape(-1, P).index_select(0, s.clamp_min(0)) * (s >= 0).view(-1, 1).double()
    ref = rows.view(B * T, C * P) @ W64.t()
    ref.backward(gout.double().view(B * T, M))
    gp = pd.grad.double().cpu()
    gw = Wd.grad.double().cpu()
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-5
    assert (gp - p64.grad).abs().max() <= tol * p64.grad.abs().max() + 1e-6
    assert (gw - W64.grad).abs().max() <= tol * W64.grad.abs().max() + 1e-6
