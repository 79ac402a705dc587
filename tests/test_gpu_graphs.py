"""The operators under HIP graph capture.

The library allocates nothing, clears its own state with kernels (no
hipMemsetAsync) and launches on torch's current stream, so a torch CUDA graph
can capture a whole call.  Each graph here is replayed several times, with eager
work and synchronizations in between, and every replay is checked bit-for-bit
against the eager call.
"""
import pytest
import torch

from ravel_em import (RavelLayerCache, causal_last_k_and_sum_lookup, causal_last_k_lookup,
                      causal_sum_lookup)

pytestmark = pytest.mark.gpu


def _replay_matches(fn, make_eager_noise, reps=4):
    ref = [t.clone() for t in fn()]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm up on the side stream, as torch requires before capture
        fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = fn()
    for _ in range(reps):
        make_eager_noise()
        torch.cuda.synchronize()
        for o in outs:
            o.fill_(7)  # stale contents must not survive a replay
        g.replay()
        torch.cuda.synchronize()
        for got, want in zip(outs, ref):
            assert torch.equal(got, want)


def _noise(device):
    def run():
        x = torch.randn(1 << 16, device=device)
        (x * 2).sum().item()
    return run


@pytest.mark.parametrize("shape", [(2, 300, 3, 40, 2), (1, 6000, 4, 5000, 1), (1, 65536, 4, 65536, 1)])
def test_latest_k_replays_match_eager(device, shape):
    B, T, C, A, k = shape
    print(f"[graph latest_k] {shape}", flush=True)
    g = torch.Generator().manual_seed(T)
    w = torch.randint(0, A, (B, T, C), generator=g).to(device)
    p = torch.randn(B, T, C, 16, generator=g).to(torch.bfloat16).to(device)
    _replay_matches(lambda: causal_last_k_lookup(w, p, address_space=A, k=k), _noise(device))


@pytest.mark.parametrize("shape", [(2, 300, 3, 40), (1, 6000, 4, 5000)])
def test_sum_replays_match_eager(device, shape):
    B, T, C, A = shape
    print(f"[graph seg_sum] {shape}", flush=True)
    g = torch.Generator().manual_seed(T + 1)
    w = torch.randint(0, A, (B, T, C), generator=g).to(device)
    r = torch.randint(0, A, (B, T, C), generator=g).to(device)
    p = torch.randn(B, T, C, 8, generator=g).to(device)
    _replay_matches(lambda: causal_sum_lookup(w, p, address_space=A), _noise(device))
    _replay_matches(lambda: causal_sum_lookup(w, p, r, address_space=A), _noise(device))


@pytest.mark.parametrize("shape", [(2, 300, 3, 40, 2, False), (2, 300, 3, 40, 4, True),
                                   (1, 6000, 4, 5000, 1, False), (2, 700, 3, 23, 12, False)])
def test_joint_replays_match_eager(device, shape):
    """The joint call in its three forms (merged short tape, long-tape walker with
    latest-1 values and the mask copy, and the two operators for k > 8)."""
    B, T, C, A, k, sep = shape
    print(f"[graph latest_k_sum] {shape}", flush=True)
    g = torch.Generator().manual_seed(T + k)
    w = torch.randint(0, A, (B, T, C), generator=g).to(device)
    r = torch.randint(0, A, (B, T, C), generator=g).to(device) if sep else None
    p = torch.randn(B, T, C, 16, generator=g).to(torch.bfloat16).to(device)
    _replay_matches(lambda: causal_last_k_and_sum_lookup(w, p, r, address_space=A, k=k),
                    _noise(device))


def test_cache_step_replays_match_eager(device):
    """A captured decode step replays against a cache that the previous replay
    advanced: every replay equals the eager step on a copy of that cache."""
    g = torch.Generator().manual_seed(5)
    B, C, A, k, D = 4, 3, 50, 2, 8
    cache = RavelLayerCache.empty(B, C, A, D, k=k, device=device, dtype=torch.float32)
    ra = torch.randint(0, A, (B, C), generator=g).to(device)
    wa = torch.randint(0, A, (B, C), generator=g).to(device)
    pay = torch.randn(B, C, D, generator=g).to(device)
    cache.step(ra, wa, pay)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    shadow = RavelLayerCache(values=cache.values.clone(), filled=cache.filled.clone())
    with torch.cuda.stream(s):
        shadow.step(ra, wa, pay)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        vals, mask = cache.step(ra, wa, pay)
    for _ in range(4):
        ra.copy_(torch.randint(0, A, (B, C), generator=g).to(device))
        wa.copy_(torch.randint(0, A, (B, C), generator=g).to(device))
        pay.copy_(torch.randn(B, C, D, generator=g).to(device))
        eager = RavelLayerCache(values=cache.values.clone(), filled=cache.filled.clone())
        ev, em = eager.step(ra, wa, pay)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(vals, ev) and torch.equal(mask, em)
        assert torch.equal(cache.values, eager.values) and torch.equal(cache.filled, eager.filled)


def test_torch_compile_traces_through_the_lookups(device):
    """fullgraph tracing goes through the registered ops (fake implementations
    and autograd formulas); results and gradients equal the eager calls."""
    g = torch.Generator().manual_seed(9)
    w = torch.randint(0, 30, (2, 200, 3), generator=g).to(device)
    p = torch.randn(2, 200, 3, 8, generator=g).to(device)

    def f(w, p):
        vals, mask = causal_last_k_lookup(w, p, address_space=30, k=2)
        s, smask = causal_sum_lookup(w, p, address_space=30)
        return vals.sum(dim=3) * mask.any(dim=3, keepdim=True) + s * smask.unsqueeze(-1)

    compiled = torch.compile(f, backend="aot_eager", fullgraph=True)
    pe = p.clone().requires_grad_(True)
    pc = p.clone().requires_grad_(True)
    want = f(w, pe)
    got = compiled(w, pc)
    assert torch.equal(got, want)
    weights = torch.randn_like(want)
    (want * weights).sum().backward()
    (got * weights).sum().backward()
    assert torch.allclose(pc.grad, pe.grad, rtol=1e-6, atol=1e-6)


def test_torch_compile_traces_through_the_joint_lookup(device):
    """fullgraph tracing goes through ravel_em::latest_k_sum (fake and autograd);
    results and gradients equal the eager call's."""
    g = torch.Generator().manual_seed(10)
    w = torch.randint(0, 30, (2, 200, 3), generator=g).to(device)
    p = torch.randn(2, 200, 3, 8, generator=g).to(device)

    def f(w, p):
        vals, mask, s, smask = causal_last_k_and_sum_lookup(w, p, address_space=30, k=2)
        return vals.sum(dim=3) * mask.any(dim=3, keepdim=True) + s * smask.unsqueeze(-1)

    compiled = torch.compile(f, backend="aot_eager", fullgraph=True)
    pe = p.clone().requires_grad_(True)
    pc = p.clone().requires_grad_(True)
    want = f(w, pe)
    got = compiled(w, pc)
    assert torch.equal(got, want)
    weights = torch.randn_like(want)
    (want * weights).sum().backward()
    (got * weights).sum().backward()
    assert torch.allclose(pc.grad, pe.grad, rtol=1e-6, atol=1e-6)
