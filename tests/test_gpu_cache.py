"""GPU parity of the decode cache (RavelLayerCache).

Checks: the reference's cache test (tests/test_memory.py:70-79); random
read/write sequences against the reference's k=1 gather/scatter semantics
(restated in oracle/torch_ref.py); the k-slot cache against the latest-k
lookup over the same prefix (the prefill/decode equivalence the reference pins
at model level, tests/test_model.py:78-90); the fused step against read-then-
write; and the one-pass prefill against the C oracle's sequential replay.
"""
import pytest
import torch

import oracle
from oracle import torch_ref
from ravel_em import RavelLayerCache, causal_last_k_lookup, workloads

pytestmark = pytest.mark.gpu


def test_decode_cache_latest_matches_semantics(device):
    cache = RavelLayerCache.empty(1, 2, 16, 3, device=device, dtype=torch.float32)
    addrs = torch.tensor([[5, 7]], device=device)
    vals, mask = cache.read(addrs)
    assert not mask.any()
    payload = torch.tensor([[[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]]], device=device)
    cache.write(addrs, payload)
    vals, mask = cache.read(addrs)
    assert mask.all()
    assert torch.allclose(vals, payload)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_k1_cache_matches_reference_sequence(device, dtype):
    g = torch.Generator().manual_seed(3)
    B, C, A, D = 3, 4, 10, 6
    cache = RavelLayerCache.empty(B, C, A, D, device=device, dtype=dtype)
    ref_v = torch.zeros(B, C, A, D, dtype=dtype)
    ref_f = torch.zeros(B, C, A, dtype=torch.bool)
    for step in range(40):
        ra = torch.randint(-3, A + 3, (B, C), generator=g)  # out-of-range addresses clamp
        wa = torch.randint(-3, A + 3, (B, C), generator=g)
        p = torch.randn(B, C, D, generator=g).to(dtype)
        vals, mask = cache.read(ra.to(device))
        rv, rm = torch_ref.cache_read(ref_v, ref_f, ra)
        assert torch.equal(mask.cpu(), rm) and torch.equal(vals.cpu(), rv)
        cache.write(wa.to(device), p.to(device))
        torch_ref.cache_write(ref_v, ref_f, wa, p)
    assert torch.equal(cache.values.cpu(), ref_v) and torch.equal(cache.filled.cpu(), ref_f)


@pytest.mark.parametrize("k", [1, 2, 4])
def test_stepped_cache_equals_latest_k_prefix(device, k):
    g = torch.Generator().manual_seed(k)
    B, T, C, A, D = 2, 60, 3, 7, 5
    w = torch.randint(0, A, (B, T, C), generator=g).to(device)
    r = torch.randint(0, A, (B, T, C), generator=g).to(device)
    p = torch.randn(B, T, C, D, generator=g).to(device)
    want, want_mask = causal_last_k_lookup(w, p, r, address_space=A, k=k)
    cache = RavelLayerCache.empty(B, C, A, D, device=device, dtype=torch.float32, k=k)
    for t in range(T):
        vals, mask = cache.step(r[:, t], w[:, t], p[:, t])
        if k == 1:
            vals, mask = vals.unsqueeze(2), mask.unsqueeze(2)
        assert torch.equal(mask, want_mask[:, t]), t
        assert torch.equal(vals, want[:, t]), t


@pytest.mark.parametrize("k", [1, 3])
def test_step_equals_read_then_write(device, k):
    g = torch.Generator().manual_seed(10 + k)
    B, C, A, D = 4, 2, 6, 16
    c1 = RavelLayerCache.empty(B, C, A, D, device=device, dtype=torch.bfloat16, k=k)
    c2 = RavelLayerCache.empty(B, C, A, D, device=device, dtype=torch.bfloat16, k=k)
    for _ in range(30):
        ra = torch.randint(0, A, (B, C), generator=g).to(device)
        wa = ra if torch.rand((), generator=g) < 0.5 else torch.randint(0, A, (B, C), generator=g).to(device)
        p = torch.randn(B, C, D, generator=g).to(device, torch.bfloat16)
        v1, m1 = c1.step(ra, wa, p)
        v2, m2 = c2.read(ra)
        c2.write(wa, p)
        assert torch.equal(v1, v2) and torch.equal(m1, m2)
    assert torch.equal(c1.values, c2.values) and torch.equal(c1.filled, c2.filled)


# A <= 8000 and short segments take the one-pass region writer (the segment's
# keys and per-address run bounds in LDS); A = 20000 the fill-then-scatter
# path.  D = 3 fp32 rows are 12 bytes (4-byte units).
@pytest.mark.parametrize("k,masked,A,D,dtype", [
    (1, False, 37, 8, torch.bfloat16), (4, False, 37, 8, torch.bfloat16),
    (3, True, 37, 8, torch.bfloat16), (2, True, 4099, 3, torch.float32),
    (4, False, 20000, 8, torch.bfloat16)])
def test_prefill_matches_sequential_writes(device, k, masked, A, D, dtype):
    g = torch.Generator().manual_seed(20 + k)
    B, T, C = 3, 500, 4
    w = torch.randint(-5, A + 5, (B, T, C), generator=g)
    p = torch.randn(B, T, C, D, generator=g).to(dtype)
    m = (torch.rand(B, T, generator=g) < 0.7) if masked else None
    cache = RavelLayerCache.prefill(w.to(device), p.to(device), address_space=A, k=k,
                                    write_mask=None if m is None else m.to(device))
    vals, filled = oracle.cache_prefill(w, p, address_space=A, k=k, write_mask=m)
    if k == 1:
        vals, filled = vals[..., 0, :], filled[..., 0]
    assert torch.equal(cache.filled.cpu(), filled)
    assert torch.equal(cache.values.cpu(), vals)


def test_cfg5_prefill_and_steps_reduced_batch(device):
    """cfg5 shape with B=16 streams: prefill from T=2048, then 64 fused steps,
    checked against the oracle's replay of the same writes."""
    d = workloads.cfg5(device, B=16, T=2048, steps=64)
    cache = RavelLayerCache.prefill(d.prefill_write, d.prefill_payload, address_space=d.address_space, k=d.k)
    for s in range(d.step_read.shape[0]):
        cache.step(d.step_read[s], d.step_write[s], d.step_payload[s])
    w_all = torch.cat([d.prefill_write, d.step_write.permute(1, 0, 2)], dim=1)
    p_all = torch.cat([d.prefill_payload, d.step_payload.permute(1, 0, 2, 3)], dim=1)
    vals, filled = oracle.cache_prefill(w_all, p_all, address_space=d.address_space, k=d.k)
    assert torch.equal(cache.filled.cpu(), filled)
    assert torch.equal(cache.values.cpu(), vals)


def test_cfg5_full_size(device):
    """cfg5 at its stated size: a [256, 8, 4096, 4, 64] bf16 cache (2^32 bytes,
    where 32-bit offset arithmetic would wrap) prefilled from T = 2048, then all
    1024 fused read-then-write steps.  The final cache against the oracle's
    sequential replay of all 2048 + 1024 writes; the reads of the first, middle
    and last steps against the oracle's latest-k sources over the prefix the
    read sees (the writes before it; a step's own write comes after its read)."""
    d = workloads.cfg5(device)
    B, T, C, D = d.prefill_payload.shape
    S = d.step_read.shape[0]
    A, k = d.address_space, d.k
    print(f"[cfg5 full] B={B} T={T} C={C} A={A} k={k} D={D} steps={S}", flush=True)
    cache = RavelLayerCache.prefill(d.prefill_write, d.prefill_payload, address_space=A, k=k)
    assert cache.values.numel() * cache.values.element_size() == 1 << 32
    checked = {0: None, S // 2: None, S - 1: None}
    for s in range(S):
        vals, mask = cache.step(d.step_read[s], d.step_write[s], d.step_payload[s])
        if s in checked:
            checked[s] = (vals.cpu(), mask.cpu())
    torch.cuda.synchronize()
    w_all = torch.cat([d.prefill_write, d.step_write.permute(1, 0, 2)], dim=1).cpu()
    p_all = torch.cat([d.prefill_payload, d.step_payload.permute(1, 0, 2, 3)], dim=1).cpu()
    rows = p_all.reshape(-1, D)
    for s, (vals, mask) in checked.items():
        tp = T + s + 1  # the read sits at time T + s, after the writes before it
        r = w_all[:, :tp].clone()
        r[:, T + s] = d.step_read[s].cpu()
        src = oracle.latest_k_src(w_all[:, :tp], r, address_space=A, k=k)[:, T + s]  # [B, C, k]
        s64 = torch.from_numpy(src.astype("int64"))
        # src indexes the [B, tp, C] prefix tape; map it to rows of p_all
        b_i, rem = s64 // (tp * C), s64 % (tp * C)
        flat = (b_i * (T + S) * C + rem).clamp_min(0)
        want = rows.index_select(0, flat.view(-1)).view(B, C, k, D)
        want = torch.where((s64 >= 0).unsqueeze(-1), want, torch.zeros((), dtype=want.dtype))
        assert torch.equal(mask, s64 >= 0), f"step {s} mask"
        assert torch.equal(vals, want), f"step {s} values"
        print(f"[cfg5 full] step {s} reads match", flush=True)
    ov, of = oracle.cache_prefill(w_all, p_all, address_space=A, k=k)
    assert torch.equal(cache.filled.cpu(), of)
    assert torch.equal(cache.values.cpu(), ov)
    print("[cfg5 full] final cache matches the replay", flush=True)


@pytest.mark.parametrize("B,C", [(0, 4), (3, 0)])
def test_prefill_without_streams_clears_status(device, B, C):
    """A prefill with no streams launches no sort, yet leaves a clear status word
    in a workspace that held garbage (and the Python call passes its check)."""
    from ravel_em import _native as nat

    lib = nat.library()
    T, A, D, k = 5, 7, 8, 2
    w = torch.zeros(B, T, C, dtype=torch.long, device=device)
    p = torch.zeros(B, T, C, D, dtype=torch.bfloat16, device=device)
    vals = torch.empty(B, C, A, k, D, dtype=torch.bfloat16, device=device)
    filled = torch.empty(B, C, A, k, dtype=torch.bool, device=device)
    nbytes = lib.ravel_em_cache_prefill_workspace(B, T, C, A, 0)
    ws = torch.full((max(int(nbytes), 256),), 0xFF, dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    nat.check(lib.ravel_em_cache_prefill(w.data_ptr(), nat.INT64, None, p.data_ptr(), nat.BFLOAT16,
                                         B, T, C, D, A, k, vals.data_ptr(), filled.data_ptr(),
                                         ws.data_ptr(), ws.numel(), stream))
    assert nat.status_word(ws) == 0
    cache = RavelLayerCache.prefill(w, p, address_space=A, k=k)
    assert cache.values.shape == (B, C, A, k, D)
