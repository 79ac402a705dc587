"""GPU parity of address production inside the kernels.

* The address kernel (literal_addresses_from_tokens, product_code_addresses)
  against the reference's own outputs (tests/golden/address_vectors.json) and
  against the CPU oracle (oracle/addresses.py) on seeded inputs, through the
  vectorized and the element-wise logit paths and through strided views.
* Lookups given a LayerAddresses (addresses produced in the key build and the
  read search) against the same lookups given the materialized address
  tensors, and their sources against the oracle: bit-exact, as integer work.
"""
import json
import math
import os

import numpy as np
import pytest
import torch

import oracle
from oracle import addresses as oa
from ravel_em import (LayerAddresses, causal_last_k_lookup, causal_last_k_sources,
                      causal_sum_lookup, fused_latest1_linear, literal_addresses_from_tokens,
                      product_code_addresses)

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
VEC = json.load(open(os.path.join(HERE, "golden", "address_vectors.json")))


def decode(values):
    special = {"nan": math.nan, "inf": math.inf, "-inf": -math.inf, "-0": -0.0}
    return [special[v] if isinstance(v, str) else float(v) for v in values]


@pytest.mark.parametrize("case", VEC["literal"], ids=lambda c: c["name"])
def test_literal_kernel_matches_reference_outputs(device, case):
    toks = torch.tensor(case["tokens"], dtype=torch.int64, device=device)
    got = literal_addresses_from_tokens(toks, address_space=case["address_space"],
                                        n_heads=case["n_heads"], bos_token_id=case["bos_token_id"])
    assert got.dtype == torch.int64
    assert got.cpu().tolist() == case["addresses"]
    if toks.abs().max().item() < 2**31:
        got32 = literal_addresses_from_tokens(toks.int(), address_space=case["address_space"],
                                              n_heads=case["n_heads"],
                                              bos_token_id=case["bos_token_id"])
        assert got32.cpu().tolist() == case["addresses"]


@pytest.mark.parametrize("case", VEC["product_codes"], ids=lambda c: c["name"])
def test_product_code_kernel_matches_reference_outputs(device, case):
    dtype = getattr(torch, case["dtype"])
    lg = torch.tensor(decode(case["logits"]), dtype=torch.float32).to(dtype).view(case["shape"])
    got = product_code_addresses(lg.to(device), n_heads=case["n_heads"],
                                 n_codebooks=case["n_codebooks"],
                                 codebook_size=case["codebook_size"],
                                 address_space=case["address_space"])
    assert got.cpu().tolist() == case["addresses"]


def test_literal_kernel_random_strided_vs_oracle(device):
    g = torch.Generator().manual_seed(31)
    base = torch.randint(-50, 70000, (3, 2 * 301), generator=g)
    toks = base.to(device)[:, ::2]  # a strided view: the kernel reads through the strides
    for A, H, bos in ((1000, 7, 257), (65536, 3, 0), (13, 9, 257)):
        got = literal_addresses_from_tokens(toks, address_space=A, n_heads=H, bos_token_id=bos)
        want = oa.literal_addresses(base[:, ::2].tolist(), address_space=A, n_heads=H,
                                    bos_token_id=bos)
        assert got.cpu().tolist() == want


# (lead shape, heads, codebooks, codebook size, A, dtype, slice of a wider packed row)
CODE_CASES = [
    ((3, 200), 4, 2, 16, 256, torch.bfloat16, False),   # 16-byte units (vector path)
    ((2, 150), 3, 3, 5, 97, torch.bfloat16, False),     # element-wise path
    ((2, 170), 2, 2, 64, 4096, torch.float32, True),    # slice of a packed projection
    ((4, 90), 8, 2, 8, 64, torch.float16, True),
    ((5, 33), 2, 2, 12, 100, torch.float32, False),     # f32, 16-byte-aligned row pieces of 3 units
]


@pytest.mark.parametrize("case", CODE_CASES)
def test_product_code_kernel_random_vs_oracle(device, case):
    lead, H, Q, S, A, dtype, packed = case
    g = torch.Generator().manual_seed(100 + CODE_CASES.index(case))
    n = H * Q * S
    # few distinct levels: many ties, which the first-maximum rule must break
    lg = (torch.randint(0, 4, (*lead, n), generator=g).float() * 0.5).to(dtype)
    lg.view(-1)[::37] = float("nan")
    if packed:
        wide = torch.zeros(*lead, n + 24, dtype=dtype)
        wide[..., 8:8 + n] = lg
        dev_lg = wide.to(device)[..., 8:8 + n]
    else:
        dev_lg = lg.to(device)
    got = product_code_addresses(dev_lg, n_heads=H, n_codebooks=Q, codebook_size=S,
                                 address_space=A)
    rows = lg.float().reshape(-1, n).tolist()
    want = oa.product_codes(rows, n_heads=H, n_codebooks=Q, codebook_size=S, address_space=A)
    assert got.cpu().reshape(-1, H).tolist() == want


# ------------------------------------------------- lookups given sources --


def make_source(device, B, T, n_lit, n_learned, Q, S, separate, dtype=torch.bfloat16, seed=5):
    g = torch.Generator().manual_seed(seed)
    toks = torch.randint(0, 40, (B, T), generator=g).to(device)
    wl = rl = None
    if n_learned:
        n = n_learned * Q * S
        # the layer slices write/read logits out of one packed projection (model.py:335-341)
        packed = torch.randn(B, T, 16 + 2 * n, generator=g).to(dtype).to(device)
        wl, rl = packed[..., 16:16 + n], packed[..., 16 + n:]
    return LayerAddresses(toks, n_lit, 257, wl, rl if separate else None, n_learned, Q, S)


LOOKUP_CASES = [
    # B, T, literal, learned, Q, S, separate reads, A, k, masked
    (2, 300, 2, 0, 2, 16, False, 61, 1, False),    # literal only: reads == writes (link path)
    (2, 300, 4, 0, 2, 16, False, 61, 3, False),
    (3, 257, 2, 1, 2, 16, True, 97, 1, False),     # the reference's 2 literal + 1 learned layer
    (2, 500, 2, 2, 2, 8, True, 64, 4, True),
    (1, 700, 0, 3, 2, 16, True, 256, 2, False),    # learned only
    (2, 400, 1, 2, 3, 5, False, 50, 1, True),      # learned, reads == writes, element-wise logits
    (2, 20000, 2, 1, 2, 16, True, 1000, 2, False), # segments past the LDS search
]


@pytest.mark.parametrize("case", LOOKUP_CASES)
def test_latest_k_with_layer_addresses(device, case):
    B, T, n_lit, n_learned, Q, S, separate, A, k, masked = case
    src = make_source(device, B, T, n_lit, n_learned, Q, S, separate)
    C = src.heads
    g = torch.Generator().manual_seed(11)
    payload = torch.randn(B, T, C, 8, generator=g).to(device)
    mask = (torch.rand(B, T, generator=g) < 0.8).to(device) if masked else None
    w, r = src.materialize(address_space=A)
    read = None if src.same else r
    v1, m1, s1 = causal_last_k_sources(src, payload, address_space=A, k=k, write_mask=mask)
    v2, m2, s2 = causal_last_k_sources(w, payload, read, address_space=A, k=k, write_mask=mask)
    assert torch.equal(s1, s2) and torch.equal(m1, m2) and torch.equal(v1, v2)
    v3, m3 = causal_last_k_lookup(src, payload, address_space=A, k=k, write_mask=mask)
    assert torch.equal(v3, v1) and torch.equal(m3, m1)
    if B * T * C <= 20000:
        lg = lambda x: None if x is None else x.float().cpu().tolist()  # noqa: E731
        ow, orr = oa.layer_addresses(src.token_ids.cpu().tolist(), lg(src.write_logits),
                                     lg(src.read_logits), address_space=A, n_literal=n_lit,
                                     bos_token_id=257, n_learned=n_learned, n_codebooks=Q,
                                     codebook_size=S, B=B, T=T)
        assert w.cpu().tolist() == ow and r.cpu().tolist() == orr
        osrc = oracle.latest_k_src(torch.tensor(ow), None if src.same else torch.tensor(orr),
                                   address_space=A, k=k, write_mask=mask)
        assert np.array_equal(s1.cpu().numpy(), osrc)


@pytest.mark.parametrize("case", LOOKUP_CASES[:6])
def test_seg_sum_with_layer_addresses(device, case):
    B, T, n_lit, n_learned, Q, S, separate, A, _, masked = case
    src = make_source(device, B, T, n_lit, n_learned, Q, S, separate)
    g = torch.Generator().manual_seed(12)
    payload = torch.randn(B, T, src.heads, 8, generator=g).to(device)
    mask = (torch.rand(B, T, generator=g) < 0.8).to(device) if masked else None
    w, r = src.materialize(address_space=A)
    s1, m1 = causal_sum_lookup(src, payload, address_space=A, write_mask=mask)
    s2, m2 = causal_sum_lookup(w, payload, None if src.same else r, address_space=A, write_mask=mask)
    assert torch.equal(m1, m2) and torch.equal(s1, s2)


@pytest.mark.parametrize("case", [(2, 300, 2, 0, False), (2, 257, 2, 1, True), (1, 400, 0, 2, True)])
def test_gradients_with_layer_addresses(device, case):
    B, T, n_lit, n_learned, separate = case
    src = make_source(device, B, T, n_lit, n_learned, 2, 16, separate)
    A = 61
    g = torch.Generator().manual_seed(13)
    base = torch.randn(B, T, src.heads, 8, generator=g).to(device)
    w, r = src.materialize(address_space=A)
    read = None if src.same else r
    grads = []
    for addr, rd in ((src, None), (w, read)):
        p = base.clone().requires_grad_(True)
        v, _ = causal_last_k_lookup(addr, p, rd, address_space=A, k=2)
        s, _ = causal_sum_lookup(addr, p, rd, address_space=A)
        (v.square().sum() + (s * 0.5).sum()).backward()
        grads.append(p.grad)
    torch.testing.assert_close(grads[0], grads[1], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("case", [(2, 300, 2, 0, False, 64), (2, 257, 2, 1, True, 192),
                                  (1, 300, 2, 1, True, 20)])
def test_fused_linear_with_layer_addresses(device, case):
    B, T, n_lit, n_learned, separate, M = case
    src = make_source(device, B, T, n_lit, n_learned, 2, 16, separate)
    A, P = 97, 16
    g = torch.Generator().manual_seed(14)
    payload = torch.randn(B, T, src.heads, P, generator=g).to(torch.bfloat16).to(device)
    weight = (torch.randn(M, src.heads * P, generator=g) * 0.1).to(torch.bfloat16).to(device)
    w, r = src.materialize(address_space=A)
    out1 = fused_latest1_linear(src, payload, None, weight, address_space=A)
    out2 = fused_latest1_linear(w, payload, None if src.same else r, weight, address_space=A)
    assert torch.equal(out1, out2)
    p1 = payload.clone().requires_grad_(True)
    w1 = weight.clone().requires_grad_(True)
    fused_latest1_linear(src, p1, None, w1, address_space=A).float().sum().backward()
    p2 = payload.clone().requires_grad_(True)
    w2 = weight.clone().requires_grad_(True)
    fused_latest1_linear(w, p2, None if src.same else r, w2, address_space=A).float().sum().backward()
    torch.testing.assert_close(p1.grad.float(), p2.grad.float(), rtol=1e-2, atol=1e-2)
    torch.testing.assert_close(w1.grad.float(), w2.grad.float(), rtol=1e-2, atol=1e-2)


def test_cfg3_shaped_lookup_from_logits(device):
    """The product-code configuration (two 64-way codebooks, A = 4096) at a
    reduced batch: addresses decoded by torch.argmax on the CPU (the
    reference's decode), then the tensor lookup, against the lookup that
    decodes the logits itself."""
    B, T, H, Q, S, A = 2, 4096, 8, 2, 64, 4096
    g = torch.Generator().manual_seed(1003)
    wl = torch.randn(B, T, H * Q * S, generator=g).to(torch.bfloat16)
    rl = torch.randn(B, T, H * Q * S, generator=g).to(torch.bfloat16)
    mult = torch.tensor([1, S])

    def decode_cpu(lg):
        codes = lg.reshape(B, T, H, Q, S).argmax(-1)
        return (codes * mult).sum(-1).remainder(A)

    w, r = decode_cpu(wl).to(device), decode_cpu(rl).to(device)
    src = LayerAddresses(None, 0, 257, wl.to(device), rl.to(device), H, Q, S)
    payload = torch.randn(B, T, H, 64, generator=g).to(torch.bfloat16).to(device)
    v1, m1, s1 = causal_last_k_sources(src, payload, address_space=A, k=4)
    v2, m2, s2 = causal_last_k_sources(w, payload, r, address_space=A, k=4)
    assert torch.equal(s1, s2) and torch.equal(v1, v2) and torch.equal(m1, m2)
    wm, rm = src.materialize(address_space=A)
    assert torch.equal(wm, w) and torch.equal(rm, r)


# ------------------------------------------------------------ decode step --


@pytest.mark.parametrize("case", VEC["literal_step"], ids=lambda c: c["name"])
def test_literal_step_kernel_matches_reference_outputs(device, case):
    from ravel_em import literal_addresses_step

    toks = torch.tensor(case["tokens"], dtype=torch.int64, device=device)
    B = toks.shape[0]
    hist = torch.tensor(case["history"], dtype=torch.int64).view(B, case["history_len"]).to(device)
    got = literal_addresses_step(toks, hist, address_space=case["address_space"],
                                 n_heads=case["n_heads"], position=case["position"],
                                 bos_token_id=case["bos_token_id"])
    assert got.cpu().tolist() == case["addresses"]


def test_chunked_prefill_with_history(device):
    """A later chunk with the two tokens before it as history and its start as
    position gives the addresses of the whole sequence at those times."""
    g = torch.Generator().manual_seed(41)
    toks = torch.randint(0, 500, (3, 200), generator=g).to(device)
    full = literal_addresses_from_tokens(toks, address_space=1000, n_heads=7, bos_token_id=257)
    for t0 in (1, 2, 77):
        src = LayerAddresses(toks[:, t0:], 7, 257, token_history=toks[:, max(0, t0 - 2):t0],
                             position=t0)
        got, _ = src.materialize(address_space=1000)
        assert torch.equal(got, full[:, t0:])


def test_decode_steps_with_produced_addresses_match_the_full_lookup(device):
    """RavelMemoryLayer's decode (model.py:401-426, history update :574) with
    the step's addresses produced in the cache kernel, against the latest-1
    lookup of the whole sequence with its addresses produced in the sort
    (the reference's stepwise == full check, tests/test_model.py:78-90)."""
    from ravel_em import RavelLayerCache

    B, T, n_lit, H, Q, S, A, D, bos = 2, 40, 3, 2, 2, 8, 97, 8, 257
    g = torch.Generator().manual_seed(43)
    toks = torch.randint(0, 60, (B, T), generator=g).to(device)
    packed = torch.randn(B, T, 2 * H * Q * S, generator=g).to(torch.bfloat16).to(device)
    wl, rl = packed[..., :H * Q * S], packed[..., H * Q * S:]
    payload = torch.randn(B, T, n_lit + H, D, generator=g).to(device)
    src = LayerAddresses(toks, n_lit, bos, wl, rl, H, Q, S)
    full_v, full_m = causal_last_k_lookup(src, payload, address_space=A, k=1)
    cache = RavelLayerCache.empty(B, n_lit + H, A, D, device=device, dtype=payload.dtype)
    hist = torch.full((B, 2), bos, dtype=torch.long, device=device)
    for t in range(T):
        step = LayerAddresses(toks[:, t], n_lit, bos, wl[:, t], rl[:, t], H, Q, S,
                              token_history=hist, position=t)
        v, m = cache.step(step, None, payload[:, t])
        assert torch.equal(m, full_m[:, t, :, 0]), t
        assert torch.equal(v, full_v[:, t, :, 0]), t
        hist = torch.cat([hist[:, 1:], toks[:, t:t + 1]], dim=1)


@pytest.mark.parametrize("k", [1, 4])
def test_cache_step_with_produced_addresses_matches_tensor_step(device, k):
    from ravel_em import RavelLayerCache, literal_addresses_step, product_code_addresses

    B, n_lit, H, Q, S, A, D, bos = 8, 2, 3, 2, 16, 300, 16, 257
    C = n_lit + H
    g = torch.Generator().manual_seed(47 + k)
    c1 = RavelLayerCache.empty(B, C, A, D, device=device, dtype=torch.bfloat16, k=k)
    c2 = RavelLayerCache.empty(B, C, A, D, device=device, dtype=torch.bfloat16, k=k)
    hist = torch.randint(0, 300, (B, 2), generator=g).to(device)
    for t in range(12):
        tok = torch.randint(0, 300, (B,), generator=g).to(device)
        wl = torch.randn(B, H * Q * S, generator=g).to(torch.bfloat16).to(device)
        rl = torch.randn(B, H * Q * S, generator=g).to(torch.bfloat16).to(device)
        pay = torch.randn(B, C, D, generator=g).to(torch.bfloat16).to(device)
        lit = literal_addresses_step(tok, hist, address_space=A, n_heads=n_lit, position=t + 5,
                                     bos_token_id=bos)
        kw = dict(n_heads=H, n_codebooks=Q, codebook_size=S, address_space=A)
        w = torch.cat([lit, product_code_addresses(wl, **kw)], dim=-1)
        r = torch.cat([lit, product_code_addresses(rl, **kw)], dim=-1)
        v2, m2 = c2.step(r, w, pay)
        src = LayerAddresses(tok, n_lit, bos, wl, rl, H, Q, S, token_history=hist, position=t + 5)
        v1, m1 = c1.step(src, None, pay)
        assert torch.equal(m1, m2) and torch.equal(v1, v2), t
        hist = torch.cat([hist[:, 1:], tok.view(-1, 1)], dim=1)
    assert torch.equal(c1.values, c2.values) and torch.equal(c1.filled, c2.filled)
