"""Address production without a GPU: the CPU oracle against the reference's own
outputs (tests/golden/address_vectors.json, written by the reference's
functions), planted mistakes that those vectors catch, the descriptor's C
layout, and descriptor checks of the C ABI that fail before any launch."""
import ctypes
import json
import math
import os
import subprocess

import pytest

from oracle import addresses as oa
from ravel_em import _native as nat

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
VEC = json.load(open(os.path.join(ROOT, "tests", "golden", "address_vectors.json")))


def decode(values):
    special = {"nan": math.nan, "inf": math.inf, "-inf": -math.inf, "-0": -0.0}
    return [special[v] if isinstance(v, str) else float(v) for v in values]


def rows_of(case):
    vals = decode(case["logits"])
    n = case["shape"][-1]
    return [vals[i:i + n] for i in range(0, len(vals), n)]


def flat(x):
    if isinstance(x, list):
        return [y for e in x for y in flat(e)]
    return [x]


@pytest.mark.parametrize("case", VEC["literal"], ids=lambda c: c["name"])
def test_literal_oracle_matches_reference_outputs(case):
    got = oa.literal_addresses(case["tokens"], address_space=case["address_space"],
                               n_heads=case["n_heads"], bos_token_id=case["bos_token_id"])
    assert got == case["addresses"]


@pytest.mark.parametrize("case", VEC["product_codes"], ids=lambda c: c["name"])
def test_product_code_oracle_matches_reference_outputs(case):
    got = oa.product_codes(rows_of(case), n_heads=case["n_heads"], n_codebooks=case["n_codebooks"],
                           codebook_size=case["codebook_size"], address_space=case["address_space"])
    assert flat(got) == flat(case["addresses"])


def test_layer_assembly_is_literal_then_learned():
    lit = VEC["literal"][0]
    pc = VEC["product_codes"][0]  # [2, 5, 3*2*8] logits
    B, T = 2, 5
    tokens = [row[:T] for row in lit["tokens"]]
    rows = rows_of(pc)
    lg = [rows[b * T:(b + 1) * T] for b in range(B)]
    rg = [[list(reversed(r)) for r in rr] for rr in lg]
    w, r = oa.layer_addresses(tokens, lg, rg, address_space=50, n_literal=2, bos_token_id=257,
                              n_learned=3, n_codebooks=2, codebook_size=8, B=B, T=T)
    lit2 = oa.literal_addresses(tokens, address_space=50, n_heads=2, bos_token_id=257)
    codes_w = [oa.product_codes(lg[b], n_heads=3, n_codebooks=2, codebook_size=8, address_space=50)
               for b in range(B)]
    codes_r = [oa.product_codes(rg[b], n_heads=3, n_codebooks=2, codebook_size=8, address_space=50)
               for b in range(B)]
    for b in range(B):
        for t in range(T):
            assert w[b][t] == lit2[b][t] + codes_w[b][t]
            assert r[b][t] == lit2[b][t] + codes_r[b][t]
    w2, r2 = oa.layer_addresses(tokens, lg, None, address_space=50, n_literal=2, bos_token_id=257,
                                n_learned=3, n_codebooks=2, codebook_size=8, B=B, T=T)
    assert r2 is w2


# ---- planted mistakes (in oracle variants, on the CPU): the vectors catch each


def _literal_variant(tokens, A, H, bos, *, big_ints=False, c1=131, prev_pad=None, pos_shift=0):
    out = []
    for row in tokens:
        orow = []
        for t, x in enumerate(row):
            pad = bos if prev_pad is None else prev_pad
            p1 = row[t - 1] if t >= 1 else pad
            p2 = row[t - 2] if t >= 2 else pad
            hs = []
            for j in range(H):
                h = [x, p1 * 257 + x * c1 + 17, p2 * 65537 + p1 * 257 + x * c1 + 31][j] if j < 3 else \
                    x * (1009 + 2 * j) + (t + pos_shift) * (9176 + j) + j * 97
                hs.append((h if big_ints else oa._i64(h)) % A)
            orow.append(hs)
        out.append(orow)
    return out


def _argmax_variant(v, *, last_max=False, skip_nan=False):
    best, bi = None, 0
    for i, x in enumerate(v):
        if skip_nan and math.isnan(x):
            continue
        if best is None or (x >= best if last_max else (x > best or math.isnan(x))):
            if best is not None and math.isnan(best) and not last_max:
                break
            best, bi = x, i
    return bi


def test_planted_literal_mistakes_are_caught():
    cases = VEC["literal"]

    def caught(**kw):
        return any(_literal_variant(c["tokens"], c["address_space"], c["n_heads"],
                                    c["bos_token_id"], **kw) != c["addresses"] for c in cases)

    assert not caught()  # the unmutated variant agrees
    assert caught(big_ints=True)      # no int64 wrap
    assert caught(c1=137)             # wrong multiplier
    assert caught(prev_pad=0)         # zero instead of bos before the start
    assert caught(pos_shift=1)        # 1-based positions


def test_planted_argmax_mistakes_are_caught():
    def codes(case, **kw):
        H, Q, S, A = case["n_heads"], case["n_codebooks"], case["codebook_size"], case["address_space"]
        out = []
        for row in rows_of(case):
            for h in range(H):
                addr, m = 0, 1
                for q in range(Q):
                    lo = (h * Q + q) * S
                    addr += _argmax_variant(row[lo:lo + S], **kw) * m
                    m *= S
                out.append(addr % A)
        return out

    cases = VEC["product_codes"]
    assert all(codes(c) == flat(c["addresses"]) for c in cases)
    assert any(codes(c, last_max=True) != flat(c["addresses"]) for c in cases)
    assert any(codes(c, skip_nan=True) != flat(c["addresses"]) for c in cases)


# ---- the C descriptor and the ABI's checks of it


def test_descriptor_layout_matches_the_c_header(tmp_path):
    fields = [f for f, _ in nat.AddrGen._fields_]
    prog = tmp_path / "layout.c"
    body = "".join(f'  printf("%zu ", offsetof(ravel_em_addr_gen, {f}));\n' for f in fields)
    prog.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "ravel_em.h"\nint main(void) {\n'
                    + body + '  printf("%zu\\n", sizeof(ravel_em_addr_gen));\n  return 0;\n}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", os.path.join(ROOT, "include"), str(prog), "-o", str(exe)],
                   check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True,
                                          check=True).stdout.split()]
    want = [getattr(nat.AddrGen, f).offset for f in fields] + [ctypes.sizeof(nat.AddrGen)]
    assert got == want


def _err():
    return nat.library().ravel_em_last_error().decode()


def _call_latest_k(desc, C=3):
    lib = nat.library()
    fake = 256  # never dereferenced: the descriptor check fails before any launch
    return lib.ravel_em_latest_k_fwd(nat.ref(desc), None, nat.ADDR_GEN, None, fake, nat.FLOAT32,
                                     2, 4, C, 8, 16, 1, fake, fake, None, fake, 1 << 30, None)


def test_descriptor_errors_fail_before_launch():
    g = nat.AddrGen()
    g.n_literal, g.n_learned = 2, 0
    g.tokens, g.token_dtype = 256, nat.INT64
    assert _call_latest_k(g, C=3) == 1 and "heads" in _err()
    g.tokens = None
    assert _call_latest_k(g, C=2) == 1 and "tokens" in _err()
    g.tokens, g.token_dtype = 256, nat.FLOAT32
    assert _call_latest_k(g, C=2) == 1 and "token ids" in _err()
    h = nat.AddrGen()
    h.n_learned, h.n_codebooks, h.codebook_size = 2, 2, 4
    assert _call_latest_k(h, C=2) == 1 and "logits" in _err()
    h.logits, h.logits_dtype = 256, nat.INT64
    assert _call_latest_k(h, C=2) == 1 and "logits must be" in _err()
    h.logits_dtype, h.codebook_size = nat.BFLOAT16, 0
    assert _call_latest_k(h, C=2) == 1 and "codebook_size" in _err()
    h.codebook_size, h.n_codebooks = 1 << 20, 4
    assert _call_latest_k(h, C=2) == 1 and "2^62" in _err()
    lib = nat.library()
    assert lib.ravel_em_addresses(None, 1, 1, 4, nat.INT64, 256, None) == 1
    ok = nat.AddrGen()
    ok.n_literal, ok.tokens, ok.token_dtype = 1, 256, nat.INT64
    assert lib.ravel_em_addresses(nat.ref(ok), 1, 1, 4, nat.FLOAT32, 256, None) == 1
    assert "int32 or int64" in _err()
    # the decode cache's read/write/step take address tensors only
    rc = lib.ravel_em_cache_read(256, 256, nat.ref(ok), nat.ADDR_GEN, nat.BFLOAT16, 1, 1, 4, 1, 8,
                                 256, 256, None)
    assert rc == 1 and "address dtype" in _err()


def test_torch_restatement_matches_reference_outputs():
    """The CPU baseline's address ops (oracle/torch_ref.py) against the same vectors."""
    import torch

    from oracle import torch_ref

    for case in VEC["literal"]:
        got = torch_ref.literal_addresses(torch.tensor(case["tokens"]), address_space=case["address_space"],
                                          n_heads=case["n_heads"], bos_token_id=case["bos_token_id"])
        assert got.tolist() == case["addresses"], case["name"]
    for case in VEC["product_codes"]:
        dtype = getattr(torch, case["dtype"])
        lg = torch.tensor(decode(case["logits"])).to(dtype).view(case["shape"])
        got = torch_ref.product_codes(lg, n_heads=case["n_heads"], n_codebooks=case["n_codebooks"],
                                      codebook_size=case["codebook_size"],
                                      address_space=case["address_space"])
        assert got.tolist() == case["addresses"], case["name"]


@pytest.mark.parametrize("case", VEC["literal_step"], ids=lambda c: c["name"])
def test_literal_step_oracle_matches_reference_outputs(case):
    hist = case["history"] if case["history_len"] > 0 else [[] for _ in case["tokens"]]
    got = oa.literal_addresses_step(case["tokens"], hist, address_space=case["address_space"],
                                    n_heads=case["n_heads"], position=case["position"],
                                    bos_token_id=case["bos_token_id"])
    assert got == case["addresses"]


def test_step_equals_sequence_at_its_position():
    """Invariant linking the two reference functions: the step at time t with
    the previous two tokens as history gives row t of the whole sequence."""
    case = VEC["literal"][0]
    A, H, bos = case["address_space"], case["n_heads"], case["bos_token_id"]
    for b, row in enumerate(case["tokens"]):
        for t in range(len(row)):
            hist = [[(row[t - 2] if t >= 2 else bos), (row[t - 1] if t >= 1 else bos)]]
            got = oa.literal_addresses_step([row[t]], hist, address_space=A, n_heads=H,
                                            position=t, bos_token_id=bos)
            assert got[0] == case["addresses"][b][t]
