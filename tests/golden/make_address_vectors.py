"""Write tests/golden/address_vectors.json: input/output vectors of the
reference's address producers, computed by the reference itself on the CPU.

literal_addresses_from_tokens (ravel_lm/model.py:195-231), its decode-step form
literal_addresses_step (:234-263) and the product-code decode
(ProductCodeAddressor, model.py:150-187; RavelMemoryLayer._decode_codes,
model.py:303-307) have no known-answer test in the reference's own suite, so
this script imports ravel_lm.model from a reference checkout (in the build
container only; the fixture, not the reference, travels with the tests) and
records what those functions return for small seeded inputs, including int64
overflow, negative ids, ties, signed zeros, infinities and NaN in the logits.

Run: python tests/golden/make_address_vectors.py [/root/reference]
"""
import json
import math
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "address_vectors.json")


def _floats(t):
    def enc(v):
        if math.isnan(v):
            return "nan"
        if math.isinf(v):
            return "inf" if v > 0 else "-inf"
        if v == 0.0 and math.copysign(1.0, v) < 0:
            return "-0"
        return v
    return [enc(v) for v in t.float().reshape(-1).tolist()]


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from ravel_lm.model import (ProductCodeAddressor, RavelMemoryLayer,  # noqa: E402
                                literal_addresses_from_tokens, literal_addresses_step)

    g = torch.Generator().manual_seed(2024)
    literal = []
    token_cases = [
        ("uniform", torch.randint(0, 300, (2, 9), generator=g), 512, 6, 257),
        ("odd_space", torch.randint(0, 1024, (3, 7), generator=g), 7, 5, 257),
        ("unit_space", torch.randint(0, 50, (1, 4), generator=g), 1, 4, 3),
        ("large_space", torch.randint(0, 1 << 20, (2, 6), generator=g), (1 << 31) + 11, 8, 257),
        ("min_length", torch.tensor([[4, 9]]), 97, 3, 257),
        ("two_heads_t1", torch.tensor([[11], [12]]), 97, 2, 5),
        ("negative_ids", torch.tensor([[-5, 3, -1000, 7, -2]]), 61, 6, 257),
        ("int64_wrap", torch.tensor([[1 << 50, (1 << 49) + 3, 1 << 48, 7, (1 << 62) - 1]]),
         1000003, 7, 257),
        ("bos_minus_one", torch.randint(0, 256, (2, 5), generator=g), 4096, 4, -1),
    ]
    for name, toks, A, H, bos in token_cases:
        out = literal_addresses_from_tokens(toks, address_space=A, n_heads=H, bos_token_id=bos)
        literal.append({"name": name, "tokens": toks.tolist(), "address_space": A, "n_heads": H,
                        "bos_token_id": bos, "addresses": out.tolist()})

    step = []
    def ri(hi, shape):
        return torch.randint(0, hi, shape, generator=g)

    step_cases = [  # name, token ids [B], history [B, h], position, A, heads, bos
        ("history2", ri(300, (4,)), ri(300, (4, 2)), 0, 512, 6, 257),
        ("history2_pos", ri(300, (4,)), ri(300, (4, 2)), 777, 1000, 8, 257),
        ("history_empty", ri(50, (3,)), torch.zeros(3, 0, dtype=torch.long), 0, 97, 4, 257),
        ("history1", ri(50, (3,)), ri(50, (3, 1)), 3, 97, 5, 11),
        ("history3", ri(50, (2,)), ri(50, (2, 3)), 12, 61, 7, 257),
        ("large_position", ri(1 << 20, (2,)), ri(1 << 20, (2, 2)), (1 << 40) + 3, (1 << 31) + 11, 9, 257),
        ("bos_history", torch.full((2,), 5), torch.full((2, 2), 257), 1, 4096, 3, 257),
    ]
    for name, toks, hist, pos, A, H, bos in step_cases:
        out = literal_addresses_step(toks, hist, address_space=A, n_heads=H, position=pos,
                                     bos_token_id=bos)
        step.append({"name": name, "tokens": toks.tolist(), "history": hist.tolist(),
                     "history_len": int(hist.shape[1]), "position": pos, "address_space": A,
                     "n_heads": H, "bos_token_id": bos, "addresses": out.tolist()})

    codes = []
    code_cases = []
    x = torch.randn(2, 5, 3 * 2 * 8, generator=g)
    code_cases.append(("normal_f32", x, 3, 2, 8, 50))
    lv = torch.randint(0, 3, (2, 4, 2 * 2 * 16), generator=g).float().to(torch.bfloat16)
    code_cases.append(("ties_bf16", lv, 2, 2, 16, 256))
    sp = torch.randn(1, 6, 2 * 3 * 4, generator=g)
    sp[0, 0, 1] = float("nan")                       # NaN beats a larger number
    sp[0, 1, 2] = float("nan")
    sp[0, 1, 3] = float("nan")                       # first of two NaNs
    sp[0, 2, 0:4] = torch.tensor([0.0, -0.0, -1.0, -0.0])  # signed-zero tie
    sp[0, 3, 4:8] = torch.tensor([-0.0, 0.0, -2.0, -3.0])
    sp[0, 4, 8:12] = float("-inf")                   # all -inf
    sp[0, 5, 12:16] = torch.tensor([1.0, float("inf"), float("inf"), 2.0])
    code_cases.append(("specials_f32", sp, 2, 3, 4, 64))
    code_cases.append(("specials_f16", sp.to(torch.float16), 2, 3, 4, 7))
    code_cases.append(("one_codebook", torch.randn(3, 2, 4 * 1 * 32, generator=g), 4, 1, 32, 20))
    for name, lg, H, ncb, cbs, A in code_cases:
        addressor = ProductCodeAddressor(1, H, ncb, cbs, A)
        out = RavelMemoryLayer._decode_codes(None, addressor, lg)
        codes.append({"name": name, "dtype": str(lg.dtype).split(".")[-1], "shape": list(lg.shape),
                      "logits": _floats(lg), "n_heads": H, "n_codebooks": ncb,
                      "codebook_size": cbs, "address_space": A, "addresses": out.tolist()})

    doc = {
        "source": "ravel_lm/model.py:195-231 (literal_addresses_from_tokens), :234-263 "
                  "(literal_addresses_step), "
                  ":150-187 + :303-307 (product-code decode), evaluated by the reference on the CPU",
        "generator": "tests/golden/make_address_vectors.py",
        "literal": literal,
        "literal_step": step,
        "product_codes": codes,
    }
    with open(OUT, "w") as f:
        json.dump(doc, f, indent=1)
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
