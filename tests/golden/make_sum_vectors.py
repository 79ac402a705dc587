"""Write tests/golden/sum_vectors.json: input/output vectors of the reference's
causal_sum_lookup (ravel_lm/ravel_memory.py:179-241), computed by the
reference itself on the CPU.

The reference's segmented sum rounds a global cumulative sum in the payload
dtype and subtracts the prefix before each segment (:216-224), so its exact
floating-point result is fixed by that arithmetic and not by the mathematics.
Its own suite pins one integer case (tests/test_memory.py:61-67).  This script
imports ravel_lm.ravel_memory from a reference checkout (in the build
container only; the fixture, not the reference, travels with the tests) and
records what causal_sum_lookup returns on small seeded inputs:

  int_*     small integer payloads whose every global prefix is exactly
            representable, so the reference result is exact (bit-exact pin);
  normal_*  Gaussian payloads in fp32 / fp64 / bf16 / fp16 (tolerance pin);
  plus separate read addresses, write masks, an all-masked tape, and
  negative / out-of-range addresses (Python remainder).

Run: python tests/golden/make_sum_vectors.py [/root/reference]
"""
import json
import math
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "sum_vectors.json")


def _floats(t):
    def enc(v):
        if math.isnan(v):
            return "nan"
        if math.isinf(v):
            return "inf" if v > 0 else "-inf"
        if v == 0.0 and math.copysign(1.0, v) < 0:
            return "-0"
        return v
    return [enc(v) for v in t.double().reshape(-1).tolist()]


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from ravel_lm.ravel_memory import causal_sum_lookup  # noqa: E402

    g = torch.Generator().manual_seed(1729)

    def ri(lo, hi, shape):
        return torch.randint(lo, hi, shape, generator=g)

    cases = []  # name, write [B,T,C], read or None, payload [B,T,C,D], A, write_mask or None
    cases.append(("int_f32", ri(0, 5, (2, 33, 3)), None, ri(-3, 4, (2, 33, 3, 4)).float(), 5, None))
    cases.append(("int_f32_reads_mask", ri(0, 6, (2, 40, 2)), ri(0, 6, (2, 40, 2)),
                  ri(-4, 5, (2, 40, 2, 3)).float(), 6, torch.rand(2, 40, generator=g) < 0.7))
    cases.append(("int_bf16", ri(0, 3, (1, 12, 2)), None,
                  ri(-1, 2, (1, 12, 2, 3)).to(torch.bfloat16), 3, None))
    cases.append(("int_f16", ri(0, 4, (2, 20, 2)), ri(0, 4, (2, 20, 2)),
                  ri(-2, 3, (2, 20, 2, 2)).to(torch.float16), 4, None))
    cases.append(("int_f64_wrap", ri(-9, 20, (2, 24, 3)), None,
                  ri(-5, 6, (2, 24, 3, 2)).double(), 7, None))
    cases.append(("normal_f32", ri(0, 7, (2, 64, 2)), None,
                  torch.randn(2, 64, 2, 5, generator=g), 7, None))
    cases.append(("normal_f32_reads_mask", ri(0, 5, (3, 48, 2)), ri(0, 5, (3, 48, 2)),
                  torch.randn(3, 48, 2, 4, generator=g), 5, torch.rand(3, 48, generator=g) < 0.5))
    cases.append(("normal_f64", ri(0, 9, (2, 50, 3)), None,
                  torch.randn(2, 50, 3, 3, generator=g).double(), 9, None))
    cases.append(("normal_bf16", ri(0, 5, (2, 48, 2)), None,
                  torch.randn(2, 48, 2, 4, generator=g).to(torch.bfloat16), 5, None))
    cases.append(("normal_f16", ri(0, 6, (2, 40, 2)), ri(0, 6, (2, 40, 2)),
                  torch.randn(2, 40, 2, 3, generator=g).to(torch.float16), 6, None))
    cases.append(("all_masked", ri(0, 4, (2, 9, 2)), None, torch.randn(2, 9, 2, 3, generator=g), 4,
                  torch.zeros(2, 9, dtype=torch.bool)))
    cases.append(("single_address", torch.zeros(1, 30, 1, dtype=torch.long), None,
                  ri(-2, 3, (1, 30, 1, 2)).float(), 1, None))

    out = []
    for name, w, r, p, A, m in cases:
        s, mask = causal_sum_lookup(w, p, r, address_space=A, write_mask=m)
        out.append({
            "name": name, "dtype": str(p.dtype).split(".")[-1], "shape": list(p.shape),
            "address_space": A, "write": w.tolist(), "read": None if r is None else r.tolist(),
            "write_mask": None if m is None else m.tolist(), "payload": _floats(p),
            "sum": _floats(s), "mask": mask.tolist(),
        })

    doc = {
        "source": "ravel_lm/ravel_memory.py:179-241 (causal_sum_lookup), evaluated by the "
                  "reference on the CPU",
        "generator": "tests/golden/make_sum_vectors.py",
        "cases": out,
    }
    with open(OUT, "w") as f:
        json.dump(doc, f)
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
