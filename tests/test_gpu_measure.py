"""The suite's timing leaves the workload as it found it.

`ravel_em.suite.tape_lines` times every tape op back to back and fresh (after a
cache flush and a rewrite of the payload with its own copy): each line carries
both times, and the payload the calls read is bit-identical afterwards.
"""
import pytest
import torch

from ravel_em import suite, workloads

pytestmark = pytest.mark.gpu


def test_tape_lines_fresh_timing_keeps_the_payload(device):
    w = workloads.cfg1(device)
    before = w.payload.clone()
    lines = suite.tape_lines(w, iters=5)
    torch.cuda.synchronize()
    assert [d["op"] for d in lines] == ["latest_k_sum", "latest_k", "seg_sum"]
    for d in lines:
        print(f"[measure] {d['config']} {d['op']} {d['us_per_call']} us, fresh {d['us_fresh']} us",
              flush=True)
        assert d["us_per_call"] > 0 and d["us_fresh"] > 0
    assert torch.equal(w.payload, before)
    assert all(d["us_fresh"] is None for d in suite.tape_lines(w, iters=3, fresh=False))
