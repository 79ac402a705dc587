"""Device timing of every BASELINE configuration (cfg1-cfg5) on one GPU.

``python -m ravel_em.suite`` (or ``python bench.py --suite``) prints one JSON
line per measurement:

  latest_k   causal_last_k_lookup on the config's tape
  seg_sum    causal_sum_lookup on the same tape
  prefill    RavelLayerCache.prefill of the cfg5 decode cache
  decode     cfg5 RavelLayerCache.step, eager and replayed from a HIP graph

Each op is timed with HIP events around every call on torch's current stream
(warmup first, then the median of the calls).  Bytes are the algorithmic bytes
of the call (inputs read once plus outputs written once), and ``frac`` is the
achieved rate over 8 TB/s.  A caller may pass ``cpu(workload, op)``, which
returns a CPU-baseline dict for the same inputs; it is added to each line.
"""
from __future__ import annotations

import json
import statistics
import sys
from typing import Callable, List, Optional

import torch

from . import workloads
from .ravel_memory import RavelLayerCache, causal_last_k_lookup, causal_sum_lookup

PEAK_GBPS = 8000.0


def time_calls(fn: Callable[[], object], warmup: int = 5, iters: int = 50) -> List[float]:
    """Device microseconds of each of `iters` calls of fn (after `warmup` calls)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
    for e0, e1 in events:
        e0.record()
        fn()
        e1.record()
    torch.cuda.synchronize()
    return [e0.elapsed_time(e1) * 1e3 for e0, e1 in events]


def _line(config: str, op: str, us: float, nbytes: int, tokens: int, **extra) -> dict:
    gbps = nbytes / (us * 1e-6) / 1e9
    out = {
        "config": config, "op": op, "us_per_call": round(us, 2), "bytes": int(nbytes),
        "GBps": round(gbps, 1), "frac": round(gbps / PEAK_GBPS, 4),
        "tokens_per_s": tokens / (us * 1e-6),
    }
    out.update(extra)
    return out


def tape_lines(w: workloads.Workload, iters: int, cpu: Optional[Callable] = None) -> List[dict]:
    B, T, C, D = w.shape
    lines = []
    us = statistics.median(time_calls(
        lambda: causal_last_k_lookup(w.write, w.payload, w.read, address_space=w.address_space, k=w.k),
        iters=iters))
    lines.append(_line(w.name, "latest_k", us, workloads.algorithmic_bytes_latest_k(w), B * T,
                       shape=[B, T, C, D], k=w.k, A=w.address_space, dtype=str(w.payload.dtype).split(".")[-1],
                       read="separate" if w.read is not None else "same"))
    us = statistics.median(time_calls(
        lambda: causal_sum_lookup(w.write, w.payload, w.read, address_space=w.address_space), iters=iters))
    N = B * T * C
    esz = w.payload.element_size()
    addr = N * w.write.element_size() * (1 if w.read is None else 2)
    sum_bytes = addr + N * D * esz + N * D * esz + N
    lines.append(_line(w.name, "seg_sum", us, sum_bytes, B * T, shape=[B, T, C, D], A=w.address_space))
    if cpu is not None:
        for line in lines:
            line["cpu_baseline"] = cpu(w, line["op"])
    return lines


def decode_lines(dev: torch.device, steps: int = 1024, graph_chunk: int = 128,
                 cpu: Optional[Callable] = None) -> List[dict]:
    w = workloads.cfg5(dev, steps=steps)
    B, T, H = w.prefill_write.shape
    D = w.prefill_payload.shape[-1]
    lines = []
    us = statistics.median(time_calls(
        lambda: RavelLayerCache.prefill(w.prefill_write, w.prefill_payload, address_space=w.address_space, k=w.k),
        iters=10))
    cache_bytes = B * H * w.address_space * w.k * (D * 2 + 1)
    pre_bytes = w.prefill_write.numel() * 8 + w.prefill_payload.numel() * 2 + cache_bytes
    lines.append(_line("cfg5", "prefill", us, pre_bytes, B * T, shape=[B, T, H, D], k=w.k, A=w.address_space))

    cache = RavelLayerCache.prefill(w.prefill_write, w.prefill_payload, address_space=w.address_space, k=w.k)
    # Per step: 2 address tensors, the payload, the k-slot read (values + mask out),
    # and the shift-insert of the written slot (k-1 moves + 1 new row, filled bits).
    step_bytes = 2 * B * H * 8 + B * H * D * 2 + 2 * (B * H * w.k * D * 2 + B * H * w.k) \
        + B * H * (2 * w.k - 1) * D * 2 + B * H * w.k

    def eager():
        for s in range(steps):
            cache.step(w.step_read[s], w.step_write[s], w.step_payload[s])

    t = time_calls(eager, warmup=1, iters=3)
    us = statistics.median(t) / steps
    lines.append(_line("cfg5", "decode_step_eager", us, step_bytes, B, steps=steps,
                       steps_per_s=1e6 / us))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for s in range(3):
            cache.step(w.step_read[s], w.step_write[s], w.step_payload[s])
    torch.cuda.current_stream().wait_stream(side)
    graphs = []
    for c0 in range(0, steps, graph_chunk):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for s in range(c0, min(steps, c0 + graph_chunk)):
                cache.step(w.step_read[s], w.step_write[s], w.step_payload[s])
        graphs.append(g)

    def replay():
        for g in graphs:
            g.replay()

    t = time_calls(replay, warmup=1, iters=5)
    us = statistics.median(t) / steps
    lines.append(_line("cfg5", "decode_step_graph", us, step_bytes, B, steps=steps,
                       steps_per_s=1e6 / us, graph_steps=graph_chunk))
    if cpu is not None:
        for line in lines:
            line["cpu_baseline"] = cpu(w, line["op"])
    return lines


def run(dev: torch.device, iters: int = 50, cpu: Optional[Callable] = None) -> List[dict]:
    lines: List[dict] = []
    tapes = [
        lambda: workloads.cfg1(dev, "1"),
        lambda: workloads.cfg1(dev, "1b"),
        lambda: workloads.cfg2(dev, torch.float32),
        lambda: workloads.cfg2(dev, torch.bfloat16),
        lambda: workloads.cfg3(dev),
        lambda: workloads.cfg4(dev),
        lambda: workloads.cfg4(dev, adversarial=True),
    ]
    for make in tapes:
        w = make()
        for line in tape_lines(w, iters, cpu):
            print(json.dumps(line), flush=True)
            lines.append(line)
        del w
        torch.cuda.empty_cache()
    for line in decode_lines(dev, cpu=cpu):
        print(json.dumps(line), flush=True)
        lines.append(line)
    return lines


def main(argv=None) -> None:
    if not torch.cuda.is_available():
        sys.exit("the suite needs a ROCm GPU")
    run(torch.device("cuda", 0))


if __name__ == "__main__":
    main()
