"""Device timing of every benchmark configuration (cfg1-cfg5) on one GPU.

``python -m ravel_em.suite`` (or ``python bench.py --suite``) prints one JSON
line per measurement:

  latest_k   causal_last_k_lookup on the config's tape
  seg_sum    causal_sum_lookup on the same tape
  latest_k_sum  causal_last_k_and_sum_lookup: both on the same tape in one
             call (the memory layer's pair with use_sum_read); its bytes are
             the latest-k call's plus the sum rows and mask written
  prefill    RavelLayerCache.prefill of the cfg5 decode cache
  decode     cfg5 RavelLayerCache.step, eager and replayed from a HIP graph
  *_from_*   the memory layer's address production and lookup together
             (cfg1/cfg2 literal heads from token ids, cfg3 product codes from
             bf16 logits): the reference's torch address ops then the lookup
             ("chain"), the address kernel then the lookup ("kernel"), and
             the lookup producing its addresses in place ("fused")

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
from .ravel_memory import (RavelLayerCache, causal_last_k_and_sum_lookup, causal_last_k_lookup,
                           causal_sum_lookup)

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


def time_calls_fresh(fn: Callable[[], object], payload: torch.Tensor, warmup: int = 3,
                     iters: int = 20) -> List[float]:
    """Device microseconds of each of `iters` calls of fn, each made after a 1 GiB fill (more
    than the last-level cache) and a rewrite of `payload`, as when the layer op before the
    call has just written it.  Both are enqueued ahead of the call with no host wait, so the
    events time the call's own kernels."""
    flush = torch.empty(1 << 28, dtype=torch.float32, device=payload.device)
    src = payload.clone()

    def prep(i: int) -> None:
        flush.fill_(float(i))
        payload.copy_(src)

    for i in range(warmup):
        prep(i)
        fn()
    torch.cuda.synchronize()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
    for i, (e0, e1) in enumerate(events):
        prep(i)
        e0.record()
        fn()
        e1.record()
    torch.cuda.synchronize()
    del flush, src
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


def tape_lines(w: workloads.Workload, iters: int, cpu: Optional[Callable] = None,
               ops=("latest_k", "seg_sum", "latest_k_sum"), fresh: bool = True) -> List[dict]:
    """Each line's us_per_call repeats the call back to back (the inputs it read in its previous
    call may still be in the caches); us_fresh times it after a cache flush and a rewrite of
    the payload (time_calls_fresh), unless `fresh` is False."""
    B, T, C, D = w.shape
    lines = []

    def timed(fn):
        warm = statistics.median(time_calls(fn, iters=iters))
        if not fresh:
            return warm, None
        return warm, round(statistics.median(time_calls_fresh(fn, w.payload)), 2)

    if "latest_k_sum" in ops:
        us, us_f = timed(lambda: causal_last_k_and_sum_lookup(w.write, w.payload, w.read,
                                                               address_space=w.address_space, k=w.k))
        lines.append(_line(w.name, "latest_k_sum", us, workloads.algorithmic_bytes_latest_k_sum(w),
                           B * T, shape=[B, T, C, D], k=w.k, A=w.address_space,
                           dtype=str(w.payload.dtype).split(".")[-1],
                           read="separate" if w.read is not None else "same", us_fresh=us_f))
    if "latest_k" in ops:
        us, us_f = timed(lambda: causal_last_k_lookup(w.write, w.payload, w.read,
                                                       address_space=w.address_space, k=w.k))
        lines.append(_line(w.name, "latest_k", us, workloads.algorithmic_bytes_latest_k(w), B * T,
                           shape=[B, T, C, D], k=w.k, A=w.address_space,
                           dtype=str(w.payload.dtype).split(".")[-1],
                           read="separate" if w.read is not None else "same", us_fresh=us_f))
    if "seg_sum" not in ops:
        if cpu is not None:
            for line in lines:
                line["cpu_baseline"] = cpu(w, line["op"])
        return lines
    us, us_f = timed(lambda: causal_sum_lookup(w.write, w.payload, w.read, address_space=w.address_space))
    N = B * T * C
    esz = w.payload.element_size()
    addr = N * w.write.element_size() * (1 if w.read is None else 2)
    sum_bytes = addr + N * D * esz + N * D * esz + N
    lines.append(_line(w.name, "seg_sum", us, sum_bytes, B * T, shape=[B, T, C, D], A=w.address_space,
                       us_fresh=us_f))
    if cpu is not None:
        for line in lines:
            line["cpu_baseline"] = cpu(w, line["op"])
    return lines


def reference_addresses(src, A: int):
    """The reference layer's address ops on the device (ravel_lm/model.py:195-231,
    :303-307, :338-346): torch elementwise ops, argmax, cat."""
    parts_w, parts_r = [], []
    if src.n_literal_heads > 0:
        lit = workloads.literal_addresses(src.token_ids, address_space=A, n_heads=src.n_literal_heads,
                                          bos=src.bos_token_id)
        parts_w.append(lit)
        parts_r.append(lit)
    if src.n_learned_heads > 0:
        H, Q, S = src.n_learned_heads, src.n_codebooks, src.codebook_size
        mult = torch.tensor([S ** q for q in range(Q)], device=src.write_logits.device)

        def dec(lg):
            codes = lg.reshape(*lg.shape[:-1], H, Q, S).argmax(dim=-1).long()
            return (codes * mult).sum(dim=-1).remainder(A)

        parts_w.append(dec(src.write_logits))
        parts_r.append(dec(src.read_logits) if src.read_logits is not None else parts_w[-1])
    w = torch.cat(parts_w, dim=-1)
    r = w if src.same else torch.cat(parts_r, dim=-1)
    return w, r


def address_lines(w: workloads.Workload, iters: int, cpu: Optional[Callable] = None,
                  with_sum: bool = False) -> List[dict]:
    """latest-k (and optionally the sum) of a workload whose addresses come from
    its layer inputs, in the three forms chain / kernel / fused."""
    B, T, C, D = w.shape
    src, A, k = w.source, w.address_space, w.k
    inp = f"from_{'logits' if src.n_learned_heads else 'tokens'}"
    in_bytes = 0
    if src.n_literal_heads:
        in_bytes += src.token_ids.numel() * src.token_ids.element_size()
    for lg in (src.write_logits, src.read_logits if not src.same else None):
        if lg is not None:
            in_bytes += lg.numel() * lg.element_size()
    esz = w.payload.element_size()
    N = B * T * C

    def lookup(wa, ra):
        return causal_last_k_lookup(wa, w.payload, ra, address_space=A, k=k)

    forms = {
        "chain": lambda: lookup(*reference_addresses(src, A)),
        "kernel": lambda: lookup(*src.materialize(address_space=A)),
        "fused": lambda: causal_last_k_lookup(src, w.payload, address_space=A, k=k),
    }
    lk_bytes = in_bytes + N * D * esz + N * k * D * esz + N * k
    lines = []
    for form, fn in forms.items():
        us = statistics.median(time_calls(fn, iters=iters))
        lines.append(_line(w.name, f"latest_k_{inp}_{form}", us, lk_bytes, B * T, shape=[B, T, C, D],
                           k=k, A=A, heads={"literal": src.n_literal_heads, "learned": src.n_learned_heads}))
    if with_sum:
        sforms = {
            "chain": lambda: _sum_chain(reference_addresses(src, A), w.payload, A),
            "fused": lambda: causal_sum_lookup(src, w.payload, address_space=A),
        }
        sum_bytes = in_bytes + N * D * esz + N * D * esz + N
        for form, fn in sforms.items():
            us = statistics.median(time_calls(fn, iters=iters))
            lines.append(_line(w.name, f"seg_sum_{inp}_{form}", us, sum_bytes, B * T, shape=[B, T, C, D], A=A))
    if cpu is not None:
        for line in lines:
            if line["op"].endswith("_chain"):
                line["cpu_baseline"] = cpu(w, line["op"])
    return lines


def _sum_chain(wr, payload, A):
    wa, ra = wr
    return causal_sum_lookup(wa, payload, ra, address_space=A)


def decode_lines(dev: torch.device, steps: int = 1024, graph_chunk: int = 128,
                 cpu: Optional[Callable] = None, graphs: bool = True) -> List[dict]:
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
    if not graphs:
        return lines

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
    lines += decode_address_lines(dev, cache, w)
    if cpu is not None:
        for line in lines:
            if "from_tokens" not in line["op"]:
                line["cpu_baseline"] = cpu(w, line["op"])
    return lines


def decode_address_lines(dev: torch.device, cache: RavelLayerCache, w, steps: int = 256,
                         graph_chunk: int = 128) -> List[dict]:
    """The cfg5 cache stepped by a memory layer whose 8 heads are the literal
    families of the step's token (ravel_lm/model.py:401-426, history update
    :574): the reference's address ops as torch ops then the cache step
    ("chain"), against the cache step producing its addresses itself
    ("fused"); eager and replayed from HIP graphs."""
    from .addressing import LayerAddresses

    B, H = w.step_read.shape[1:]
    g = torch.Generator(device=dev)
    g.manual_seed(1016)
    toks = workloads.zipf((steps, B), w.address_space, g)
    hist0 = workloads.zipf((B, 2), w.address_space, g)
    A, bos = w.address_space, workloads.BOS
    hist = hist0.clone()

    def chain_step(s):
        a = workloads.literal_addresses_step(toks[s], hist, address_space=A, n_heads=H, position=s)
        out = cache.step(a, a, w.step_payload[s])
        hist.copy_(torch.cat([hist[:, 1:], toks[s].view(-1, 1)], dim=1))
        return out

    def fused_step(s):
        src = LayerAddresses(toks[s], H, bos, token_history=hist, position=s)
        out = cache.step(src, None, w.step_payload[s])
        hist.copy_(torch.cat([hist[:, 1:], toks[s].view(-1, 1)], dim=1))
        return out

    # both forms read the same values on the same cache state (first steps,
    # from a saved copy of the cache)
    saved = (cache.values.clone(), cache.filled.clone())
    hist.copy_(hist0)
    ref = [chain_step(s)[0].clone() for s in range(4)]
    cache.values.copy_(saved[0])
    cache.filled.copy_(saved[1])
    hist.copy_(hist0)
    same = all(torch.equal(fused_step(s)[0], ref[s]) for s in range(4))
    del saved
    lines = []
    for form, fn in (("chain", chain_step), ("fused", fused_step)):
        def eager():
            hist.copy_(hist0)
            for s in range(steps):
                fn(s)
        t = time_calls(eager, warmup=1, iters=3)
        us = statistics.median(t) / steps
        lines.append(_line("cfg5", f"decode_step_from_tokens_{form}_eager", us, 0, B,
                           steps=steps, steps_per_s=1e6 / us, heads=int(H), same_reads=same))
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for s in range(3):
                fn(s)
        torch.cuda.current_stream().wait_stream(side)
        graphs = []
        for c0 in range(0, steps, graph_chunk):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                for s in range(c0, min(steps, c0 + graph_chunk)):
                    fn(s)
            graphs.append(gr)

        def replay():
            hist.copy_(hist0)
            for gr in graphs:
                gr.replay()
        t = time_calls(replay, warmup=1, iters=5)
        us = statistics.median(t) / steps
        lines.append(_line("cfg5", f"decode_step_from_tokens_{form}_graph", us, 0, B,
                           steps=steps, steps_per_s=1e6 / us, graph_steps=graph_chunk, heads=int(H)))
    return lines


def fused_lines(dev: torch.device, iters: int) -> List[dict]:
    """The latest-1 lookup fused into the fuse layer's linear map on the cfg4 tape
    (`fused_latest1_linear`), against the lookup followed by torch's matmul
    (hipBLASLt), for M = 64, 192, 256 output columns of a bf16 W [M, C*D]
    (ravel_lm/triton_memory.py:378-426 is the reference's fused arm).  Bytes:
    addresses + payload rows read once + W + out; the unfused form also writes
    and reads the [B*T, C*D] lookup."""
    from .fused import fused_latest1_linear
    lines: List[dict] = []
    w = workloads.cfg4(dev)
    B, T, C, D = w.shape
    for M in (64, 192, 256):
        g = torch.Generator(device=dev).manual_seed(M)
        W = (torch.randn(M, C * D, generator=g, device=dev) / (C * D) ** 0.5).to(torch.bfloat16)

        def fused():
            return fused_latest1_linear(w.write, w.payload, None, W, address_space=w.address_space)

        def unfused():
            v, _ = causal_last_k_lookup(w.write, w.payload, address_space=w.address_space, k=1)
            return torch.matmul(v.reshape(B * T, C * D), W.t())

        nbytes = w.write.numel() * 8 + w.payload.numel() * 2 + W.numel() * 2 + B * T * M * 2
        flops = 2 * B * T * C * D * M
        for form, fn in (("fused", fused), ("lookup_then_matmul", unfused)):
            us = statistics.median(time_calls(fn, iters=iters))
            lines.append(_line("cfg4", f"latest1_linear_M{M}_{form}", us, nbytes, B * T, M=M,
                               TFLOPs=round(flops / (us * 1e-6) / 1e12, 1)))
    del w
    torch.cuda.empty_cache()
    return lines


PARTS = ("tapes", "addresses", "decode", "fused")


TAPE_CONFIGS = ("cfg1", "cfg1b", "cfg2_float32", "cfg2_bfloat16", "cfg3", "cfg4", "cfg4_adv")
TAPE_OPS = ("latest_k", "seg_sum", "latest_k_sum")


def run(dev: torch.device, iters: int = 50, cpu: Optional[Callable] = None,
        parts=PARTS, configs=None, ops=None, calibrate: bool = False,
        graphs: bool = True, fresh: bool = True) -> List[dict]:
    """Runs the named parts of the suite (all by default) and returns the lines;
    `configs` and `ops` narrow the tapes part to some configs and ops,
    `graphs=False` leaves out the decode part's HIP-graph forms, and
    `fresh=False` the tape ops' fresh-payload timing.  With
    `calibrate`, a 512 MiB device copy runs first: a kernel of known traffic
    (512 MiB read, 512 MiB written) by which hardware byte counters are scaled."""
    lines: List[dict] = []
    if calibrate:
        src = torch.empty(256 << 20, dtype=torch.bfloat16, device=dev).normal_()
        dst = torch.empty_like(src)
        for _ in range(2):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        torch.cuda.empty_cache()
    makers = {
        "cfg1": lambda: workloads.cfg1(dev, "1"),
        "cfg1b": lambda: workloads.cfg1(dev, "1b"),
        "cfg2_float32": lambda: workloads.cfg2(dev, torch.float32),
        "cfg2_bfloat16": lambda: workloads.cfg2(dev, torch.bfloat16),
        "cfg3": lambda: workloads.cfg3(dev),
        "cfg4": lambda: workloads.cfg4(dev),
        "cfg4_adv": lambda: workloads.cfg4(dev, adversarial=True),
    }
    bad = [c for c in (configs or ()) if c not in makers] + [o for o in (ops or ()) if o not in TAPE_OPS]
    if bad:
        raise ValueError(f"unknown tape configs or ops {bad}; configs {TAPE_CONFIGS}, ops {TAPE_OPS}")
    tapes = [] if "tapes" not in parts else [makers[c] for c in TAPE_CONFIGS if not configs or c in configs]
    for make in tapes:
        w = make()
        for line in tape_lines(w, iters, cpu, ops=tuple(ops) if ops else TAPE_OPS, fresh=fresh):
            print(json.dumps(line), flush=True)
            lines.append(line)
        del w
        torch.cuda.empty_cache()
    sources = [] if "addresses" not in parts else [
        (lambda: workloads.cfg1(dev, "1"), False),
        (lambda: workloads.cfg2(dev, torch.bfloat16), False),
        (lambda: workloads.cfg3_logits(dev), True),
    ]
    for make, with_sum in sources:
        w = make()
        for line in address_lines(w, iters, cpu, with_sum):
            print(json.dumps(line), flush=True)
            lines.append(line)
        del w
        torch.cuda.empty_cache()
    for line in decode_lines(dev, cpu=cpu, graphs=graphs) if "decode" in parts else []:
        print(json.dumps(line), flush=True)
        lines.append(line)
    for line in fused_lines(dev, iters) if "fused" in parts else []:
        print(json.dumps(line), flush=True)
        lines.append(line)
    return lines


def main(argv=None) -> None:
    """``python -m ravel_em.suite [part ...]`` with parts among tapes, addresses, decode, fused."""
    if not torch.cuda.is_available():
        sys.exit("the suite needs a ROCm GPU")
    parts = (argv if argv is not None else sys.argv[1:]) or PARTS
    bad = [p for p in parts if p not in PARTS]
    if bad:
        sys.exit(f"unknown suite parts {bad}; choose from {PARTS}")
    run(torch.device("cuda", 0), parts=tuple(parts))


if __name__ == "__main__":
    main()
