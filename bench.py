#!/usr/bin/env python3
"""Headline benchmark of the MI355X event-memory operator.

Metric: event-memory prefill tokens/sec at 1 GPU + achieved HBM GB/s (% of
peak).  Workload: benchmark configuration cfg4, the latest-1 forward of
causal_last_k_lookup at B=4, T=65536, H=16 heads, A=65536 addresses, D=64 bf16
payload (N = 4,194,304 records), synthetic seeded inputs resident in HBM.

One "step" is one causal_last_k_lookup call over the whole batch.  `value` is
B*T tokens per step / measured step time.  Prints one JSON line with:
  roofline     the dominant kernel (the payload gather), timed with HIP events
               on its launch stream inside the timed region, against 8 TB/s;
  op_roofline  the whole operator against the same peak, using the
               inputs-read-once + outputs-written-once bytes of the call;
  cpu_baseline the reference algorithm restated on the host CPU (torch),
               timed on a bounded sample on this box's cores.
Only one GPU is supported: --gpus N with N > 1 exits with a message.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "ravel-lm_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "event-memory prefill tokens/sec at 1 GPU + achieved HBM GB/s (% of peak)"
PEAK_HBM_GBPS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gather_cfg4_traffic.json")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--adversarial", action="store_true", help="90%% of records at address 0")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU baseline sample")
    ap.add_argument("--suite", action="store_true",
                    help="time every benchmark config (cfg1-cfg5), one JSON line per op, instead of the headline")
    ap.add_argument("--suite-parts", nargs="+", default=None, metavar="PART",
                    help="with --suite: only these parts (tapes, addresses, decode, fused)")
    ap.add_argument("--suite-configs", nargs="+", default=None, metavar="CONFIG",
                    help="with --suite: only these tape configs (cfg1, cfg1b, cfg2_float32, "
                         "cfg2_bfloat16, cfg3, cfg4, cfg4_adv)")
    ap.add_argument("--suite-ops", nargs="+", default=None, metavar="OP",
                    help="with --suite: only these tape ops (latest_k, seg_sum, latest_k_sum)")
    ap.add_argument("--suite-iters", type=int, default=50, help="with --suite: timed calls per op")
    ap.add_argument("--suite-no-graphs", action="store_true",
                    help="with --suite: time the decode step eagerly only (no HIP graph capture)")
    ap.add_argument("--suite-no-fresh", action="store_true",
                    help="with --suite: time tape ops back to back only (no fresh-payload timing)")
    ap.add_argument("--suite-calibrate", action="store_true",
                    help="with --suite: first copy a 512 MiB tensor (a known-size kernel for counter scaling)")
    return ap.parse_args()


def _cgroup_cpu_quota():
    """CPUs allowed by a cgroup v2 (cpu.max) or v1 (cfs quota) limit, or None."""
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()[:2]
        if quota != "max":
            return max(1, int(int(quota) // int(period)))
        return None
    except (OSError, ValueError):
        pass
    try:
        with open("/sys/fs/cgroup/cpu/cpu.cfs_quota_us") as f:
            quota = int(f.read())
        with open("/sys/fs/cgroup/cpu/cpu.cfs_period_us") as f:
            period = int(f.read())
        return max(1, quota // period) if quota > 0 else None
    except (OSError, ValueError):
        return None


def cpu_info():
    """The host CPU the baseline runs on: model name, the cores of this
    process's affinity mask, any cgroup CPU quota, the CPU share the host
    declares in OMP_NUM_THREADS, and the threads used: every core in the mask,
    fewer only where the quota or the declared share allows fewer."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    quota = _cgroup_cpu_quota()
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        share = int(os.environ.get("OMP_NUM_THREADS", "")) or None
    except ValueError:
        share = None
    threads = max(1, min(x for x in (affinity, quota, share) if x))
    return {"model": model, "affinity_cores": affinity, "cgroup_quota_cpus": quota,
            "declared_share_OMP_NUM_THREADS": share, "threads": threads}


def cpu_threads():
    return cpu_info()["threads"]


def cpu_baseline(w, budget_s):
    """Reference algorithm on the host: torch sort / searchsorted / gathers."""
    import torch

    from oracle import torch_ref

    threads = cpu_threads()
    torch.set_num_threads(threads)
    write = w.write.cpu()
    payload = w.payload.cpu()
    B, T, C, D = w.shape
    log(f"cpu baseline: {threads} threads, full cfg4 call per sample")
    torch_ref.latest_k(write, payload, address_space=w.address_space, k=w.k)  # warmup
    times = []
    t_start = time.perf_counter()
    while len(times) < 2 or (time.perf_counter() - t_start < budget_s and len(times) < 20):
        t0 = time.perf_counter()
        torch_ref.latest_k(write, payload, address_space=w.address_space, k=w.k)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": B * T / med,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "cpu": cpu_info(),
        "sample": f"{len(times)} full cfg4 latest-1 calls (median {med:.3f} s) of the reference's "
                  "sort/searchsorted/gather algorithm restated with torch on the CPU",
    }


def _wr(addrs, payload):
    return addrs[0], payload, addrs[1]


def suite_cpu_baseline(w, op, budget_s=6.0):
    """The reference CPU path (torch restatement) on one suite workload and op."""
    import torch

    from oracle import torch_ref

    threads = cpu_threads()
    torch.set_num_threads(threads)

    def timed(fn, reps):
        times = []
        t_start = time.perf_counter()
        while len(times) < reps and (not times or time.perf_counter() - t_start < budget_s):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        times.sort()
        return times[len(times) // 2], len(times)

    if "_from_" in op:
        # the reference layer's address ops then its lookup, all on the CPU
        src = w.source
        A = w.address_space
        toks = None if src.n_literal_heads == 0 else src.token_ids.cpu()
        wl = None if src.write_logits is None else src.write_logits.cpu()
        rl = None if src.same else src.read_logits.cpu()
        payload = w.payload.cpu()
        B, T = payload.shape[:2]

        def addresses():
            parts_w, parts_r = [], []
            if toks is not None:
                lit = torch_ref.literal_addresses(toks, address_space=A, n_heads=src.n_literal_heads,
                                                  bos_token_id=src.bos_token_id)
                parts_w.append(lit)
                parts_r.append(lit)
            if wl is not None:
                kw = dict(n_heads=src.n_learned_heads, n_codebooks=src.n_codebooks,
                          codebook_size=src.codebook_size, address_space=A)
                parts_w.append(torch_ref.product_codes(wl, **kw))
                parts_r.append(parts_w[-1] if rl is None else torch_ref.product_codes(rl, **kw))
            wa = torch.cat(parts_w, dim=-1)
            return wa, (None if src.same else torch.cat(parts_r, dim=-1))

        if op.startswith("latest_k"):
            fn = lambda: torch_ref.latest_k(*_wr(addresses(), payload), address_space=A, k=w.k)
        else:
            fn = lambda: torch_ref.seg_sum(*_wr(addresses(), payload), address_space=A)
        med, n = timed(fn, 3)
        return {"value": B * T / med, "unit": "tokens/s", "cores": threads, "kind": "port",
                "sample": f"{n} full calls (address ops + lookup), median {med:.4f} s"}
    if op in ("latest_k", "seg_sum", "latest_k_sum"):
        write = w.write.cpu()
        read = None if w.read is None else w.read.cpu()
        payload = w.payload.cpu()
        B, T = write.shape[:2]
        lk = lambda: torch_ref.latest_k(write, payload, read, address_space=w.address_space, k=w.k)
        ss = lambda: torch_ref.seg_sum(write, payload, read, address_space=w.address_space)
        # the reference layer's pair of calls with use_sum_read (model.py:366-386)
        fn = {"latest_k": lk, "seg_sum": ss, "latest_k_sum": lambda: (lk(), ss())}[op]
        med, n = timed(fn, 3)
        return {"value": B * T / med, "unit": "tokens/s", "cores": threads, "kind": "port",
                "sample": f"{n} full calls, median {med:.4f} s"}
    # cfg5: the reference cache is the k = 1 one, written token by token
    # (ravel_lm/model.py:600-602) and read/written once per decode step.
    pw, pp = w.prefill_write.cpu(), w.prefill_payload.cpu()
    B, T, H = pw.shape
    D = pp.shape[-1]
    values = torch.zeros(B, H, w.address_space, D, dtype=pp.dtype)
    filled = torch.zeros(B, H, w.address_space, dtype=torch.bool)
    if op == "prefill":
        n_tok = min(T, 64)
        t0 = time.perf_counter()
        for t in range(n_tok):
            torch_ref.cache_write(values, filled, pw[:, t], pp[:, t])
        per_tok = (time.perf_counter() - t0) / n_tok
        return {"value": B / per_tok, "unit": "tokens/s", "cores": threads, "kind": "port",
                "work": "different work from the GPU line: the reference's k=1 cache written "
                        "token by token, not the k=4 cache built in one pass",
                "sample": f"{n_tok} of {T} prefill tokens written one at a time (k=1 cache)"}
    sr, sw, sp = w.step_read.cpu(), w.step_write.cpu(), w.step_payload.cpu()
    n_steps = min(sr.shape[0], 128)
    t0 = time.perf_counter()
    for s in range(n_steps):
        torch_ref.cache_read(values, filled, sr[s])
        torch_ref.cache_write(values, filled, sw[s], sp[s])
    per_step = (time.perf_counter() - t0) / n_steps
    return {"value": B / per_step, "unit": "tokens/s", "cores": threads, "kind": "port",
            "work": "different work from the GPU line: the reference's k=1 cache, one read "
                    "and one write per step, not the k=4 shift-insert step",
            "sample": f"{n_steps} decode steps, read then write (k=1 cache)"}


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print(f"bench.py runs on one GPU only (asked for {max(args.gpus, world)}): the operator shards "
              "by (batch, head) stream with no communication, so each GPU would run this same "
              "single-GPU measurement on its share.", flush=True)
        sys.exit(2)

    import torch

    from ravel_em import _native as nat
    from ravel_em import causal_last_k_lookup, workloads

    dev = torch.device("cuda", 0)
    if args.suite:
        from ravel_em import suite

        suite.run(dev, iters=args.suite_iters,
                  cpu=None if args.no_cpu_baseline else suite_cpu_baseline,
                  parts=tuple(args.suite_parts) if args.suite_parts else suite.PARTS,
                  configs=args.suite_configs, ops=args.suite_ops, calibrate=args.suite_calibrate,
                  graphs=not args.suite_no_graphs, fresh=not args.suite_no_fresh)
        return
    log("generating cfg4 inputs on the device")
    w = workloads.cfg4(dev, adversarial=args.adversarial)
    B, T, C, D = w.shape
    N, k, A = B * T * C, w.k, w.address_space
    torch.cuda.synchronize()

    with torch.no_grad():
        for _ in range(args.warmup):
            vals, mask = causal_last_k_lookup(w.write, w.payload, w.read, address_space=A, k=k)
        torch.cuda.synchronize()

        # Timed region A: the drop-in call, as model.py makes it.
        log(f"timing {args.steps} steps of causal_last_k_lookup")
        t_begin = torch.cuda.Event(enable_timing=True)
        t_end = torch.cuda.Event(enable_timing=True)
        wall0 = time.perf_counter()
        t_begin.record()
        for _ in range(args.steps):
            vals, mask = causal_last_k_lookup(w.write, w.payload, w.read, address_space=A, k=k)
        t_end.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - wall0
        ms = t_begin.elapsed_time(t_end) / args.steps

        # Timed region B: the same call with the library's stage timer on, which
        # brackets each stage (sort, resolve, gather) with HIP events on the
        # stream the kernels are launched on.
        import ctypes

        lib = nat.library()
        nat.check(lib.ravel_em_profile_start())
        b_begin = torch.cuda.Event(enable_timing=True)
        b_end = torch.cuda.Event(enable_timing=True)
        b_begin.record()
        for _ in range(args.steps):
            vals_b, mask_b = causal_last_k_lookup(w.write, w.payload, w.read, address_space=A, k=k)
        b_end.record()
        stage_ms = (ctypes.c_double * 5)()
        stage_calls = (ctypes.c_int * 5)()
        nat.check(lib.ravel_em_profile_stop(stage_ms, stage_calls, 5))
        torch.cuda.synchronize()
        stages = {name: stage_ms[i] / max(1, stage_calls[i])
                  for i, name in enumerate(["sort", "resolve", "gather"])}
        gather_ms = stages["gather"]
        timed_ms = b_begin.elapsed_time(b_end) / args.steps
        assert torch.equal(vals_b, vals) and torch.equal(mask_b, mask), "repeat call differs"
        valid_slots = int(mask.sum().item())
        row_bytes = D * w.payload.element_size()

        # Streaming references on the same device: a 512 MiB device-to-device
        # copy and a 512 MiB fill, the practical HBM ceilings for read+write and
        # write-only traffic.
        src_buf = torch.empty(256 << 20, dtype=torch.bfloat16, device=dev).normal_()
        dst_buf = torch.empty_like(src_buf)
        for _ in range(3):
            dst_buf.copy_(src_buf)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            dst_buf.copy_(src_buf)
        e1.record()
        torch.cuda.synchronize()
        copy_gbps = 2 * src_buf.numel() * 2 * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e9
        dst_buf.fill_(1.0)  # first use loads the kernel: keep it out of the timing
        torch.cuda.synchronize()
        e0.record()
        for _ in range(10):
            dst_buf.fill_(1.0)
        e1.record()
        torch.cuda.synchronize()
        fill_gbps = dst_buf.numel() * 2 * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e9
        del src_buf, dst_buf

    # Gather kernel bytes: src read (4 B/slot), values written, and one payload
    # row read per valid slot.  On this path (k = 1, reads = writes, C a power
    # of two) the source transpose writes the mask bytes, not the gather.
    gather_bytes = N * k * (4 + row_bytes) + valid_slots * row_bytes
    gather_gbps = gather_bytes / (gather_ms * 1e-3) / 1e9
    traffic = step_measured = None
    if os.path.exists(TRAFFIC_FILE) and not args.adversarial:  # measured for the uniform tape
        with open(TRAFFIC_FILE) as f:
            tf = json.load(f)
        traffic = tf.get("bytes_per_launch")
        step_measured = tf.get("step_bytes_measured")
    op_bytes = workloads.algorithmic_bytes_latest_k(w)
    op_gbps = op_bytes / (ms * 1e-3) / 1e9

    result = {
        "metric": METRIC,
        "value": B * T / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "cfg4" + ("_adversarial" if args.adversarial else "")
            + ": causal_last_k_lookup latest-1 forward, B=4 T=65536 H=16 A=65536 D=64 bf16",
            "B": B, "T": T, "H": C, "A": A, "D": D, "k": k,
            "records": N, "payload_dtype": "bf16", "sort_key": "u32 (a<<16|t) per (b,h) segment",
        },
        "achieved_GBps": op_gbps,
        "achieved_frac_of_peak": op_gbps / PEAK_HBM_GBPS,
        "roofline": {
            "bound": "hbm",
            "kernel": "gather_rows_kernel",
            "achieved": gather_gbps,
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": gather_gbps / PEAK_HBM_GBPS,
            "traffic": traffic,
            "avg_launch_ms": gather_ms,
            "bytes_per_launch": gather_bytes,
            "valid_slot_fraction": valid_slots / (N * k),
        },
        "op_roofline": {
            "bound": "hbm",
            "achieved": op_gbps,
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": op_gbps / PEAK_HBM_GBPS,
            "bytes_per_call": op_bytes,
            "stage_ms": stages,
            "ms_per_step_with_stage_timer": timed_ms,
            # the step's HBM bytes from the PMC profile (FETCH/WRITE_SIZE of its
            # kernels, scaled by the copy calibration) at this run's step time
            "physical_bytes_per_call": step_measured,
            "physical_frac": (step_measured / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS) if step_measured else None,
        },
        "wall_s_timed_region": wall,
        "hbm_reference_GBps": {"copy_512MiB": copy_gbps, "fill_512MiB": fill_gbps},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
