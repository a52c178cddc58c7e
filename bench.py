#!/usr/bin/env python3
"""Benchmark of the fused top-k + top-p sampler on one MI355X.

Prints ONE JSON line.  The headline metric has two halves and both are measured here:
  value          achieved logits-read bandwidth at C5 (B=256, V=151936, bf16, k=50, p=0.90),
                 cold: each call reads a different copy of the batch out of 14 rotated copies
                 (1.09 GB, more than 4x the 256 MB MALL), so the logits come from HBM;
  c1.us_per_call amortized microseconds per call at C1 (B=1, V=151936, bf16, k=50, p=0.90),
                 back-to-back calls from Python as the reference's harness times them
                 (benchmarks/harness.py:112-122), plus the same calls replayed from a HIP graph.
A "step" is one sampler call (one kernel launch) over one batch; inputs are resident in HBM
before the timed region; every timed region is bracketed by torch.cuda.synchronize().

Timing method (benchmarks/harness.py:112-138): the headline figures are the median of REPS
windows of back-to-back calls, each window calibrated to about WINDOW_MS, so they do not depend
on --steps.  The driver's contract is honoured as well: after --warmup untimed calls exactly
--steps calls are timed as one window, reported as `steps_window`.

roofline.achieved = algorithmic bytes per call (B*V*2 logits + B*4 u + B*8 ids) / the per-call
time measured with HIP events on the stream the kernel is launched on.
cpu_baseline: the CPU restatement of the reference's benchmarks/reference.py (oracle/), timed
on the host cores over a bounded sample of every benchmark configuration, in the reference's
own form (fp32 conversion + full stable sort per row) and in the oracle's counting-sort form.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "amortized µs/call at B=1,V=151936,k=50,p=0.9 BF16; logits GB/s at B=256"
HBM_PEAK_GBPS = 8000.0
ROTATE = 14
WINDOW_MS = 100.0
REPS = 7


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def algo_bytes(B: int, V: int) -> int:
    return B * V * 2 + B * 4 + B * 8


def window_ms(fn, iters: int) -> float:
    """Milliseconds per call over one window of `iters` back-to-back calls (HIP events on the
    current stream, which is the stream the sampler launches on)."""
    import torch

    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(iters):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / iters


def calibrated_ms(fn, warmup: int = 20, window: float = WINDOW_MS, reps: int = REPS,
                  multiple: int = 1) -> dict:
    """Median per-call ms over `reps` windows of about `window` ms each (the window length is
    calibrated from a short run, rounded to a multiple of `multiple` calls)."""
    for _ in range(warmup):
        fn()
    est = window_ms(fn, max(multiple, 50 // multiple * multiple))
    n = max(multiple, int(math.ceil(window / max(est, 1e-4) / multiple)) * multiple)
    runs = [window_ms(fn, n) for _ in range(reps)]
    return {"ms": statistics.median(runs), "calls_per_window": n, "reps": reps,
            "min_ms": min(runs), "max_ms": max(runs)}


def graph_per_call_ms(fn, calls: int = 100, reps: int = REPS, window: float = WINDOW_MS) -> float:
    """Capture `calls` back-to-back calls in one HIP graph and replay it in calibrated windows;
    median ms per call."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(calls):
            fn()
    res = calibrated_ms(g.replay, warmup=2, window=window, reps=reps)
    return res["ms"] / calls


def to_dev(bits: np.ndarray, dtype: str):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16))
    return t.view(torch.bfloat16 if dtype == "bfloat16" else torch.float16).cuda()


def launches_per_call(fn, calls: int = 20) -> dict:
    """Kernel launches per call counted by the profiler (torch.profiler's device activity, the
    method of the reference's benchmarks/launch_counts.py:21-32), plus memcpy/memset events."""
    import torch
    from torch.profiler import ProfilerActivity, profile

    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        for _ in range(calls):
            fn()
        torch.cuda.synchronize()
    kernels: dict = {}
    copies = 0
    for ev in prof.events():
        if ev.device_type != torch.autograd.DeviceType.CUDA:
            continue
        name = ev.name
        low = name.lower()
        if "memcpy" in low or "memset" in low or "copybuffer" in low or "fillbuffer" in low:
            copies += 1
            continue
        kernels[name] = kernels.get(name, 0) + 1
    total = sum(kernels.values())
    return {"launches_per_call": total / calls, "memcpy_memset_per_call": copies / calls,
            "calls": calls, "kernels": {k[:80]: v for k, v in kernels.items()}}


def cpu_baseline(budget_s: float) -> dict:
    """The CPU restatement on the host cores, every benchmark configuration.

    Two forms per case, each over a bounded sample of the case's rows:
      reference  oracle.sample_fullsort: each row converted to fp32 and fully sorted by a stable
                 merge sort, then the fp32 tail -- the algorithm of benchmarks/reference.py:48-68
                 (torch.sort(stable=True) on fp32) with an explicit u;
      counting   oracle.sample: the oracle's O(V) counting sort on the 16-bit order keys, then the
                 same tail.
    Every row of every case is timed (C5: all 256 rows per pass).  Both forms return the same
    token ids as the GPU (checked here against the fixture)."""
    from llm_sampling_kernel_amd import workloads as W
    from oracle import oracle as O

    host_cpus = os.cpu_count() or 1
    threads = max(1, min(16, host_cpus))
    fix = np.load(os.path.join(ROOT, "tests", "golden", "workloads.npz"))
    per_case = {}
    share = budget_s / (2 * len(W.CASE_NAMES))
    for name in W.CASE_NAMES:
        c = W.case(name)
        rows = c.batch
        x, u = c.logits, c.u
        want = fix[f"{name}/token_ids"][:rows]
        res = {}
        for form in ("reference", "counting"):
            def call(form=form):
                if form == "reference":
                    return O.sample_fullsort(x, c.dtype, c.top_k, c.top_p, u, nthreads=threads)[0]
                return O.sample(x, c.dtype, c.top_k, c.top_p, u, check_inputs=False,
                                nthreads=threads)
            tok = call()
            if not np.array_equal(tok, want):
                raise RuntimeError(f"CPU baseline ({form}) differs from the fixture on {name}")
            n, t0 = 0, time.perf_counter()
            while True:
                call()
                n += 1
                el = time.perf_counter() - t0
                if el >= share:
                    break
            per_rows = el / n
            ms_call = per_rows * 1e3 * c.batch / rows
            res[form] = {"ms_per_call": round(ms_call, 3),
                         "gbps": round(algo_bytes(c.batch, c.vocab) / (ms_call * 1e-3) / 1e9, 3),
                         "passes": n, "rows_per_pass": rows}
        per_case[name] = res
    c5 = per_case["C5"]["reference"]
    return {"value": c5["gbps"], "unit": "GB/s", "cores": threads, "kind": "port",
            "host_cpu_count": host_cpus,
            "sample": f"C5 value: {c5['passes']} whole 256-row calls ({c5['ms_per_call']:.0f} ms "
                      f"each), oracle in the reference's form (fp32 + full stable merge sort per "
                      f"row, fp32 tail); all {len(per_case)} cases in `per_config`, every row, "
                      f"~{budget_s:.0f} s in all",
            "ms_per_call_c5": c5["ms_per_call"], "per_config": per_case}


def traffic_probe(calls: int) -> int:
    """Workload for the HBM-traffic counters: `calls` cold C5 calls, then `calls` plain
    device-to-device copies of a buffer of the same size (the calibration kernel: it reads and
    writes exactly B*V*2 bytes).  Run under `rocprofv3 --pmc FETCH_SIZE` and again under
    `--pmc WRITE_SIZE`; --summarize-traffic turns the two CSVs into the traffic figure."""
    import torch

    from llm_sampling_kernel_amd import fused
    from llm_sampling_kernel_amd import workloads as W

    c5 = W.c5()
    x0 = to_dev(c5.logits, c5.dtype)
    u5 = torch.from_numpy(c5.u).cuda()
    bufs = [x0] + [x0.clone() for _ in range(ROTATE - 1)]
    torch.cuda.synchronize()
    for i in range(calls):
        fused.sample_fused_u(bufs[i % ROTATE], c5.top_k, c5.top_p, u5)
    torch.cuda.synchronize()
    dst = torch.empty_like(x0)
    for i in range(calls):
        dst.copy_(bufs[(i + 7) % ROTATE])
    torch.cuda.synchronize()
    log(f"traffic probe: {calls} C5 calls + {calls} copies of {x0.numel() * 2} bytes")
    return 0


def _pmc_means(path: str, counter: str) -> dict:
    """Mean counter value per dispatch, by kernel family (sampler / copy), from a rocprofv3
    counter_collection.csv."""
    import csv

    acc: dict = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            name = r["Kernel_Name"]
            fam = "sampler" if "fsamp_kernel" in name else ("copy" if "copy" in name.lower()
                                                             else None)
            if fam is None:
                continue
            acc.setdefault(fam, []).append(float(r["Counter_Value"]))
    return {k: (sum(v) / len(v), len(v)) for k, v in acc.items()}


def summarize_traffic(fetch_csv: str, write_csv: str, out_path: str) -> int:
    """HBM bytes per sampler launch from the two counter runs, each counter scaled by what it
    reads for the copy kernel, whose true traffic is B*V*2 bytes read and B*V*2 written."""
    B, V = 256, 151936
    copy_bytes = B * V * 2
    f = _pmc_means(fetch_csv, "FETCH_SIZE")
    w = _pmc_means(write_csv, "WRITE_SIZE")
    f_scale = copy_bytes / (f["copy"][0] * 1024.0)
    w_scale = copy_bytes / (w["copy"][0] * 1024.0)
    fetch_b = f["sampler"][0] * 1024.0 * f_scale
    write_b = w["sampler"][0] * 1024.0 * w_scale
    res = {
        "kernel": "fsamp_kernel (C5 plan)",
        "workload": "C5 cold: B=256, V=151936, bf16, k=50, p=0.90, 14 rotated input copies",
        "fetch_kib_per_dispatch": round(f["sampler"][0], 1),
        "write_kib_per_dispatch": round(w["sampler"][0], 1),
        "copy_fetch_kib": round(f["copy"][0], 1), "copy_write_kib": round(w["copy"][0], 1),
        "copy_bytes": copy_bytes, "fetch_scale": round(f_scale, 4),
        "write_scale": round(w_scale, 4),
        "dispatches": {"sampler": f["sampler"][1], "copy": f["copy"][1]},
        "bytes_per_launch": round(fetch_b + write_b),
        "algorithmic_bytes": algo_bytes(B, V),
    }
    with open(out_path, "w") as fo:
        json.dump(res, fo, indent=1)
        fo.write("\n")
    print(json.dumps(res))
    return 0


def c5_cold_only(steps: int, warmup: int) -> int:
    """Only cold C5 calls (for a kernel trace whose sampler dispatches are all cold): `warmup`
    untimed calls, then the calibrated windows, then exactly `steps` timed calls."""
    import torch

    from llm_sampling_kernel_amd import fused
    from llm_sampling_kernel_amd import workloads as W

    c5 = W.c5()
    x0 = to_dev(c5.logits, c5.dtype)
    u5 = torch.from_numpy(c5.u).cuda()
    bufs = [x0] + [x0.clone() for _ in range(ROTATE - 1)]
    it = [0]

    def call():
        i = it[0]
        it[0] = i + 1
        fused.sample_fused_u(bufs[i % ROTATE], 50, 0.90, u5)

    cal = calibrated_ms(call, warmup=warmup, multiple=ROTATE)
    k_ms = window_ms(call, steps)
    gb = algo_bytes(c5.batch, c5.vocab)
    print(json.dumps({"workload": "C5 cold only", "calls": it[0],
                      "us_per_call_median": round(cal["ms"] * 1e3, 3),
                      "us_per_call_steps_window": round(k_ms * 1e3, 3),
                      "gbps": round(gb / (cal["ms"] * 1e-3) / 1e9, 1),
                      "frac": round(gb / (cal["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}),
          flush=True)
    return 0


def vocab_parallel(x, c, fix_tokens, n_shards: int = 8) -> dict:
    """The vocabulary-parallel form of one configuration on one GPU: the row cut into n_shards
    column shards (each what one GPU of a tensor-parallel LM head would hold), the shard
    selection (fused_sampling.topk_shard) timed on one shard, the merge of the n_shards sorted
    lists and the draw (fused_sampling.merge_sample) timed on their stack; the merged tokens are
    checked against the whole-row fixture."""
    import torch

    from llm_sampling_kernel_amd import _lib, fused_sampling

    B, V = x.shape
    vs = V // n_shards
    bounds = [(i * vs, (i + 1) * vs if i + 1 < n_shards else V) for i in range(n_shards)]
    words = torch.stack([fused_sampling.topk_shard(x[:, lo:hi], c.top_k, lo) for lo, hi in bounds],
                        dim=1).contiguous()
    code = _lib.DTYPE_BF16 if c.dtype == "bfloat16" else _lib.DTYPE_F16
    u = torch.from_numpy(c.u).cuda()
    tok = fused_sampling.merge_sample(words, code, c.top_p, u).cpu().numpy()
    if not np.array_equal(tok, fix_tokens):
        raise RuntimeError(f"{c.name}: merged shard tokens differ from the fixture")
    lo, hi = bounds[0]
    shard = x[:, lo:hi]
    t_shard = calibrated_ms(lambda: fused_sampling.topk_shard(shard, c.top_k, lo), warmup=20,
                            window=50.0, reps=5)["ms"] * 1e3
    t_merge = calibrated_ms(lambda: fused_sampling.merge_sample(words, code, c.top_p, u),
                            warmup=20, window=50.0, reps=5)["ms"] * 1e3
    return {"shards": n_shards, "shard_columns": vs, "merge_width": n_shards * c.top_k,
            "us_per_shard_call": round(t_shard, 3), "us_per_merge_call": round(t_merge, 3),
            "note": "one shard's selection (sorted candidate words with global ids) and the merge "
                    "of the shards' lists plus the draw; no collective on one GPU"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-budget", type=float, default=24.0,
                    help="seconds of CPU baseline, split over the configurations")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--c5-cold-only", action="store_true",
                    help="run only cold C5 calls (for a cold-only kernel trace) and exit")
    ap.add_argument("--traffic-probe", type=int, metavar="CALLS", default=0,
                    help="run the workload for the HBM-traffic counters and exit")
    ap.add_argument("--summarize-traffic", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "OUT"),
                    help="turn two rocprofv3 counter CSVs into the traffic summary and exit")
    args = ap.parse_args()
    if args.summarize_traffic:
        return summarize_traffic(*args.summarize_traffic)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for "
              f"--gpus {args.gpus}); run with --gpus 1", file=sys.stderr)
        return 2
    if args.traffic_probe:
        return traffic_probe(args.traffic_probe)
    if args.c5_cold_only:
        return c5_cold_only(args.steps, args.warmup)

    import torch

    from llm_sampling_kernel_amd import _lib, fused, fused_sampling
    from llm_sampling_kernel_amd import workloads as W

    if not torch.cuda.is_available():
        print("no HIP device visible", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)
    dev_name = torch.cuda.get_device_properties(0).name

    # ---- C5: throughput, cold (rotated) and hot ----
    log("generating C5 inputs")
    c5 = W.c5()
    fix = np.load(os.path.join(ROOT, "tests", "golden", "workloads.npz"))
    x0 = to_dev(c5.logits, c5.dtype)
    u5 = torch.from_numpy(c5.u).cuda()
    got = fused.sample_fused_u(x0, c5.top_k, c5.top_p, u5).cpu().numpy()
    if not np.array_equal(got, fix["C5/token_ids"]):
        print("C5 token ids differ from the golden fixture; refusing to time a wrong kernel",
              file=sys.stderr)
        return 1
    bufs = [x0] + [x0.clone() for _ in range(ROTATE - 1)]
    torch.cuda.synchronize()
    it = [0]

    def c5_cold():
        i = it[0]
        it[0] = i + 1
        fused.sample_fused_u(bufs[i % ROTATE], 50, 0.90, u5)

    def c5_hot():
        fused.sample_fused_u(x0, 50, 0.90, u5)

    log(f"C5 cold: {args.warmup} warmup + exactly {args.steps} timed steps")
    for _ in range(args.warmup):
        c5_cold()
    ms_steps = window_ms(c5_cold, args.steps)
    log(f"C5 cold, {args.steps}-step window: {ms_steps * 1e3:.2f} us/call")
    cal5 = calibrated_ms(c5_cold, warmup=ROTATE, multiple=ROTATE)
    ms_cold = cal5["ms"]
    log(f"C5 cold, median of {cal5['reps']} windows of {cal5['calls_per_window']} calls: "
        f"{ms_cold * 1e3:.2f} us/call (min {cal5['min_ms'] * 1e3:.2f}, "
        f"max {cal5['max_ms'] * 1e3:.2f})")
    gi = [0]

    def c5_cold_graphable():
        i = gi[0]
        gi[0] = i + 1
        fused.sample_fused_u(bufs[i % ROTATE], 50, 0.90, u5)

    ms_cold_graph = graph_per_call_ms(c5_cold_graphable, calls=ROTATE)
    log(f"C5 cold from a HIP graph {ms_cold_graph * 1e3:.2f} us/call")
    ms_hot = calibrated_ms(c5_hot)["ms"]
    log(f"C5 hot {ms_hot * 1e3:.2f} us/call")
    # floors over the same cold buffers: one argmax pass (probes.cu's row-block scan) and the
    # load-only pass in the sampler's launch shape
    si = [0]

    def scan_cold():
        i = si[0]
        si[0] = i + 1
        fused_sampling.probe_scan_rowblock(bufs[i % ROTATE])

    ms_scan = calibrated_ms(scan_cold, multiple=ROTATE)["ms"]
    li = [0]
    wave_max = torch.empty(c5.batch * 8, dtype=torch.int32, device="cuda")

    def load_cold():
        i = li[0]
        li[0] = i + 1
        fused_sampling.probe_load(bufs[i % ROTATE], wave_max)

    ms_load = calibrated_ms(load_cold, multiple=ROTATE)["ms"]
    ti = [0]
    stream_max = torch.empty(_lib.load().fsamp_probe_stream_words(c5.batch, c5.vocab),
                             dtype=torch.int32, device="cuda")

    def stream_cold():
        i = ti[0]
        ti[0] = i + 1
        fused_sampling.probe_stream(bufs[i % ROTATE], stream_max)

    ms_stream = calibrated_ms(stream_cold, multiple=ROTATE)["ms"]
    log(f"C5 floors: one-pass scan {ms_scan * 1e3:.2f}, load only {ms_load * 1e3:.2f}, "
        f"stream read {ms_stream * 1e3:.2f} us/call")
    B5, V5 = c5.batch, c5.vocab
    gb5 = algo_bytes(B5, V5)
    gbps_cold = gb5 / (ms_cold * 1e-3) / 1e9
    gbps_hot = gb5 / (ms_hot * 1e-3) / 1e9
    plan5 = fused_sampling.make_plan(x0, 50)
    try:
        lc5 = launches_per_call(c5_hot)
    except Exception as exc:  # the profiler is a measurement aid, not the product
        lc5 = {"error": repr(exc)[:200]}
    del bufs

    # ---- C1: latency ----
    c1 = W.c1()
    x1 = to_dev(c1.logits, c1.dtype)
    u1 = torch.from_numpy(c1.u).cuda()
    got1 = fused.sample_fused_u(x1, 50, 0.9, u1).cpu().numpy()
    if not np.array_equal(got1, fix["C1/token_ids"]):
        print("C1 token ids differ from the golden fixture", file=sys.stderr)
        return 1
    c1_call = lambda: fused.sample_fused_u(x1, 50, 0.90, u1)  # noqa: E731
    log("timing C1")
    c1_us = calibrated_ms(c1_call, warmup=200)["ms"] * 1e3
    c1_graph_us = graph_per_call_ms(c1_call) * 1e3
    noop = lambda: fused_sampling.probe_noop(x1)  # noqa: E731
    floor_us = calibrated_ms(noop, warmup=200)["ms"] * 1e3
    floor_graph_us = graph_per_call_ms(noop) * 1e3
    # torch's own smallest kernel call on the same box (an in-place fill of one int64), for
    # comparison with the op's floor
    o1 = torch.empty(1, dtype=torch.int64, device="cuda")
    torch_fill_us = calibrated_ms(lambda: o1.zero_(), warmup=200)["ms"] * 1e3
    scan1 = lambda: fused_sampling.probe_scan_rowblock(x1)  # noqa: E731
    scan1_us = calibrated_ms(scan1, warmup=200)["ms"] * 1e3
    scan1_graph_us = graph_per_call_ms(scan1) * 1e3
    plan1 = fused_sampling.make_plan(x1, 50)
    try:
        lc1 = launches_per_call(c1_call)
    except Exception as exc:
        lc1 = {"error": repr(exc)[:200]}
    log(f"C1 {c1_us:.2f} us/call eager, {c1_graph_us:.2f} graph; floor {floor_us:.2f} / "
        f"{floor_graph_us:.2f}; launches per call {lc1.get('launches_per_call')}")

    vp = {}
    for name, xc_ in (("C1", x1), ("C5", x0)):
        vp[name] = vocab_parallel(xc_, W.case(name), fix[f"{name}/token_ids"])
        log(f"{name} vocabulary-parallel: shard {vp[name]['us_per_shard_call']:.2f} us, merge "
            f"{vp[name]['us_per_merge_call']:.2f} us")

    # the other benchmark configurations, eager back-to-back calls (hot: one buffer each)
    others = {}
    for name in ("C2_B1_k20", "C2_B1_k50", "C2_B4_k50", "C2_B16_k50", "C2_B64_k20",
                 "C2_B64_k50", "C3", "C4_k256", "C4_k1024"):
        c = W.case(name)
        xc = to_dev(c.logits, c.dtype)
        uc = torch.from_numpy(c.u).cuda()
        gotc = fused.sample_fused_u(xc, c.top_k, c.top_p, uc).cpu().numpy()
        if not np.array_equal(gotc, fix[f"{name}/token_ids"]):
            print(f"{name} token ids differ from the golden fixture", file=sys.stderr)
            return 1
        call = lambda xc=xc, uc=uc, c=c: fused.sample_fused_u(xc, c.top_k, c.top_p, uc)  # noqa: E731
        us = calibrated_ms(call, warmup=50, window=50.0, reps=5)["ms"] * 1e3
        pl = fused_sampling.make_plan(xc, c.top_k)
        others[name] = {"B": c.batch, "V": c.vocab, "k": c.top_k, "p": c.top_p,
                        "us_per_call": round(us, 3),
                        "gbps": round(algo_bytes(c.batch, c.vocab) / (us * 1e-6) / 1e9, 1),
                        "plan": {"splits": pl.splits, "threads": pl.threads,
                                 "chunks": pl.chunks}}
        log(f"{name}: {us:.2f} us/call")

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "fsamp_kernel_c5_hbm_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("bytes_per_launch")

    cpu = None
    if not args.no_cpu:
        log(f"CPU baseline (~{args.cpu_budget:.0f} s over every configuration)")
        cpu = cpu_baseline(args.cpu_budget)

    out = {
        "metric": METRIC,
        "value": round(gbps_cold, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_cold, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u16+f32",
        "data": "synthetic",
        "config": {
            "workload": "C5: B=256, V=151936, bf16 logits N(0,3^2) + Zipf(1.1)-ranked bias, "
                        "k=50, p=0.90, one fp32 u per row; cold: 14 rotated copies (1.09 GB)",
            "global_batch": B5, "vocab": V5, "top_k": 50, "top_p": 0.9,
            "parallelism": "single GPU",
            "plan": {"splits": plan5.splits, "threads": plan5.threads, "chunks": plan5.chunks},
        },
        "timing": {"method": f"median of {cal5['reps']} windows of {cal5['calls_per_window']} "
                             f"back-to-back cold calls (~{WINDOW_MS:.0f} ms each)",
                   "min_us": round(cal5["min_ms"] * 1e3, 3),
                   "max_us": round(cal5["max_ms"] * 1e3, 3)},
        "steps_window": {"steps": args.steps, "warmup": args.warmup,
                         "us_per_call": round(ms_steps * 1e3, 3),
                         "gbps": round(gb5 / (ms_steps * 1e-3) / 1e9, 1)},
        "roofline": {"bound": "hbm", "achieved": round(gbps_cold, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(gbps_cold / HBM_PEAK_GBPS, 4),
                     "traffic": traffic},
        "cpu_baseline": cpu,
        "c5_hot": {"us_per_call": round(ms_hot * 1e3, 3), "gbps": round(gbps_hot, 1),
                   "note": "one buffer: served from the 256 MB MALL, not HBM"},
        "c5_cold_graph": {"us_per_call": round(ms_cold_graph * 1e3, 3),
                          "gbps": round(gb5 / (ms_cold_graph * 1e-3) / 1e9, 1),
                          "note": "the same cold calls replayed from a HIP graph"},
        "c5_scan_floor": {"us_per_call": round(ms_scan * 1e3, 3),
                          "gbps": round(gb5 / (ms_scan * 1e-3) / 1e9, 1),
                          "note": "one pass over the same cold buffers: argmax per row, one "
                                  "1024-thread workgroup per row (the reference's probes.cu "
                                  "row-block scan)"},
        "c5_load_floor": {"us_per_call": round(ms_load * 1e3, 3),
                          "gbps": round(gb5 / (ms_load * 1e-3) / 1e9, 1),
                          "note": "fsamp_probe_load: the sampler's B=256 launch shape and load "
                                  "order (512 threads, 38 nontemporal 16-byte loads each, 6 in "
                                  "flight, the slice kept in registers) with only a per-wave "
                                  "maximum after the loads"},
        "c5_stream_floor": {"us_per_call": round(ms_stream * 1e3, 3),
                            "gbps": round(gb5 / (ms_stream * 1e-3) / 1e9, 1),
                            "note": "fsamp_probe_stream: the same batch read once by 4,748 "
                                    "short workgroups (256 threads x 4 nontemporal 16-byte "
                                    "loads), no row shape: the read floor of the memory "
                                    "system"},
        "c5_launches": lc5,
        "configs": others,
        "vocab_parallel": vp,
        "c1": {"us_per_call": round(c1_us, 3), "us_per_call_graph": round(c1_graph_us, 3),
               "launches": lc1, "launch_floor_us": round(floor_us, 3),
               "launch_floor_graph_us": round(floor_graph_us, 3),
               "torch_fill_floor_us": round(torch_fill_us, 3),
               "scan_floor_us": round(scan1_us, 3), "scan_floor_graph_us": round(scan1_graph_us, 3),
               "plan": {"splits": plan1.splits, "threads": plan1.threads,
                        "chunks": plan1.chunks}},
        "device": dev_name,
        "compute": "bf16 logits in; u16 order keys and u64 (key, ~id) words for the selection "
                   "(integer), fp32 softmax/prefix/draw",
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
