#!/usr/bin/env python3
"""Headline benchmark: one MI355X sampling step over a batch of logit rows.

A step is one sas_sample launch over one batch of synthetic inputs that are
already resident in HBM: 262,144-vocab fp32 logits, the packed grammar
bitmask, repetition / presence / frequency penalties from a 512-id history,
then temperature 1.0 / top-k 50 / top-p 0.9 and the seeded draw, batch 128
(workload C3P).  Inputs rotate over several independent sets totalling more
than 512 MB so the 256 MB Infinity Cache cannot serve them.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload C3P]

Prints ONE JSON line (rank 0): rows/s, the roofline of the sampling step
(its two launches, sas::sample_parts_kernel then sas::sample_merge_kernel:
algorithmic bytes / average step time, HIP events on the launch stream;
the median of per-step event pairs is reported beside it)
and the CPU baseline: the Node restatement of the reference's JS sampling
path timed on this host's cores on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import tempfile

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "rows/s + % HBM peak: 262k-vocab penalties+mask+top-k/top-p, B=128"
HBM_PEAK_GBPS = 8000.0
KERNEL = "sampler_step"  # the profiles/ summaries of the two launches of one step
WORKLOAD_DOC = {
    "C1": "greedy + repetition 1.1 over 512 history ids, vocab 151936, one row (the case the reference runs on "
          "the CPU)",
    "C2": "T0.7 top-k40 top-p0.95, vocab 151936, batch 64, Zipf-biased N(0,3) logits",
    "C3": "bitmask 0.5-20% + top-k50 top-p0.9 T1.0, vocab 262144, batch 128, N(0,4) logits",
    "C3P": "C3 + repetition 1.1 / presence 0.5 / frequency 0.3 over 512 history ids, vocab 262144, batch 128",
    "C3P8": "one GPU's share of C3P sharded 8 ways over the vocabulary: vocab 32768, batch 128, 64 history ids "
            "per row (the step before the records' all-gather)",
    "C4": "repetition 1.15 / presence 0.5 / frequency 0.3 over 4096 Zipf history ids, greedy, vocab 262144, "
          "batch 256",
    "C5": "speculative verify (rejection sampling): 32 sequences x (4 drafts + 1 bonus), vocab 151936, draft "
          "logits 0.8-correlated with the target, 5% mask on both",
    "LMH1": "the LM head with the sampling step fused (sas_lm_head_sample): one decode row, hidden 2560 fp32 times "
            "a 262144 x 2560 bf16 head (Gemma-4 E4B shape), softcap 30, then C3P's mask, penalties and "
            "top-k 50 / top-p 0.9",
    "LMH3": "as LMH1 with the three rows of a speculative verify round over the same head",
    "LMQ1": "the LM head with the sampling step fused over Qwen3.5-4B's tied Q6_K head (GGUF blocks, vocabulary "
            "248320, hidden 2560, the hidden state quantized to Q8_1 on chip, exact integer block dots), one decode "
            "row, then C3P's mask, penalties and top-k 50 / top-p 0.9",
    "LMQ3": "as LMQ1 with the three rows of a speculative verify round over the same head",
}
CPU_THREADS = 16  # the GPU box's CPU share for one GPU (its nproc may show more)


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--workload", default="C3P", choices=sorted(WORKLOAD_DOC))
    ap.add_argument("--min-set-mb", type=float, default=512.0,
                    help="rotate over input sets totalling at least this many MB")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="approximate CPU work of the baseline sample (0 disables it)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graph-steps", type=int, default=0,
                    help="record this many steps (input sets in turn) into one HIP graph by stream capture and "
                         "time its replays (the k-step submit of a decode loop)")
    ap.add_argument("--row-params", action="store_true",
                    help="pass the workload's parameters per row (row_params, with the no-softcap hint) "
                         "instead of one sas_params for every row")
    ap.add_argument("--stream-probe", action="store_true",
                    help="time sasp_read (libsas_probe.so): the parts kernel's loads alone over one C3P step's "
                         "bytes")
    ap.add_argument("--mask-probe", action="store_true",
                    help="time sasp_masked_read (libsas_probe.so): C3's logits read whole or only where the "
                         "grammar mask allows an id")
    ap.add_argument("--mask-probe-mode", type=int, default=-1, help="with --mask-probe: one mode only")
    ap.add_argument("--memset-order-probe", action="store_true",
                    help="sasp_memset_order (libsas_probe.so): whether a kernel on a non-blocking stream "
                         "launched right after hipMemset sees the fill")
    ap.add_argument("--calibrate-copy-mb", type=float, default=0.0,
                    help="instead of the benchmark, run device-to-device copies of this many MB (the "
                         "reference kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    return ap.parse_args()


def calibrate_copy(mb: float, steps: int) -> int:
    """Copies of a known size: under rocprofv3 --pmc, FETCH_SIZE and WRITE_SIZE
    of this copy kernel against its true byte count give the factor that turns
    the counters into bytes."""
    import torch

    n = int(mb * 1e6) // 16 * 4
    src = torch.randn(n, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "bytes_read_per_launch": src.numel() * 4,
                      "bytes_written_per_launch": dst.numel() * 4, "launches": steps}), flush=True)
    return 0


def _probe_lib():
    """libsas_probe.so: the measurement probes (never part of the sampling
    library)."""
    import ctypes
    from ctypes import c_int, c_int32, c_size_t, c_void_p

    path = os.path.join(ROOT, "shared_amd", "libsas_probe.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with python -m shared_amd.build")
    lib = ctypes.CDLL(path)
    lib.sasp_read.restype = c_int
    lib.sasp_read.argtypes = [c_void_p, c_size_t, c_int32, c_void_p, c_void_p]
    lib.sasp_masked_read.restype = c_int
    lib.sasp_masked_read.argtypes = [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p]
    lib.sasp_memset_order.restype = c_int
    lib.sasp_memset_order.argtypes = [c_size_t, c_int32, c_void_p]
    return lib


def memset_order_probe(args) -> int:
    """Whether hipMemset (the null stream) is ordered before a kernel that a
    non-blocking stream runs right after it: sasp_memset_order over a 256 MB
    buffer, 20 runs.  Prints one JSON line."""
    import ctypes

    class Res(ctypes.Structure):
        _fields_ = [("reps", ctypes.c_int32), ("stale_runs", ctypes.c_int32), ("host_us", ctypes.c_double),
                    ("fill_us", ctypes.c_double)]

    lib = _probe_lib()
    r = Res()
    rc = lib.sasp_memset_order(256 << 20, 20, ctypes.byref(r))
    if rc != 0:
        raise RuntimeError(f"sasp_memset_order failed ({rc})")
    print(json.dumps({"probe": "hipMemset then a kernel on a non-blocking stream (sasp_memset_order)",
                      "bytes": 256 << 20, "runs": r.reps, "runs_reading_unfilled_words": r.stale_runs,
                      "hipMemset_host_us": round(r.host_us, 2), "fill_us_on_a_stream": round(r.fill_us, 2)}),
          flush=True)
    return 0


def _probe_time(args, stream, launch) -> float:
    """Microseconds per launch of launch(i): warm-up, then args.steps launches
    between two HIP events on `stream`."""
    import torch

    for i in range(args.warmup):
        launch(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(args.steps):
        launch(i)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / args.steps


def stream_probe(args) -> int:
    """The streaming bound of the sampling kernels: sasp_read reads the C3P
    step's algorithmic bytes with the parts kernel's access pattern and
    nothing else, over rotating buffers (more bytes than the caches hold),
    for several grid sizes.  Prints one JSON line."""
    import ctypes

    import torch

    from shared_amd import workloads as W

    lib = _probe_lib()
    set_bytes = W.c3p().algorithmic_bytes() // 16 * 16  # one C3P step
    nsets = max(2, int(-(-args.min_set_mb * 1e6 // set_bytes)))
    bufs = [torch.empty(set_bytes // 4, dtype=torch.float32, device="cuda").uniform_() for _ in range(nsets)]
    sink = torch.zeros(256, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()
    res = {}
    for blocks in (1024, 2048, 4096, 8192):
        def launch(i):
            rc = lib.sasp_read(ctypes.c_void_p(bufs[i % nsets].data_ptr()), set_bytes, blocks,
                               ctypes.c_void_p(sink.data_ptr()), ctypes.c_void_p(stream.cuda_stream))
            if rc != 0:
                raise RuntimeError(f"sasp_read failed ({rc})")
        us = _probe_time(args, stream, launch)
        res[blocks] = {"us_per_launch": us, "gbps": set_bytes / us / 1e3}
    best = max(res.values(), key=lambda r: r["gbps"])
    print(json.dumps({"probe": "streaming read (sasp_read)", "bytes_per_launch": set_bytes, "sets": nsets,
                      "by_blocks": res, "best_us": best["us_per_launch"], "best_gbps": best["gbps"],
                      "frac": best["gbps"] / HBM_PEAK_GBPS}), flush=True)
    return 0


MASK_PROBE_MODES = {0: "every float4, loads issued with the mask's", 5: "every float4, after the mask words",
                    1: "float4s whose 16 B hold an allowed id", 4: "float4s whose 32 B span holds an allowed id",
                    3: "float4s whose 64 B span holds an allowed id", 2: "float4s whose 128 B line holds an allowed id"}


def mask_probe(args) -> int:
    """Whether a grammar mask can cut the logits' HBM bytes: sasp_masked_read
    over C3's logits and masks (128 rows x 262,144 ids, densities 0.5-20 %),
    reading every float4 or only those whose 16/32/64/128-byte span holds an
    allowed id.  With --mask-probe-mode M only that mode runs (one kernel
    per process, for rocprofv3 --pmc).  Prints one JSON line."""
    import ctypes

    import numpy as np
    import torch

    from shared_amd import workloads as W

    lib = _probe_lib()
    first = W.c3()
    set_bytes = first.rows * first.vocab * 4 + first.mask.nbytes
    nsets = max(2, int(np.ceil(args.min_set_mb * 1e6 / set_bytes)))
    batches = [first] + [W.c3(seed=1000 + i) for i in range(1, nsets)]
    logits = [torch.from_numpy(np.ascontiguousarray(b.logits)).cuda() for b in batches]
    masks = [torch.from_numpy(np.ascontiguousarray(b.mask).view(np.int32)).cuda() for b in batches]
    # the fraction of each span size that holds an allowed id (what a skipping read must still fetch)
    words = first.mask.astype(np.uint64)
    touched = {}
    for ids in (4, 8, 16, 32):
        per = 32 // ids
        spans = (words[..., None] >> (np.arange(per, dtype=np.uint64) * ids)) & np.uint64((1 << ids) - 1)
        touched[f"{ids * 4}B"] = float((spans != 0).mean())
    sink = torch.zeros(256, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()
    modes = [args.mask_probe_mode] if args.mask_probe_mode >= 0 else [0, 5, 1, 4, 3, 2]
    res = {}
    for mode in modes:
        def launch(i):
            j = i % nsets
            rc = lib.sasp_masked_read(ctypes.c_void_p(logits[j].data_ptr()), ctypes.c_void_p(masks[j].data_ptr()),
                                      first.rows, first.vocab, mode, ctypes.c_void_p(sink.data_ptr()),
                                      ctypes.c_void_p(stream.cuda_stream))
            if rc != 0:
                raise RuntimeError(f"sasp_masked_read failed ({rc})")
        us = _probe_time(args, stream, launch)
        res[mode] = {"reads": MASK_PROBE_MODES[mode], "us_per_launch": us, "gbps": set_bytes / us / 1e3}
    print(json.dumps({"probe": "mask-predicated read (sasp_masked_read)", "bytes_per_launch": set_bytes,
                      "sets": nsets, "spans_touched": touched, "by_mode": res}), flush=True)
    return 0


def traffic_from_profiles(workload: str, kernel: str = KERNEL):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    scaled by the copy-kernel calibration), if a summary for this workload is
    committed under profiles/."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_{workload}_pmc.md")
    try:
        with open(path) as f:
            for line in f:
                m = re.match(r"\s*traffic_bytes_per_launch:\s*([0-9.eE+]+)", line)
                if m:
                    return float(m.group(1))
    except OSError:
        pass
    return None


def cpu_baseline(batch, target_s: float) -> dict:
    """Time the Node restatement of the reference JS path (oracle/sample_js.js)
    on a bounded sample of the same workload: the first set's rows, repeated
    until about target_s seconds of single-thread work (the reference samples
    on one JS thread), then the same rows split over worker_threads on the
    box's CPU share, and configuration C1 (the case the reference runs on the
    CPU) single-threaded.  Falls back to the C restatement when Node is
    absent."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import oracle as O
    from shared_amd import workloads as W

    if O.node_binary() is not None:
        with tempfile.TemporaryDirectory(prefix="sas_cpu_") as tmp:
            _, probe = O.run_node(batch, threads=1, repeat=1, workdir=tmp)
            repeat = max(1, min(50, int(round(target_s / max(probe["median_s"], 1e-3)))))
            out, t = O.run_node(batch, threads=1, repeat=repeat, workdir=tmp)
            threads = max(1, min(CPU_THREADS, os.cpu_count() or 1))
            _, tp = O.run_node(batch, threads=threads, repeat=max(3, repeat // 2), workdir=tmp)
        c1 = W.c1()
        with tempfile.TemporaryDirectory(prefix="sas_cpu_c1_") as tmp:
            _, t1 = O.run_node(c1, threads=1, repeat=20, workdir=tmp)
        return {"value": batch.rows / t["median_s"], "unit": "rows/s", "cores": 1, "kind": "port",
                "sample": f"{batch.rows} rows of the first input set, {repeat} timed passes (median), "
                          f"Node {t['node']} single thread on {t['cpu_model']} ({t['host_cpus']} host cpus)",
                "parallel": {"value": batch.rows / tp["median_s"], "unit": "rows/s", "cores": tp["threads"],
                             "sample": f"the same rows split over {tp['threads']} worker_threads, "
                                       f"{tp['repeat']} passes (median)"},
                "c1": {"value": 1.0 / t1["median_s"], "unit": "rows/s", "ms_per_row": t1["median_s"] * 1e3,
                       "cores": 1, "sample": "configuration C1 (greedy + repetition 1.1, vocab 151936, one row, "
                                             "512 history ids), 20 passes (median)"},
                "ids": out["ids"]}
    import time
    t0 = time.perf_counter()
    o = O.sample_rows(batch, threads=1)
    dt = time.perf_counter() - t0
    return {"value": batch.rows / dt, "unit": "rows/s", "cores": 1, "kind": "port",
            "sample": f"{batch.rows} rows of the first input set, C restatement single thread (Node absent)",
            "ids": np.asarray(o["ids"])}


def timed_steps(args, stream, issue) -> dict:
    """Times args.steps calls of issue(i, stream): one HIP event pair on
    `stream` around all of them (the timed region), then a second pass of
    max(args.steps, 200) calls with an event after every step (or graph
    replay), whose per-step times give the median.  With --graph-steps N, N
    calls (i = 0 .. N-1) are recorded into one HIP graph by stream capture
    and the graph is replayed (a replay's time / N is each of its steps);
    args.steps is rounded down to a multiple of N.  Returns {"mean_ms": the
    timed region / args.steps, "total_ms", "median_ms", "events_mean_ms":
    the second pass's mean, "samples"}; an event record between steps costs
    time of its own, which events_mean_ms - mean_ms shows."""
    import statistics

    import torch
    per = args.graph_steps
    g = None
    if per > 0:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            cs = torch.cuda.current_stream()
            for i in range(per):
                issue(i, cs)
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize()
        args.steps = max(1, args.steps // per) * per

    def one(k):
        if g is not None:
            g.replay()
        else:
            issue(k, stream)
    n = args.steps // per if g is not None else args.steps
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for k in range(n):
        one(k)
    end.record(stream)
    torch.cuda.synchronize()
    total = start.elapsed_time(end)
    m = max(n, -(-200 // (per if g is not None else 1)))
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(m + 1)]
    ev[0].record(stream)
    for k in range(m):
        one(k)
        ev[k + 1].record(stream)
    torch.cuda.synchronize()
    div = per if g is not None else 1
    each = [ev[k].elapsed_time(ev[k + 1]) / div for k in range(m)]
    return {"mean_ms": total / args.steps, "total_ms": total, "median_ms": statistics.median(each),
            "events_mean_ms": ev[0].elapsed_time(ev[m]) / (m * div), "samples": m}


def timing_doc(t: dict, args) -> dict:
    return {"ms_per_step_median": t["median_ms"], "ms_per_step_mean_with_events": t["events_mean_ms"],
            "event_pairs": t["samples"],
            "rule": "ms_per_step and value: the timed region of --steps back-to-back steps between one HIP event "
                    "pair (its mean); ms_per_step_median: a second pass with an event recorded after every step "
                    "(each graph replay / its steps with --graph-steps), the median over those pairs; an event "
                    "between steps adds its own time, as ms_per_step_mean_with_events shows"}


def launch_doc(args) -> str:
    return f"HIP graph of {args.graph_steps} steps, replayed" if args.graph_steps > 0 else "stream launches"


def verify_bytes(inp) -> int:
    """Compulsory HBM bytes of one verify step as the C ABI takes it: every
    target and draft logit row once, one mask row per position (read once,
    it applies to the target and the draft row of that position), the draft
    ids and the two uniforms per position, the tokens and the accepted counts
    written once."""
    seqs, L, vocab = inp["seqs"], inp["drafts"], inp["vocab"]
    b = inp["target"].nbytes + inp["draft"].nbytes
    if inp.get("mask") is not None:
        b += seqs * (L + 1) * ((vocab + 31) // 32) * 4
    return b + seqs * (L * 4 + (L + 1) * 16 + (L + 1) * 4 + 4)


def bench_verify(args) -> int:
    """C5: sas_verify steps (three launches each) over rotating input sets."""
    import time

    import numpy as np
    import torch

    from shared_amd import Sampler
    from shared_amd import workloads as W

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    first = W.c5()
    set_bytes = verify_bytes(first)
    nsets = max(2, int(np.ceil(args.min_set_mb * 1e6 / set_bytes)))
    sets_h = [first] + [W.c5(seed=1000 + i) for i in range(1, nsets)]
    base = None
    if not args.no_cpu_baseline and args.cpu_seconds > 0:
        import oracle as O
        t0 = time.perf_counter()
        O.verify(first)
        one = time.perf_counter() - t0
        reps = max(1, min(20, int(round(args.cpu_seconds / max(one, 1e-3)))))
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            O.verify(first)
            times.append(time.perf_counter() - t0)
        med = sorted(times)[len(times) // 2]
        base = {"value": first["seqs"] / med, "unit": "sequences/s", "cores": 1, "kind": "port",
                "sample": f"the first input set ({first['seqs']} sequences), {reps} passes (median), the C "
                          "restatement of rejection sampling (oracle/sampler_oracle.c), single thread"}
    if not torch.cuda.is_available():
        print("bench.py: no HIP device is visible", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)

    def dev(a, view=None):
        t = torch.from_numpy(np.ascontiguousarray(a))
        return (t.view(view) if view is not None else t).cuda()

    sets = []
    for inp in sets_h:
        sets.append(dict(target=dev(inp["target"]), draft=dev(inp["draft"]),
                         draft_ids=dev(np.ascontiguousarray(inp["draft_ids"], np.uint32), torch.int32),
                         uniforms=dev(np.ascontiguousarray(inp["uniforms"], np.float64)),
                         mask=dev(np.ascontiguousarray(inp["mask"], np.uint32), torch.int32)))
    seqs, L, vocab = first["seqs"], first["drafts"], first["vocab"]
    toks = [torch.empty((seqs, L + 1), dtype=torch.int32, device="cuda") for _ in sets]
    acc = [torch.empty(seqs, dtype=torch.int32, device="cuda") for _ in sets]
    stream = torch.cuda.current_stream()
    with Sampler(0) as s:
        def step(i, st_stream=stream):
            j = i % nsets
            st = sets[j]
            s.verify_into(st["target"], st["draft"], st["draft_ids"], st["uniforms"], toks[j], acc[j],
                          temperature=first["temperature"], mask=st["mask"], vocab=vocab, stream=st_stream)
        for i in range(args.warmup):
            step(i)
        torch.cuda.synchronize()
        t = timed_steps(args, stream, step)
    ms_step = t["mean_ms"]
    achieved = set_bytes / (ms_step * 1e-3) / 1e9
    line = {
        "metric": METRIC, "value": seqs / (ms_step / 1e3), "unit": "sequences/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_step, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"C5: {WORKLOAD_DOC['C5']}", "sequences": seqs, "drafts": L, "vocab": vocab,
                   "input_sets": nsets, "rotating_set_mb": round(nsets * set_bytes / 1e6, 1),
                   "launch": launch_doc(args)},
        "timing": timing_doc(t, args),
        "gbps": achieved,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": traffic_from_profiles("C5", "verify_step"),
                     "kernel": "sas::verify_stats_kernel + verify_decide_kernel + verify_draw_kernel (one step)",
                     "algorithmic_bytes_per_launch": set_bytes},
        "cpu_baseline": base,
    }
    print(json.dumps(line), flush=True)
    return 0


def bench_lm_head(args) -> int:
    """LMH1 / LMH3: sas_lm_head_sample steps (three launches: the head with
    the parts pass, the part groups, the merge).  The 1.34 GB head exceeds
    the Infinity Cache, so one input set is read from HBM every step."""
    import numpy as np
    import torch

    from shared_amd import Sampler
    from shared_amd import workloads as W

    rows = int(args.workload[3:])
    quant = args.workload.startswith("LMQ")
    b = W.lmhq(W.HEAD_Q6_K, rows=rows) if quant else W.lmh(rows=rows)
    set_bytes = b.algorithmic_bytes()
    base = None
    if not args.no_cpu_baseline and args.cpu_seconds > 0:
        import time
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O

        def cpu_step():
            lo = O.lm_head_q_logits(b.fmt, b.hidden, b.weight_q) if quant else O.lm_head_logits(b.hidden, b.weight_bits)
            O.sample_rows(b.with_logits(lo), threads=1)
        t0 = time.perf_counter()
        cpu_step()
        one = time.perf_counter() - t0
        reps = max(1, min(10, int(round(args.cpu_seconds / max(one, 1e-3)))))
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            cpu_step()
            times.append(time.perf_counter() - t0)
        med = sorted(times)[len(times) // 2]
        base = {"value": rows / med, "unit": "rows/s", "cores": 1, "kind": "port",
                "sample": f"the whole step ({rows} row(s), vocab {b.vocab}, dim {b.dim}), {reps} passes (median): "
                          "the C restatement of the head's dot products ("
                          + ("orc_lm_head_q_logits: Q8_1 operand, integer block dots" if quant else
                             "orc_lm_head_logits, eight FMA chains per id")
                          + ") then of the sampling step (oracle/sampler_oracle.c), single thread"}
    if not torch.cuda.is_available():
        print("bench.py: no HIP device is visible", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)

    def dev(a, view=None):
        if a is None:
            return None
        t = torch.from_numpy(np.ascontiguousarray(a))
        return (t.view(view) if view is not None else t).cuda()

    hidden = dev(b.hidden)
    weight = dev(b.weight_q) if quant else dev(b.weight_bits.view(np.int16))
    fmt = b.fmt
    kw = dict(mask=dev(b.mask, torch.int32), hist_ids=dev(b.hist_ids, torch.int32),
              hist_offsets=dev(b.hist_offsets), uniforms=dev(b.uniforms), params=b.params)
    out_ids = torch.empty(rows, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()
    with Sampler(0) as s:
        for _ in range(args.warmup):
            s.lm_head_sample_into(hidden, weight, out_ids, stream=stream, fmt=fmt, **kw)
        torch.cuda.synchronize()
        t = timed_steps(args, stream,
                        lambda i, st: s.lm_head_sample_into(hidden, weight, out_ids, stream=st, fmt=fmt, **kw))
    ms_step = t["mean_ms"]
    achieved = set_bytes / (ms_step * 1e-3) / 1e9
    line = {
        "metric": METRIC, "value": rows / (ms_step / 1e3), "unit": "rows/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_step, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "Q6_K x Q8_1 int8 dots, f32 scales" if quant else "f32 (bf16 head widened to f32)", "data": "synthetic",
        "config": {"workload": f"{args.workload}: {WORKLOAD_DOC[args.workload]}", "rows": rows,
                   "vocab": b.vocab, "dim": b.dim, "top_k": b.params.top_k, "top_p": b.params.top_p,
                   "temperature": b.params.temperature, "softcap": b.params.softcap, "launch": launch_doc(args)},
        "timing": timing_doc(t, args),
        "gbps": achieved,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": traffic_from_profiles(args.workload, "lm_head"),
                     "head_format": W.HEAD_NAMES[fmt], "head_bytes": int(b.weight.nbytes),
                     "kernel": "sas::lmh_parts_kernel + lmh_group_kernel + sample_merge_kernel (one step)",
                     "algorithmic_bytes_per_launch": set_bytes},
        "cpu_baseline": base,
    }
    print(json.dumps(line), flush=True)
    return 0


def main() -> int:
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "rows shard across GPUs with no exchange, so run one process per GPU.", file=sys.stderr)
        return 2
    if args.calibrate_copy_mb > 0:
        return calibrate_copy(args.calibrate_copy_mb, min(args.steps, 50))
    if args.stream_probe:
        return stream_probe(args)
    if args.memset_order_probe:
        return memset_order_probe(args)
    if args.mask_probe:
        return mask_probe(args)
    if args.workload == "C5":
        return bench_verify(args)
    if args.workload.startswith("LMH") or args.workload.startswith("LMQ"):
        return bench_lm_head(args)

    import numpy as np

    from shared_amd import workloads as W

    gen = W.CONFIGS[args.workload]
    first = gen()
    set_bytes = first.algorithmic_bytes()
    nsets = max(2, int(np.ceil(args.min_set_mb * 1e6 / set_bytes)))
    batches = [first] + [gen(seed=1000 + i) for i in range(1, nsets)]

    # CPU baseline before the GPU is touched (its Node child never sees HIP).
    base = None
    if not args.no_cpu_baseline and args.cpu_seconds > 0:
        base = cpu_baseline(first, args.cpu_seconds)

    import torch

    from shared_amd import Sampler
    from shared_amd._capi import FLAG_TOPP_EDGE

    if not torch.cuda.is_available():
        print("bench.py: no HIP device is visible", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)

    def dev(a, view=None):
        if a is None:
            return None
        t = torch.from_numpy(np.ascontiguousarray(a))
        return (t.view(view) if view is not None else t).cuda()

    sets = []
    for b in batches:
        sets.append(dict(logits=dev(b.logits), vocab=b.vocab, mask=dev(b.mask, torch.int32),
                         hist_ids=dev(b.hist_ids, torch.int32), hist_offsets=dev(b.hist_offsets),
                         uniforms=dev(b.uniforms), params=b.params))
    rows, vocab = first.rows, first.vocab
    if args.row_params:
        from shared_amd import pack_params
        from shared_amd.sampler import row_hints
        plist = [first.params] * rows
        rp = dev(pack_params(plist).view(np.uint8))
        for st in sets:
            st["row_params"] = rp
            st["row_hints"] = row_hints(plist)
    out_ids = [torch.empty(rows, dtype=torch.int32, device="cuda") for _ in sets]
    stream = torch.cuda.current_stream()

    with Sampler(0) as s:
        s.reserve(rows, vocab)
        # untimed: the rows whose top-p running mass lies within 1e-6 of top_p
        # (SAS_FLAG_TOPP_EDGE), over every input set
        flags = torch.empty(rows, dtype=torch.int32, device="cuda")
        edge_rows = 0
        for j in range(nsets):
            s.sample_into(out_ids=out_ids[j], out_flags=flags, stream=stream, **sets[j])
            edge_rows += int(((flags & FLAG_TOPP_EDGE) != 0).sum().item())
        for i in range(args.warmup):
            j = i % nsets
            s.sample_into(out_ids=out_ids[j], stream=stream, **sets[j])
        torch.cuda.synchronize()
        # the handle's scratch is sized by reserve() and the calls above, so
        # a captured call records kernel launches only
        t = timed_steps(args, stream,
                        lambda i, st: s.sample_into(out_ids=out_ids[i % nsets], stream=st, **sets[i % nsets]))
        gpu_ids0 = out_ids[0].cpu().numpy().view(np.uint32)

    ms_step = t["mean_ms"]
    value = rows / (ms_step / 1e3)
    achieved = set_bytes / (ms_step * 1e-3) / 1e9
    traffic = traffic_from_profiles(args.workload)
    line = {
        "metric": METRIC,
        "value": value,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"{args.workload}: {WORKLOAD_DOC[args.workload]}", "rows": rows, "vocab": vocab,
                   "top_k": first.params.top_k, "top_p": first.params.top_p,
                   "temperature": first.params.temperature, "input_sets": nsets,
                   "rotating_set_mb": round(nsets * set_bytes / 1e6, 1),
                   "params": "per row (row_params)" if args.row_params else "one sas_params for every row",
                   "launch": launch_doc(args)},
        "timing": timing_doc(t, args),
        "topp_edge_rows": {"rows": edge_rows, "of": nsets * rows,
                           "rule": "top-p running mass within 1e-6 of top_p (SAS_FLAG_TOPP_EDGE)"},
        "gbps": achieved,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": traffic,
                     "kernel": "sas::sample_parts_kernel + sas::sample_merge_kernel (one step: two launches)",
                     "algorithmic_bytes_per_launch": set_bytes},
        "cpu_baseline": None,
    }
    if base is not None:
        ids = base.pop("ids")
        base["ids_match_gpu"] = f"{int((ids == gpu_ids0).sum())}/{rows}"
        line["cpu_baseline"] = base
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
