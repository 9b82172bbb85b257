#!/usr/bin/env python3
"""Benchmark of the alignment hot path on one MI355X.

Workload: config C2 (B=64 wav2vec2-char-shaped records, T~U{250..1750}, V=32,
peaky synthetic emissions), optimized mode, inputs resident in HBM. A step is
one ``align`` call over the whole batch (host preparation, descriptor upload,
kernels); K steps run back to back with no host synchronization in between.

Prints one JSON line: aligned frames/s as ``value`` (the median of five passes
of K steps), DP cells/s, the dominant kernel's HBM roofline fraction (kernel
duration from HIP events recorded on the launch stream around that kernel in
five further passes of K steps, kept out of the throughput passes because the
event records are host work), the same figures for conventional mode, and a CPU
baseline (conventional-mode alignment on the host cores, a bounded sample of
the same batch: the reference's own CPU comparator where it was built, else the
C oracle).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for path in (REPO, REPO / "fast-forced-aligner_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))

METRIC = "aligned frames/sec + DP cells/sec on 1 MI355X; % of HBM roofline"
HBM_PEAK_GBS = 8000.0


HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000  # hip_runtime_api.h: timing-only events, no cache writeback


def hip_runtime():
    lib = ctypes.CDLL("libamdhip64.so.7")
    lib.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
    lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
    lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    return lib


_SLEEP_CYCLES_PER_US = None


def hold_stream(us):
    """Keeps the current stream busy for about `us` microseconds with torch's
    bounded spin kernel, so that the launches enqueued behind it are all in
    the queue before the GPU reaches them. Event pairs around a kernel then
    time the kernel itself, not how long the host took to submit it (without
    this, a GPU that outruns the host starts the timing event early)."""
    import torch

    global _SLEEP_CYCLES_PER_US
    if _SLEEP_CYCLES_PER_US is None:
        torch.cuda._sleep(100000)  # warm the spin kernel
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        torch.cuda._sleep(1000000)
        b.record()
        b.synchronize()
        _SLEEP_CYCLES_PER_US = 1000000 / max(a.elapsed_time(b) * 1e3, 1.0)
    torch.cuda._sleep(int(us * _SLEEP_CYCLES_PER_US))


def measure(capi_lib, hip, call, steps, warmup, repeats=5):
    """Pipelined wall time per call of `call` (an align entry): `repeats`
    passes of `steps` calls back to back with nothing else on the host between
    them, each pass bracketed by two synchronizations; the median pass. Then
    the average duration of its dominant kernel, from timing-only HIP events
    armed around that kernel in `repeats` further passes of `steps` calls (the
    event records are host work of their own, so they stay out of the
    throughput passes; the stream is held while they are enqueued, so that
    each event pair times its kernel rather than the host's submission); the
    median pass."""
    import statistics

    import torch

    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    passes = []
    for _ in range(repeats):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            call()
        torch.cuda.synchronize()
        passes.append((time.perf_counter() - t0) / steps)
    kernel_passes = []
    result = None
    for _ in range(repeats):
        starts, stops = [], []
        for _ in range(steps):
            a, b = ctypes.c_void_p(), ctypes.c_void_p()
            assert hip.hipEventCreateWithFlags(ctypes.byref(a), HIP_EVENT_DISABLE_SYSTEM_FENCE) == 0
            assert hip.hipEventCreateWithFlags(ctypes.byref(b), HIP_EVENT_DISABLE_SYSTEM_FENCE) == 0
            starts.append(a)
            stops.append(b)
        torch.cuda.synchronize()
        hold_stream(steps * 60.0)
        for i in range(steps):
            capi_lib.ffa_profile_next_launch(starts[i], stops[i])
            result = call()
        torch.cuda.synchronize()
        kernel_ms = []
        for a, b in zip(starts, stops):
            ms = ctypes.c_float()
            assert hip.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
            kernel_ms.append(ms.value)
            hip.hipEventDestroy(a)
            hip.hipEventDestroy(b)
        kernel_passes.append(sum(kernel_ms) / len(kernel_ms))
    return statistics.median(passes), statistics.median(kernel_passes), result


def launch_floor(capi_lib, hip, workgroups, steps):
    """Mean duration, timed like the dominant kernel (one timing-only event
    pair per launch, launches back to back on the current stream behind a
    held stream), of a kernel
    that does nothing, launched with the dominant kernel's workgroup count: the
    fixed cost of one dispatch under this timing method, beneath every
    measured kernel duration (the block size does not change it)."""
    import torch

    stream = torch.cuda.current_stream().cuda_stream
    pairs = []
    for _ in range(steps):
        a, b = ctypes.c_void_p(), ctypes.c_void_p()
        assert hip.hipEventCreateWithFlags(ctypes.byref(a), HIP_EVENT_DISABLE_SYSTEM_FENCE) == 0
        assert hip.hipEventCreateWithFlags(ctypes.byref(b), HIP_EVENT_DISABLE_SYSTEM_FENCE) == 0
        pairs.append((a, b))
    for _ in range(10):
        assert capi_lib.ffa_launch_floor(workgroups, 256, stream) == 0
    torch.cuda.synchronize()
    hold_stream(steps * 20.0)
    for a, b in pairs:
        assert hip.hipEventRecord(a, stream) == 0
        assert capi_lib.ffa_launch_floor(workgroups, 256, stream) == 0
        assert hip.hipEventRecord(b, stream) == 0
    torch.cuda.synchronize()
    total = 0.0
    for a, b in pairs:
        ms = ctypes.c_float()
        assert hip.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        total += ms.value
        hip.hipEventDestroy(a)
        hip.hipEventDestroy(b)
    return total / steps * 1e3


def measured_traffic(config, mode, kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summaries (a line
    `traffic_bytes_per_launch[<config> <mode> <kernel>] = <bytes>`), or None."""
    import re

    key = f"{config} {mode} {kernel}"
    for path in sorted((REPO / "profiles").glob("*traffic*.md")):
        for m in re.finditer(r"traffic_bytes_per_launch\[(.+?)\] = (\d+)", path.read_text()):
            if m.group(1) == key:
                return int(m.group(2))
    return None


def extras(ffa, es, ys, result, steps=100):
    """Pipelined per-call wall time of the path's neighbours on the same batch:
    emission_validity (the NaN/+inf scan in front of align) and token_spans
    (the timestamp epilogue after it)."""
    import torch

    def timed(fn):
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps

    scan_bytes = sum(e.numel() * 4 for e in es)
    t_scan = timed(lambda: ffa.emission_validity(es))
    span_bytes = result.labels.numel() * 8 + sum(int(y.numel()) for y in ys) * 16
    t_spans = timed(lambda: ffa.token_spans(result, ys))
    return {"emission_validity": {"us_per_call": t_scan * 1e6, "bytes": scan_bytes,
                                  "GB_per_s": scan_bytes / t_scan / 1e9},
            "token_spans": {"us_per_call": t_spans * 1e6, "bytes": span_bytes,
                            "GB_per_s": span_bytes / t_spans / 1e9}}


def logits_figures(ffa, capi_lib, hip, config, mode, steps=100):
    """The fused logits path (align_logits) on the same config's raw logits,
    beside the two unfused pipelines it replaces: torch's log_softmax per
    record then align (the reference callers' pipeline,
    examples/transformers_ctc/align.py:55-67), and this build's materialized
    log_softmax then align. Bytes: every logit read once (the normalizer needs
    the whole row), int64 label + fp32 score written per frame, targets read."""
    import torch

    from fast_forced_aligner import workloads

    raw = workloads.make(config, raw=True)
    xs = [torch.from_numpy(x).to("cuda:0") for x in raw.emissions]
    ys = [torch.from_numpy(y).to("cuda:0") for y in raw.targets]
    step_s, kernel_ms, fused = measure(capi_lib, hip, lambda: ffa.align_logits(xs, ys, mode=mode), steps, 10)
    plain = ffa.align(ffa.log_softmax(xs), ys, mode=mode)

    def bits(t):
        return t.view(torch.int32) if t.dtype == torch.float32 else t

    parity = all(torch.equal(bits(getattr(fused, f)), bits(getattr(plain, f)))
                 for f in ("labels", "scores", "status", "objective"))

    def timed(fn):
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps

    t_torch = timed(lambda: ffa.align([x.log_softmax(-1) for x in xs], ys, mode=mode))
    t_mat = timed(lambda: ffa.align(ffa.log_softmax(xs), ys, mode=mode))
    nbytes = sum(4 * x.size + 12 * x.shape[0] for x in raw.emissions) + sum(8 * y.size for y in raw.targets)
    achieved = nbytes / (kernel_ms * 1e-3) / 1e9
    return {"workload": f"{config} raw logits, {mode} mode", "us_per_call": step_s * 1e6,
            "frames_per_s": raw.frames / step_s, "kernel_us": kernel_ms * 1e3, "algorithmic_bytes": nbytes,
            "roofline_frac": achieved / HBM_PEAK_GBS,
            "torch_log_softmax_then_align_us": t_torch * 1e6, "log_softmax_then_align_us": t_mat * 1e6,
            "parity_vs_materialized": bool(parity)}


def cpu_model():
    """The host CPU's model name from /proc/cpuinfo (None where unreadable)."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(batch, seconds=10.0):
    """Conventional-mode CPU alignment of the same batch on the host cores, one
    record per task, repeated for about `seconds`. Prefers the reference's own
    CPU comparator (benchmarks/patches/cpu_corrected.cpp, built from the
    reference sources into oracle/_ref; same fp32 recurrence and tie rule as the
    reference's conventional mode; run on a thread pool as the reference's
    adapter does, benchmarks/adapters/cpp.py:86-117) when it was built and the
    batch lies in its domain; otherwise the C oracle's conventional DP."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    from oracle import oracle

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    cores = max(1, min(cores, 16))
    ref = oracle.reference_comparator()
    in_domain = all(y.size > 0 and e.shape[0] >= y.size + int((y[1:] == y[:-1]).sum()) + 2
                    for e, y in zip(batch.emissions, batch.targets))
    if ref is not None and in_domain:
        items = [(np.ascontiguousarray(e[None]), np.ascontiguousarray(y[None])) for e, y in
                 zip(batch.emissions, batch.targets)]
        pool = ThreadPoolExecutor(max_workers=cores)

        def run():
            list(pool.map(lambda item: ref.forced_align(item[0], item[1], 0), items))

        kind, what = "reference", "the reference's CPU comparator (cpu_corrected.cpp, oracle/_ref)"
    else:
        pool = None

        def run():
            oracle.align(batch.emissions, batch.targets, mode="conventional", threads=cores)

        kind, what = "port", "the C oracle's conventional DP"
    run()  # warm caches and the thread pool outside the timed region
    reps, t0 = 0, time.perf_counter()
    while True:
        run()
        reps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    elapsed = time.perf_counter() - t0
    if pool is not None:
        pool.shutdown()
    return {"value": batch.frames * reps / elapsed, "unit": "aligned frames/s", "cores": cores, "kind": kind,
            "cpu_model": cpu_model(), "dp_cells_per_s": batch.cells * reps / elapsed,
            "sample": f"{batch.name} full batch x{reps} ({elapsed:.1f} s), conventional DP, {what}, "
                      f"one record per task on {cores} threads"}


def line_bound(name: str) -> dict:
    """Line-granular HBM lower bound of a config's greedy reads: per record and
    frame, every L2 line (128 B) or memory sector (64 / 32 B) of the row that
    holds a transcript-alphabet column is fetched whole, plus the int64 label
    and fp32 score written per frame and the targets read once. Host only."""
    import numpy as np

    from fast_forced_aligner import workloads

    batch = workloads.make(name)
    lines = {128: 0, 64: 0, 32: 0}
    frames = 0
    for e, y in zip(batch.emissions, batch.targets):
        cols = np.unique(np.r_[y, 0])
        for g in lines:
            lines[g] += e.shape[0] * len(np.unique(cols // (g // 4))) * g
        frames += e.shape[0]
    rest = 12 * frames + 8 * sum(int(y.size) for y in batch.targets)
    return {"config": name, "algorithmic_bytes": batch.min_bytes(),
            **{f"bound_{g}B_lines": v + rest for g, v in lines.items()}}


def matrix(path: str) -> int:
    """Every config of BASELINE.json in both modes, with and without
    check_inputs, by the reference's timing contract (benchmarks/README.md:
    165-200 as restated for this path): inputs resident; single-call latency
    (host sync, one align, host sync) and pipelined time per call (K calls back
    to back, no sync in between), each the median of repeats; the dominant
    kernel's duration from HIP events; parity of labels, scores, status and
    objective with the CPU oracle, bit for bit; the oracle's conventional DP on
    the host cores as the CPU baseline. Writes a markdown table to `path` and
    prints one JSON line per row."""
    import statistics

    import numpy as np
    import torch

    import fast_forced_aligner as ffa
    from fast_forced_aligner import capi, workloads
    from oracle import oracle

    ffa.load_extension()
    capi_lib = capi.load()
    hip = hip_runtime()
    rows = []
    header = ("| Config | Mode | check_inputs | Single call (ms) | Pipelined (ms/call) | Aligned frames/s | "
              "DP cells/s | Dominant kernel (µs) | % HBM roofline | Parity vs oracle | CPU baseline frames/s |")
    for name in ("c1", "c2", "c3", "c4", "c5"):
        batch = workloads.make(name)
        es = [torch.from_numpy(e).to("cuda:0") for e in batch.emissions]
        ys = [torch.from_numpy(y).to("cuda:0") for y in batch.targets]
        cpu = cpu_baseline(batch, seconds=3.0)
        for mode in ("conventional", "optimized"):
            for check in (True, False):
                def call():
                    return ffa.align(es, ys, mode=mode, check_inputs=check)

                result = call()
                torch.cuda.synchronize()
                singles = []
                for _ in range(7):
                    t0 = time.perf_counter()
                    call()
                    torch.cuda.synchronize()
                    singles.append(time.perf_counter() - t0)
                single = statistics.median(singles)
                k = max(3, min(100, int(0.3 / single)))
                step, kernel_ms, result = measure(capi_lib, hip, call, k, 2, repeats=5)
                want = oracle.align(batch.emissions, batch.targets, mode=mode, check_inputs=check, threads=16)
                got = {f: getattr(result, f).cpu().numpy() for f in ("labels", "scores", "status", "objective")}
                parity = all(np.array_equal(got[f].view(np.int32) if got[f].dtype == np.float32 else got[f],
                                            want[f].view(np.int32) if want[f].dtype == np.float32 else want[f])
                             for f in got)
                frac = batch.min_bytes() / (kernel_ms * 1e-3) / 1e9 / HBM_PEAK_GBS
                row = {"config": name, "mode": mode, "check_inputs": check, "single_call_ms": single * 1e3,
                       "pipelined_ms": step * 1e3, "calls_per_repeat": k, "frames_per_s": batch.frames / step,
                       "dp_cells_per_s": batch.cells / step, "kernel_us": kernel_ms * 1e3,
                       "roofline_frac": frac, "parity_vs_oracle": parity, "cpu_frames_per_s": cpu["value"],
                       "cpu_cores": cpu["cores"], "records": len(es), "frames": batch.frames,
                       "algorithmic_bytes": batch.min_bytes()}
                print(json.dumps(row), flush=True)
                rows.append(row)
    lines = [header, "|" + "---|" * 11]
    for r in rows:
        lines.append(f"| {r['config'].upper()} ({r['records']} records, {r['frames']} frames) | {r['mode']} | "
                     f"{r['check_inputs']} | {r['single_call_ms']:.3f} | {r['pipelined_ms']:.3f} | "
                     f"{r['frames_per_s']:.3g} | {r['dp_cells_per_s']:.3g} | {r['kernel_us']:.1f} | "
                     f"{100 * r['roofline_frac']:.2f} | {'bit-exact' if r['parity_vs_oracle'] else 'MISMATCH'} | "
                     f"{r['cpu_frames_per_s']:.3g} ({r['cpu_cores']} threads) |")
    Path(path).write_text("\n".join(lines) + "\n")
    return 0 if all(r["parity_vs_oracle"] for r in rows) else 1


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5"])
    parser.add_argument("--mode", default="optimized", choices=["optimized", "conventional"])
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    parser.add_argument("--no-conventional", action="store_true", help="skip the conventional-mode figures")
    parser.add_argument("--no-extras", action="store_true",
                        help="skip the neighbouring entry points (emission scan, token spans, logits path)")
    parser.add_argument("--matrix", metavar="PATH",
                        help="instead of the bench line: measure every config in both modes (single-call and "
                             "pipelined times, kernel, roofline, parity, CPU baseline) and write a markdown table")
    parser.add_argument("--line-bound", metavar="CONFIG",
                        help="print the line-granular HBM lower bound of CONFIG's greedy reads and exit (host only)")
    parser.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                        help="after the timed work, run 10 plain device copies of MIB MiB (a known-size "
                             "reference for rocprofv3 FETCH_SIZE / WRITE_SIZE counter passes)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: the alignment path has no multi-GPU mode in this build "
              f"(records are independent; see DESIGN.md for how a batch would shard). Got --gpus {args.gpus}.",
              file=sys.stderr)
        return 2
    if args.matrix:
        return matrix(args.matrix)
    if args.line_bound:
        print(json.dumps(line_bound(args.line_bound)))
        return 0

    import numpy as np
    import torch

    import fast_forced_aligner as ffa
    from fast_forced_aligner import capi, workloads

    batch = workloads.make(args.config)
    dev = "cuda:0"
    es = [torch.from_numpy(e).to(dev) for e in batch.emissions]
    ys = [torch.from_numpy(y).to(dev) for y in batch.targets]
    ffa.load_extension()
    capi_lib = capi.load()
    hip = hip_runtime()
    min_bytes = batch.min_bytes()

    def figures(mode, steps, warmup):
        step_s, kernel_ms, result = measure(capi_lib, hip, lambda: ffa.align(es, ys, mode=mode), steps, warmup)
        achieved = min_bytes / (kernel_ms * 1e-3) / 1e9
        return step_s, kernel_ms, achieved, result

    # conventional mode cuts transcripts of more than 1,024 states into bands of
    # 256 states, one single-wave workgroup each (band_kernel, ffa_kernels.hip)
    states = [2 * len(y) + 1 for y in batch.targets]
    banded = args.mode == "conventional" and max(states) > 1024
    kernel_name = "chunk_kernel" if args.mode == "optimized" else "band_kernel" if banded else "conventional_kernel"
    # optimized mode runs each record's tail inside the chunk kernel (one launch
    # per call) for batches of log-probabilities with at most 1,024 chunks, at
    # most 4,096 states and no record of 2,048+ frames (the split tail's
    # batches); otherwise a tail kernel follows (align_launch, ffa_kernels.hip)
    chunks = sum((e.shape[0] + 127) // 128 for e in batch.emissions)
    fused_tail = (args.mode == "optimized" and chunks <= 1024 and max(e.shape[0] for e in batch.emissions) < 2048
                  and max(2 * len(y) + 1 for y in batch.targets) <= 4096)
    step_s, kernel_ms, achieved, result = figures(args.mode, args.steps, args.warmup)
    # parity spot check outside the timed region
    from oracle import oracle
    want = oracle.align(batch.emissions, batch.targets, mode=args.mode, threads=8)
    parity = bool(np.array_equal(result.labels.cpu().numpy(), want["labels"]) and
                  np.array_equal(result.scores.cpu().numpy().view(np.int32), want["scores"].view(np.int32)) and
                  np.array_equal(result.status.cpu().numpy(), want["status"]))
    line = {
        "metric": METRIC,
        "value": batch.frames / step_s,
        "unit": "aligned frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"{args.config}: {len(es)} records, {batch.frames} frames, V="
                               f"{batch.emissions[0].shape[1]}, {args.mode} mode",
                   "mode": args.mode, "records": len(es), "frames": batch.frames, "dp_cells": batch.cells},
        "dp_cells_per_s": batch.cells / step_s,
        "parity_vs_oracle": parity,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": measured_traffic(args.config, args.mode, kernel_name),
                     "kernel": kernel_name, "kernel_us": kernel_ms * 1e3, "algorithmic_bytes": min_bytes},
    }
    if args.mode == "optimized":
        line["roofline"]["tail"] = "fused" if fused_tail else "tail_kernel"
    # the same timing of an empty kernel with the dominant kernel's workgroup
    # count, and the fraction a kernel of exactly that duration would reach
    groups = 8 * ((sum((e.shape[0] + 127) // 128 for e in batch.emissions) + 7) // 8) \
        if args.mode == "optimized" else sum((s + 255) // 256 for s in states) if banded else len(es)
    floor_us = launch_floor(capi_lib, hip, groups, args.steps)
    line["roofline"]["launch_floor_us"] = floor_us
    line["roofline"]["frac_ceiling"] = min_bytes / (floor_us * 1e-6) / 1e9 / HBM_PEAK_GBS
    if not args.no_conventional and args.mode == "optimized":
        c_step, c_kernel_ms, c_achieved, _ = figures("conventional", max(10, args.steps // 10), 3)
        line["conventional"] = {"ms_per_step": c_step * 1e3, "frames_per_s": batch.frames / c_step,
                                "dp_cells_per_s": batch.cells / c_step, "kernel_us": c_kernel_ms * 1e3,
                                "roofline_frac": c_achieved / HBM_PEAK_GBS}
    if not args.no_extras:
        line["extras"] = extras(ffa, es, ys, result)
        line["extras"]["align_logits"] = logits_figures(ffa, capi_lib, hip, args.config, args.mode)
    line["cpu_baseline"] = None if args.no_cpu else cpu_baseline(batch)
    if args.calibrate_copy > 0:
        src = torch.ones(args.calibrate_copy << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        line["calibration_copy_bytes"] = src.numel() * 4
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
