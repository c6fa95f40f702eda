"""Benchmark of the fused FFN on one MI355X: fused FFN TFLOP/s and fraction of MFMA peak,
Basic vs Stream-K down-projection.

A step is one PreparedFFN.run() (up GEMM + GELU epilogue, then the down GEMM) over
one batch of seeded synthetic input already resident in HBM.  The headline
workload is the largest configuration, the DiT-style FFN (X [2,4096,3072] bf16,
W1 [12288,3072], W2 [3072,12288]), on which the 60%-of-MFMA-peak target is
stated; the other workloads are reported beside it.  ms_per_step follows
performance/collect.py:8-35 of the reference: warmup, then one device event pair
around every run(), median; the K timed runs of the Basic path, the Stream-K path
and torch's unfused path are taken in alternating rounds (time_interleaved), so
that all three see the same stretch of the GPU's power and thermal state
(memory-bound workloads path by path, each warm time with its own weights in the
last-level cache; their cold times are timed apart).  The
mean of the same steps issued back to back under
one event pair is reported beside it (it leaves out the host's per-call launch
gap).  Each path also reports max_abs, rms and mean_rel of its own output against
the FP32 golden on a seeded sample of output rows.

Prints ONE JSON line.  --gpus above 1 is refused: this operator runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

METRIC = "fused FFN TFLOP/s (4·M·K·H-equiv FLOPs) and % of MFMA peak, Basic vs Stream-K"
MFMA_PEAK_TFLOPS = 2500.0   # MI355X dense FP16/BF16 MFMA, published
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, published
HEADLINE = "c5_dit_bf16"
EXTRA = ("c2_aligned_bf16", "c4_decode_bf16", "c3_unaligned_fp16", "c1_smoke_fp16",
         "c5_tp8_shard_bf16", "c4_tp8_shard_bf16")   # last two: one GPU's share of an H split over 8


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--case", default=HEADLINE)
    p.add_argument("--no-extra", action="store_true", help="headline workload only")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU oracle time budget")
    p.add_argument("--counters", action="store_true",
                   help="untimed pass for rocprofv3 --pmc: a copy of known size (calibration), "
                        "then each kernel of the workload's paths three times")
    return p.parse_args(argv)


def workload_numbers(case):
    from ffn_optim_amd.cases import case_problem
    p = case_problem(case)
    m, k, h, n = p.m, p.k, p.h, p.n
    esz = 2
    return {
        "m": m, "k": k, "h": h, "n": n,
        "flops_4mkh": 4.0 * m * k * h,
        "flops": 2.0 * m * h * (k + n),
        "flops_up": 2.0 * m * k * h,
        "flops_down": 2.0 * m * h * n,
        "bytes": float(esz * (m * k + h * k + n * h + m * n)),
        "bytes_up": float(esz * (m * k + h * k + m * h)),
        "bytes_down": float(esz * (m * h + n * h + m * n)),
    }


WARM_SECONDS = 0.2   # warmup floor: the GPU leaves its idle clocks within tens of milliseconds


def warm(fn, warmup):
    """`warmup` untimed calls, then untimed calls for at least WARM_SECONDS."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t_end = time.perf_counter() + WARM_SECONDS
    while time.perf_counter() < t_end:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()


def time_back_to_back(fn, steps, warmup):
    """Mean per-call device time (ms) of `steps` calls issued back to back under one event
    pair on the current stream (the stream the kernels are launched on)."""
    import torch
    warm(fn, warmup)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    end.synchronize()
    total = start.elapsed_time(end)
    return {"mean_ms": total / steps, "total_ms": total}


def time_per_step(fn, steps, warmup, flush=None):
    """One event pair around each of `steps` calls, after warm-up (performance/collect.py:8-35);
    `flush`, if given, runs before each call outside its event pair.  Median and mean (ms)."""
    import torch
    warm(fn, warmup)
    torch.cuda.synchronize()
    samples = []
    for _ in range(steps):
        if flush is not None:
            flush()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        fn()
        end.record()
        end.synchronize()
        samples.append(start.elapsed_time(end))
    torch.cuda.synchronize()
    return {"median_ms": statistics.median(samples), "mean_ms": statistics.fmean(samples),
            "total_ms": sum(samples)}


def time_interleaved(fns, steps, warmup, rounds=5):
    """Per-run timing of several paths in alternating rounds: every path gets exactly `steps`
    calls, each under its own event pair as in time_per_step, split over `rounds` rounds whose
    path order alternates (forward, then reversed), so that no path is timed only in a later,
    hotter or more power-limited stretch of the run than another.  Median and mean (ms) per path."""
    import torch
    names = list(fns)
    rounds = max(1, min(rounds, steps))
    if rounds > 1:
        for name in names:
            warm(fns[name], warmup)
    torch.cuda.synchronize()
    samples = {name: [] for name in names}
    for r in range(rounds):
        n = steps // rounds + (1 if r < steps % rounds else 0)
        for name in (names if r % 2 == 0 else names[::-1]):
            fn = fns[name]
            if rounds == 1:
                warm(fn, warmup)   # path by path: each warmed right before its own calls
            for _ in range(n):
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                start.record()
                fn()
                end.record()
                end.synchronize()
                samples[name].append(start.elapsed_time(end))
    torch.cuda.synchronize()
    return {name: {"median_ms": statistics.median(v), "mean_ms": statistics.fmean(v), "total_ms": sum(v),
                   "steps": len(v)} for name, v in samples.items()}


def accuracy_of(case, prepared, inputs):
    """max_abs, rms and mean_rel of the path's output on a seeded sample of rows against the
    FP32 golden (performance/run.py:198-219 records the same per case)."""
    import torch
    from ffn_optim_amd.performance.accuracy import compare, golden_rows, sample_rows
    x, w1, w2 = inputs
    out = prepared.run()
    torch.cuda.synchronize()
    m, n = x.numel() // x.shape[-1], w2.shape[0]
    rows = sample_rows(m)
    got = out.reshape(m, n)[rows.to(out.device)].cpu()
    res = compare(got, golden_rows(x.cpu(), w1.cpu(), w2.cpu(), rows))
    return {"rows": len(rows), "max_abs": res["max_abs"], "rms": res["rms"],
            "mean_rel": res["mean_rel"], "passed": res["passed"]}


def measure_path(case, down, steps, warmup, inputs, prepared=None):
    """Whole steps back to back, then the up and down kernels alone, for one down implementation
    (the per-run step time comes from time_interleaved)."""
    import ctypes
    import torch
    from ffn_optim_amd import _lib, prepare_ffn
    x, w1, w2 = inputs
    if prepared is None:
        prepared = prepare_ffn(x, w1, w2, down_impl=down)
    lib = _lib.load()
    plan = prepared.plan.native
    xs, w1s, w2s, hid, out, ws = prepared.tensors
    stream = torch.cuda.current_stream().cuda_stream

    torch.cuda.synchronize()
    step_b2b = time_back_to_back(prepared.run, steps, warmup)

    def up():
        lib.ffn_mi355x_up(ctypes.byref(plan), xs, w1s, hid, ws, stream)

    def dn():
        lib.ffn_mi355x_down(ctypes.byref(plan), hid, w2s, out, ws, stream)

    t_up = time_back_to_back(up, steps, warmup)
    t_dn = time_back_to_back(dn, steps, warmup)
    return prepared, step_b2b, t_up, t_dn


def traffic_from_profiles(kernel_tag, case_id):
    """HBM-side bytes per launch of one kernel role, measured with rocprofv3 --pmc (FETCH_SIZE and
    WRITE_SIZE, each scaled by what the counter reads for a copy of known size), read from the
    committed summary profiles/traffic_<case>.md if one exists."""
    path = REPO / "profiles" / f"traffic_{case_id}.md"
    if not path.exists():
        return None
    text = path.read_text()
    m = re.search(r"^hbm_bytes_per_launch\[" + re.escape(kernel_tag) + r"\]:\s*([0-9.eE+]+)", text, re.M)
    return float(m.group(1)) if m else None


def cpu_baseline(case, budget_s):
    """The oracle's torch FP32 path (validation/reference.py:16-23) on this host's cores."""
    import torch
    from ffn_optim_amd.cases import make_inputs
    from oracle.reference import ffn_torch
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    x, w1, w2 = make_inputs(case, "cpu")
    nums = workload_numbers(case)
    ffn_torch(x, w1, w2)  # warmup
    samples = []
    t_end = time.perf_counter() + budget_s
    while len(samples) < 3 or (time.perf_counter() < t_end and len(samples) < 50):
        t0 = time.perf_counter()
        ffn_torch(x, w1, w2)
        samples.append(time.perf_counter() - t0)
    med = statistics.median(samples)
    cpu = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": nums["flops_4mkh"] / med / 1e12, "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"{len(samples)} full runs of {case['case_id']} (median {med*1e3:.1f} ms, "
                      f"{sum(samples):.1f} s total) with torch FP32 on {threads} threads, {cpu}"}


COPY_BYTES = 512 << 20   # calibration copy: reads and writes exactly this many bytes


def counters_pass(case):
    """Launch sequence for a counter run: the calibration copy (torch's elementwise copy kernel
    over COPY_BYTES, so FETCH_SIZE/WRITE_SIZE of a kernel with known traffic can be read off),
    then up and down of both down paths, three times each, then torch's unfused path three
    times (the library comparison), all untimed."""
    import ctypes
    import torch
    import torch.nn.functional as F
    from ffn_optim_amd import _lib, prepare_ffn
    from ffn_optim_amd.cases import make_inputs
    src = torch.ones(COPY_BYTES // 4, device="cuda", dtype=torch.float32)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    x, w1, w2 = make_inputs(case, "cuda")
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    for down in ("basic", "streamk"):
        try:
            prepared = prepare_ffn(x, w1, w2, down_impl=down)
        except ValueError:
            continue
        plan = prepared.plan.native
        xs, w1s, w2s, hid, out, ws = prepared.tensors
        for _ in range(3):
            lib.ffn_mi355x_up(ctypes.byref(plan), xs, w1s, hid, ws, stream)
        for _ in range(3):
            lib.ffn_mi355x_down(ctypes.byref(plan), hid, w2s, out, ws, stream)
        torch.cuda.synchronize()
        print(f"counters pass: {case['case_id']} {down} up v{plan.up_variant} down v{plan.down_variant}",
              flush=True)
    # torch's unfused path on the same inputs (hipBLASLt GEMM, elementwise GELU, hipBLASLt GEMM),
    # three times, for the library comparison
    x2 = x.reshape(-1, x.shape[-1])
    for _ in range(3):
        F.gelu(x2 @ w1.t()) @ w2.t()
    torch.cuda.synchronize()
    print(f"counters pass: {case['case_id']} torch unfused", flush=True)


def cold_step_time(case, down, steps, inputs):
    """Per-step time with the 256 MiB MALL and the L2s flushed before every step (a 1 GiB
    scratch buffer is read between steps, which leaves only clean lines behind), for shapes
    whose weights would otherwise stay cached."""
    import torch
    from ffn_optim_amd import prepare_ffn
    x, w1, w2 = inputs
    prepared = prepare_ffn(x, w1, w2, down_impl=down)
    scratch = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
    t = time_per_step(prepared.run, steps, 3, flush=lambda: scratch.sum())
    del scratch
    return t


def library_path(case, steps, warmup, inputs):
    """torch's unfused eager path on the same inputs, as a callable timed like the fused path
    (time_interleaved): GEMM (hipBLASLt) -> F.gelu (exact) -> GEMM, with the hidden activation in
    the input dtype.  A same-run yardstick for the fused operator; the golden stays the FP32
    oracle."""
    import torch
    import torch.nn.functional as F
    x, w1, w2 = inputs
    x2 = x.reshape(-1, x.shape[-1])
    w1t, w2t = w1.t(), w2.t()

    def run():
        return F.gelu(x2 @ w1t) @ w2t

    return run


def library_record(case, step):
    """The bench record of torch's unfused path from its per-run timing."""
    nums = workload_numbers(case)
    ms = step["median_ms"]
    return {"ms_per_step": ms, "tflops_4mkh": nums["flops_4mkh"] / ms / 1e9,
            "path": "torch eager: x @ w1.T (hipBLASLt), F.gelu, @ w2.T (hipBLASLt)"}


def bench_case(case, steps, warmup):
    import torch
    from ffn_optim_amd.cases import make_inputs
    from ffn_optim_amd import prepare_ffn
    nums = workload_numbers(case)
    inputs = make_inputs(case, "cuda")
    x, w1, w2 = inputs
    res = {}
    preps = {}
    for down in ("basic", "streamk"):
        try:
            preps[down] = prepare_ffn(x, w1, w2, down_impl=down)
        except ValueError as exc:
            res[down] = {"status": "not_applicable", "reason": str(exc)}
    # per-run step times of both fused paths and torch's unfused path, interleaved
    fns = {down: p.run for down, p in preps.items()}
    fns["torch_unfused"] = library_path(case, steps, warmup, inputs)
    # A memory-bound workload's warm time depends on which weights the previous path left in the
    # last-level cache: time it path by path (one round), and compare its cold times.
    steps_of = time_interleaved(fns, steps, warmup, rounds=1 if case.get("memory_bound") else 5)
    for down, prepared in list(preps.items()):
        step = steps_of[down]
        prepared, step_b2b, t_up, t_dn = measure_path(case, down, steps, warmup, inputs, prepared)
        ms = step["median_ms"]
        res[down] = {
            "ms_per_step": ms,
            "ms_per_step_mean": step["mean_ms"],
            "ms_back_to_back": step_b2b["mean_ms"],
            "tflops_back_to_back": nums["flops_4mkh"] / step_b2b["mean_ms"] / 1e9,
            "tflops_4mkh": nums["flops_4mkh"] / ms / 1e9,
            "mfma_peak_frac": nums["flops_4mkh"] / ms / 1e9 / MFMA_PEAK_TFLOPS,
            "hbm_gbs": nums["bytes"] / ms / 1e6,
            "up_ms": t_up["mean_ms"], "down_ms": t_dn["mean_ms"],
            "up_tflops": nums["flops_up"] / t_up["mean_ms"] / 1e9,
            "down_tflops": nums["flops_down"] / t_dn["mean_ms"] / 1e9,
            "up_tile": [prepared.plan.up.bm, prepared.plan.up.bn, prepared.plan.up.bk],
            "down_tile": [prepared.plan.down.bm, prepared.plan.down.bn, prepared.plan.down.bk],
            "block_num": prepared.plan.block_num,
            "variants": [prepared.plan.up.variant, prepared.plan.down.variant],
            "accuracy": accuracy_of(case, prepared, inputs),
        }
        del prepared
        preps.pop(down)
        if case.get("memory_bound"):
            cold = cold_step_time(case, down, min(steps, 20), inputs)
            res[down].update(cold_ms_per_step=cold["median_ms"],
                             cold_hbm_gbs=nums["bytes"] / cold["median_ms"] / 1e6)
    res["torch_unfused"] = library_record(case, steps_of["torch_unfused"])
    torch.cuda.synchronize()
    return nums, res


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py: this operator runs on one GPU; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is design-only)", file=sys.stderr)
        return 2
    import torch
    from ffn_optim_amd.cases import get_case

    case = get_case(args.case)
    if args.counters:
        counters_pass(case)
        return 0
    nums, res = bench_case(case, args.steps, args.warmup)
    paths = {k: v for k, v in res.items() if k in ("basic", "streamk") and "ms_per_step" in v}
    if not paths:
        raise RuntimeError(f"no runnable path for {args.case}: {res}")
    best_down = min(paths, key=lambda k: paths[k]["ms_per_step"])
    best = paths[best_down]
    # dominant kernel of the best path
    if best["up_ms"] >= best["down_ms"]:
        kname, kms, kflops, ktag = "up GEMM + GELU", best["up_ms"], nums["flops_up"], "up"
    else:
        kname, kms, kflops, ktag = f"down GEMM ({best_down})", best["down_ms"], nums["flops_down"], f"down_{best_down}"
    achieved = kflops / kms / 1e9
    roofline = {"bound": "mfma", "achieved": achieved, "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": achieved / MFMA_PEAK_TFLOPS,
                "traffic": traffic_from_profiles(ktag, args.case),
                "kernel": kname, "kernel_ms": kms, "algorithmic_flops_per_launch": kflops}
    workloads = {}
    if not args.no_extra:
        for cid in EXTRA:
            if cid == args.case:
                continue
            c = get_case(cid)
            wn, wr = bench_case(c, max(10, args.steps // 2), args.warmup)
            workloads[cid] = {"flops_4mkh": wn["flops_4mkh"], "alg_bytes": wn["bytes"], **wr}
    line = {
        "metric": METRIC,
        "value": best["tflops_4mkh"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_floor_s": WARM_SECONDS,
        "ms_per_step": best["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if case["dtype"] == "bfloat16" else "fp16",
        "data": "synthetic: seeded randn, X ~ N(0,1), W1 ~ N(0,1/K), W2 ~ N(0,1/H)",
        "config": {"workload": f"{args.case}: X{case['shape']} W1{case['weight1_shape']} "
                               f"W2{case['weight2_shape']}",
                   "down_impl": best_down, "block_num": best["block_num"],
                   "mfma_peak_frac": best["mfma_peak_frac"]},
        "roofline": roofline,
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline(case, args.cpu_seconds),
        "paths": res,
        "workloads": workloads,
        "device": torch.cuda.get_device_name(0),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
