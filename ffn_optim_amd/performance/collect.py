"""Device timing and profiler evidence for one PreparedFFN (restates performance/collect.py).

time_prepared ranks candidates with unprofiled device events; capture_profile records a
separate single run with torch.profiler (ROCm kineto) and never feeds the ranking;
extract_summary reads rocprofv3 outputs (kernel trace, kernel stats, counter collection)
and extract_task_duration a Chrome trace.  Nothing here invents a metric: what a file
does not carry stays None.
"""
from __future__ import annotations

import csv
import json
import math
import statistics
from pathlib import Path

FFN_KERNEL = "ffn_"   # kernel-name fragment of every FFN kernel (ffn_gemm_kernel)


def _event_us(fn):
    """Device time of one fn() call on the current stream, in microseconds: an event pair around
    the call, waited for before returning (so calls never queue up behind each other)."""
    import torch
    pair = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    pair[0].record()
    fn()
    pair[1].record()
    pair[1].synchronize()
    return pair[0].elapsed_time(pair[1]) * 1000.0


def time_prepared(prepared, warmup=5, repeats=20, *, progress=None):
    """The harness's ranking time of one PreparedFFN: `warmup` untimed run() calls, then
    `repeats` calls with an event pair each; the median in microseconds (the protocol of
    performance/collect.py:8-35).  Returns device_median_us with the samples; a non-finite or
    non-positive sample refuses the candidate (RuntimeError)."""
    if warmup < 0 or repeats < 1:
        raise ValueError("warmup >= 0 and repeats >= 1 required")
    import torch
    say = progress or (lambda message: None)
    device = prepared.storage[0].device
    with torch.cuda.device(device):
        say(f"device warm-up: {warmup} runs")
        for _ in range(warmup):
            prepared.run()
        torch.cuda.synchronize(device)
        say(f"warm-up done, timing {repeats} runs")
        samples = [_event_us(prepared.run) for _ in range(repeats)]
    if not all(math.isfinite(v) and v > 0 for v in samples):
        raise RuntimeError("Invalid device timing; refusing to rank this candidate")
    return {"device_median_us": statistics.median(samples), "device_samples_us": samples,
            "warmup": warmup, "repeats": repeats, "task_duration_us": None,
            "pipeline_utilization": None,
            "profiler_note": "Unavailable until a profiler trace is captured and inspected"}


def time_interleaved(prepareds, rounds=9, batch=20, warmup=3):
    """Round-robin timing of several prepared FFNs on their common preparation stream.

    Each round times `batch` back-to-back run() calls of every candidate in turn with one
    event pair, so the clock drift of a long search and the host's per-call launch gap
    (which time_prepared's one-run event pairs include) do not decide between near-equal
    candidates.  Returns each candidate's median over the rounds of the per-run mean, in us."""
    if not prepareds or rounds < 1 or batch < 1 or warmup < 0:
        raise ValueError("candidates, rounds >= 1, batch >= 1 and warmup >= 0 required")
    import torch
    device = prepareds[0].storage[0].device
    means = [[] for _ in prepareds]
    with torch.cuda.device(device):
        for prepared in prepareds:
            for _ in range(warmup):
                prepared.run()
        torch.cuda.synchronize(device)
        for _ in range(rounds):
            for slot, prepared in enumerate(prepareds):
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                start.record()
                for _ in range(batch):
                    prepared.run()
                end.record()
                end.synchronize()
                means[slot].append(start.elapsed_time(end) * 1000 / batch)
    if any(not math.isfinite(v) or v <= 0 for row in means for v in row):
        raise RuntimeError("Invalid device timing; refusing to rank these candidates")
    return [statistics.median(row) for row in means]


def capture_profile(prepared, directory):
    """Separate pass: record one FFN run with torch.profiler and export a Chrome trace to
    directory/trace.json (performance/collect.py:38-74).  Hardware counters need a
    rocprofv3 --pmc run of the process instead; see extract_summary."""
    import torch
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=False)
    activities = [torch.profiler.ProfilerActivity.CPU, torch.profiler.ProfilerActivity.CUDA]
    with torch.cuda.device(prepared.storage[0].device):
        torch.cuda.synchronize()
        with torch.profiler.profile(activities=activities, record_shapes=False) as prof:
            prepared.run()
            torch.cuda.synchronize()
    trace = directory / "trace.json"
    prof.export_chrome_trace(str(trace))
    return {"profiler_path": str(directory),
            "profiler_note": "torch.profiler device trace of one run; counters need rocprofv3 --pmc"}


def _median(values):
    return statistics.median(values) if values else None


def _rows(path):
    with open(path, newline="") as stream:
        return list(csv.DictReader(stream))


def kernels_per_run(plan):
    """Kernel launches of one FFN under a plan: the up GEMM and the down GEMM.  A split up GEMM
    and a Stream-K down finish their split tiles inside the same launch."""
    return 2


def _group_runs(rows, per_run):
    """Summed duration (us) of each FFN run in a time-ordered list of kernel dispatches.

    With per_run (the launch count of one FFN, kernels_per_run) the dispatches are cut
    into consecutive groups of that size; a trailing partial group is dropped.  Without
    it a new run starts wherever the first kernel name recurs, which miscounts a plan
    whose split up GEMM and Stream-K down GEMM are the same kernel instantiation."""
    durs = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0 for r in rows]
    if per_run:
        return [sum(durs[i:i + per_run]) for i in range(0, len(durs) - per_run + 1, per_run)]
    first, runs, cur = rows[0]["Kernel_Name"], [], None
    for r, dur in zip(rows, durs):
        if r["Kernel_Name"] == first and cur is not None:
            runs.append(cur)
            cur = None
        cur = dur if cur is None else cur + dur
    runs.append(cur)
    return runs


def extract_summary(directory, kernel_name=FFN_KERNEL, kernels_per_run=None):
    """Durations and counters of the FFN kernels from rocprofv3 CSV outputs under directory.

    task_duration_us: median over runs of the summed durations of the matching kernels of
    one FFN, from *kernel_trace.csv (per dispatch; dispatches are grouped into runs of
    kernels_per_run launches, or, when that is not given, by recurrence of the first
    matching kernel name) or, failing that, the summed AverageNs of matching rows of
    *kernel_stats.csv.  pipeline_utilization: 'mfma_busy' per matching kernel when
    SQ_VALU_MFMA_BUSY_CYCLES and GRBM_GUI_ACTIVE were collected, as busy cycles over
    (SIMDs x GRBM_GUI_ACTIVE / XCDs) with the SIMD and XCD counts of *agent_info.csv; raw
    counter medians are kept under 'counters'.  Files of other schemas are ignored.
    """
    directory = Path(directory)
    traces = sorted(directory.rglob("*kernel_trace.csv"))
    stats = sorted(directory.rglob("*kernel_stats.csv"))
    counters = sorted(directory.rglob("*counter_collection.csv"))
    agents = sorted(directory.rglob("*agent_info.csv"))
    task, sources = None, []
    for path in traces:
        rows = [r for r in _rows(path) if kernel_name in r.get("Kernel_Name", "")
                and r.get("Start_Timestamp") and r.get("End_Timestamp")]
        if not rows:
            continue
        rows.sort(key=lambda r: int(r["Start_Timestamp"]))
        runs = _group_runs(rows, kernels_per_run)
        task = _median([x for x in runs if x and x > 0])
        sources.append(str(path.relative_to(directory)))
        break
    if task is None:
        for path in stats:
            rows = [r for r in _rows(path) if kernel_name in r.get("Name", "")]
            if rows and all("AverageNs" in r for r in rows):
                task = sum(float(r["AverageNs"]) for r in rows) / 1000.0
                sources.append(str(path.relative_to(directory)))
                break
    simds = xcds = None
    for path in agents:
        for r in _rows(path):
            if r.get("Agent_Type", "").upper() != "GPU":
                continue
            try:
                simds = int(r["Simd_Count"]) or int(r["Cu_Count"]) * int(r["Simd_Per_Cu"])
                xcds = int(r["Num_Xcc"]) or 1
            except (KeyError, ValueError):
                simds = xcds = None
            break
    raw, busy = {}, {}
    for path in counters:
        per = {}
        for r in _rows(path):
            if kernel_name not in r.get("Kernel_Name", ""):
                continue
            try:
                key = (int(r["Dispatch_Id"]), r["Kernel_Name"].split("(")[0])
                per.setdefault(key, {})
                name = r["Counter_Name"]
                per[key][name] = per[key].get(name, 0.0) + float(r["Counter_Value"])
            except (KeyError, ValueError):
                continue
        for (_dispatch, kernel), values in per.items():
            for name, value in values.items():
                raw.setdefault(f"{kernel}:{name}", []).append(value)
            if ("SQ_VALU_MFMA_BUSY_CYCLES" in values and values.get("GRBM_GUI_ACTIVE")
                    and simds and xcds):
                busy.setdefault(kernel, []).append(
                    values["SQ_VALU_MFMA_BUSY_CYCLES"] / simds / (values["GRBM_GUI_ACTIVE"] / xcds))
        if per:
            sources.append(str(path.relative_to(directory)))
    return {"task_duration_us": task,
            "pipeline_utilization": {f"mfma_busy:{k}": _median(v) for k, v in busy.items()} or None,
            "counters": {k: _median(v) for k, v in raw.items()} or None,
            "summary_sources": sorted(set(sources)),
            "summary_note": "Medians over FFN dispatches; no metric is inferred beyond the stated ratio"}


def extract_task_duration(trace_path, kernel_name=FFN_KERNEL):
    """Summed device duration of the FFN kernels in a one-run Chrome trace (microseconds),
    from device kernel events only, never host API time (performance/collect.py:110-122)."""
    data = json.loads(Path(trace_path).read_text())
    events = [e for e in data.get("traceEvents", []) if e.get("ph") == "X"
              and e.get("cat", "").lower() in ("kernel", "gpu_op")
              and kernel_name in e.get("name", "") and isinstance(e.get("dur"), (int, float))]
    if not events:
        return {"task_duration_us": None, "task_duration_note": "No matching device kernel trace event"}
    return {"task_duration_us": float(sum(e["dur"] for e in events)),
            "profiled_kernels": [{"name": e["name"].split("(")[0], "dur_us": e["dur"]} for e in events],
            "task_duration_note": "Sum of the FFN's device kernel durations in one traced run"}
