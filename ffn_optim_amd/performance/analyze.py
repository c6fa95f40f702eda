"""Evidence-limited report of a harness run (restates performance/analyze.py): measured
numbers only, no inferred pipeline utilisation or stage split."""
from __future__ import annotations


def _fmt(value):
    if value is None:
        return "unavailable"
    if isinstance(value, float):
        return f"{value:.3f}"
    return str(value)


def report(records, best):
    """Markdown table of every evaluated candidate plus the per-case best."""
    lines = ["# Performance analysis", "",
             "Ranking: unprofiled device-event median (µs); profiler task duration listed apart.", "",
             "| case | down | up/down variant | status | event median µs | task duration µs | mean_rel |",
             "| --- | --- | --- | --- | --- | --- | --- |"]
    for row in records:
        cfg = row["configuration"]
        variants = (f"{cfg['up_variant']}/{cfg['down_variant']}" if "up_variant" in cfg
                    else "planner")
        acc = (row.get("accuracy") or {}).get("mean_rel")
        lines.append("| " + " | ".join(_fmt(v) for v in (
            row["case_id"], cfg.get("down_impl"), variants, row["status"],
            row.get("device_median_us"), row.get("task_duration_us"), acc)) + " |")
    lines += ["", "## Best per case", ""]
    for case_id, b in best.items():
        lines.append(f"- {case_id}: {b.get('configuration')} "
                     f"({_fmt(b.get('device_median_us'))} µs, complete={b.get('complete')})")
    lines += ["", "## Scope", "",
              "- A best configuration holds only for this case, input, device, library revision and search space.",
              "- Pipeline utilisation comes only from collected counters (rocprofv3 --pmc); "
              "it is reported as unavailable otherwise, never estimated from totals.",
              "- The FFN is two kernels (up, down); a step time is not split into "
              "up, GELU and down from event timing alone.", ""]
    return "\n".join(lines)
