"""Serial exhaustive search over an explicit candidate list (restates performance/tune.py).

combinations() builds the reference's implementation Cartesian product;
tile_space_up()/tile_space_down() add the MI355X-specific dimension, the tile variants
the library accepts for a problem, searched one GEMM at a time.  search() evaluates candidates in order, checkpoints after each
one and ranks only candidates whose status is 'passed' with a finite positive
unprofiled device-event median.  refine_candidates() picks the near-equal finalists that tune
mode re-times side by side, and pick_fastest() ranks by that re-timing where it exists.
"""
from __future__ import annotations

import itertools
import math


def combinations(up, down):
    """[{'up_impl': u, 'down_impl': d}] over the de-duplicated product (performance/tune.py:6-9)."""
    if not up or not down:
        raise ValueError("Search spaces must be non-empty")
    return [{"up_impl": u, "down_impl": d}
            for u, d in itertools.product(dict.fromkeys(up), dict.fromkeys(down))]


def _applicable(problem, down, block_num, gelu, up_variant, down_variant):
    from ..host.dispatch import Selection
    from ..host.tiling import make_plan
    try:
        return make_plan(problem, Selection("basic", down), block_num, gelu=gelu,
                         up_variant=up_variant, down_variant=down_variant, tuned=False)
    except ValueError:
        return None


def tile_space_up(problem, down, block_num, gelu="erf"):
    """Tune phase 1: every up tile variant, with the planner's down variant for `down`.

    The up and down GEMMs are separate launches whose times add, so the up variant
    is searched with the down fixed and the down variant afterwards (tile_space_down).
    """
    from .. import _lib
    base = _applicable(problem, down, block_num, gelu, None, None)
    if base is None:
        raise ValueError(f"{down} is not applicable to this problem")
    dv = base.down.variant
    out = [{"up_impl": "basic", "down_impl": down, "up_variant": uv, "down_variant": dv}
           for uv in range(_lib.load().ffn_mi355x_num_variants())
           if _applicable(problem, down, block_num, gelu, uv, dv) is not None]
    if not out:
        raise ValueError("no applicable up tile variant for this problem")
    return out


def tile_space_down(problem, downs, up_variant, block_num, gelu="erf"):
    """Tune phase 2: every down tile variant of each implementation in downs the library
    accepts (Stream-K without remainder tiles and the like are left out), with the up
    variant fixed."""
    from .. import _lib
    nvar = _lib.load().ffn_mi355x_num_variants()
    return [{"up_impl": "basic", "down_impl": d, "up_variant": up_variant, "down_variant": dv}
            for d in dict.fromkeys(downs) for dv in range(nvar)
            if _applicable(problem, d, block_num, gelu, up_variant, dv) is not None]


def refine_candidates(rows, within=0.05, limit=4):
    """The passed records of one down implementation worth re-timing side by side: distinct
    (up, down) variant pairs whose one-run median is within `within` of the fastest, at most
    `limit`, fastest first."""
    seen, out = set(), []
    passed = sorted((r for r in rows if r.get("status") == "passed"), key=lambda r: r["device_median_us"])
    for r in passed:
        pair = (r["configuration"].get("up_variant"), r["configuration"].get("down_variant"))
        if pair in seen or r["device_median_us"] > passed[0]["device_median_us"] * (1 + within):
            continue
        seen.add(pair)
        out.append(r)
    return out[:limit]


def pick_fastest(rows):
    """The record to keep among one down implementation's passed records: by the interleaved
    re-timing (refined_median_us) where any record has one, else by the one-run median."""
    passed = [r for r in rows if r.get("status") == "passed"]
    if not passed:
        return None
    refined = [r for r in passed if isinstance(r.get("refined_median_us"), (int, float))]
    if refined:
        return min(refined, key=lambda r: r["refined_median_us"])
    return min(passed, key=lambda r: r["device_median_us"])


def search(configurations, evaluate, checkpoint=None):
    """Evaluate every configuration; returns (records, best) (performance/tune.py:12-31).

    best['configuration'] stays None unless some candidate passed with a finite,
    positive device_median_us; checkpoint(records, best) runs after every candidate
    and once more with best['complete'] set.
    """
    records = []
    best = {"configuration": None, "device_median_us": None, "complete": False,
            "ranking_metric": "unprofiled_device_event_median_us", "scope": configurations}
    for index, configuration in enumerate(configurations, start=1):
        print(f"[search] evaluating configuration {index}/{len(configurations)}: {configuration}",
              flush=True)
        row = dict(evaluate(configuration), configuration=configuration)
        records.append(row)
        value = row.get("device_median_us")
        if (row["status"] == "passed" and isinstance(value, (int, float))
                and math.isfinite(value) and value > 0
                and (best["device_median_us"] is None or value < best["device_median_us"])):
            best.update(configuration=configuration, device_median_us=value)
        if checkpoint:
            checkpoint(records, best)
    best["complete"] = True
    if checkpoint:
        checkpoint(records, best)
    return records, best
