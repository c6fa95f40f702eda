"""Candidate spaces and ranking of the measurement harness (the counterpart of performance/tune.py).

A harness run evaluates candidates one at a time; each evaluation returns a record whose
``status`` says how far it got (planned, unavailable, not_applicable, compile_failed,
accuracy_failed, passed, ...).  Only a ``passed`` record with a finite, positive unprofiled
device-event median (``device_median_us``) can become a case's best: the ``Leaderboard`` below
keeps that rule in one place.

Candidate spaces:
* ``combinations`` -- the implementation product the reference searches (up x down impls);
* ``tile_space_up`` / ``tile_space_down`` -- the MI355X dimension, the compiled tile variants the
  library accepts for a problem, searched one GEMM at a time (the two launches' times add).

``search`` sweeps a candidate list with a checkpoint after every record; ``refine_candidates`` and
``pick_fastest`` serve tune mode's side-by-side re-timing of near-equal finalists.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

RANKING_METRIC = "unprofiled_device_event_median_us"


def rank_value(record):
    """The record's ranking time, or None when it may not rank (not passed, or a median that is
    missing, non-finite or not positive)."""
    value = record.get("device_median_us")
    if record.get("status") != "passed" or isinstance(value, bool) or not isinstance(value, (int, float)):
        return None
    return float(value) if math.isfinite(value) and value > 0 else None


@dataclass
class Leaderboard:
    """Running best of one sweep over `scope` (a candidate list)."""

    scope: list
    configuration: dict | None = None
    device_median_us: float | None = None
    complete: bool = False
    records: list = field(default_factory=list)

    def add(self, record):
        """Append an evaluated record; it takes the lead if it ranks and beats the current best."""
        self.records.append(record)
        value = rank_value(record)
        if value is not None and (self.device_median_us is None or value < self.device_median_us):
            self.configuration, self.device_median_us = record["configuration"], value

    def state(self):
        """The best_configs.json entry of this sweep (a fresh dict)."""
        return {"configuration": self.configuration, "device_median_us": self.device_median_us,
                "complete": self.complete, "ranking_metric": RANKING_METRIC, "scope": self.scope}


def _distinct(values):
    out = []
    for value in values:
        if value not in out:
            out.append(value)
    return out


def combinations(up, down):
    """The up x down implementation product as candidate dicts, duplicates dropped, order kept
    (performance/tune.py:6-9); ValueError when either side is empty."""
    ups, downs = _distinct(up), _distinct(down)
    if not ups or not downs:
        raise ValueError("Search spaces must be non-empty")
    return [{"up_impl": u, "down_impl": d} for u in ups for d in downs]


def search(configurations, evaluate, checkpoint=None, progress=print):
    """Evaluate `configurations` in order; returns (records, best) (performance/tune.py:12-31).

    Each record is evaluate(configuration) with the configuration attached.  checkpoint(records,
    best) runs after every record -- so an interruption leaves what was measured, with best
    marked incomplete -- and once more when the sweep is complete.
    """
    board = Leaderboard(list(configurations))
    total = len(board.scope)
    for position, configuration in enumerate(board.scope, start=1):
        if progress is not None:
            progress(f"[search {position}/{total}] {configuration}")
        board.add(dict(evaluate(configuration), configuration=configuration))
        if checkpoint is not None:
            checkpoint(list(board.records), board.state())
    board.complete = True
    if checkpoint is not None:
        checkpoint(list(board.records), board.state())
    return list(board.records), board.state()


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
            for d in _distinct(downs) for dv in range(nvar)
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
