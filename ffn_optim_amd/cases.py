"""Workload files and their seeded synthetic inputs (the role of common/cases.py).

A workload file is JSON: {"schema_version": 1, "cases": [case, ...]}, each case
{case_id, shape, weight1_shape, weight2_shape, dtype, layout, seed,
noncontiguous?, x_view?, memory_bound?} (schema of common/cases.py:7-25).

make_inputs draws from one CPU torch.Generator seeded with the case's seed, in
the order X (std 1), W1 (std K^-1/2), W2 (std H^-1/2), each FP32 randn scaled
and then cast -- the draw sequence of common/cases.py:34-50, which
tests/golden/input_vectors.json pins with the reference's own outputs.  Two
layout options change strides, never values: noncontiguous gives every operand
a stride of 2 along its last dim, x_view='transpose12' gives X the strides of a
buffer whose dims 1 and 2 are swapped (the unaligned 4-D workload).
memory_bound marks a workload judged on HBM bandwidth, also timed with the
caches flushed between steps.
"""
from __future__ import annotations

import json
from pathlib import Path

from .host.inputs import problem_from_shapes

CONFIGS = Path(__file__).resolve().parent / "configs"
BENCH_CASES = CONFIGS / "benchmark_cases.json"
V1_CASES = CONFIGS / "v1_cases.json"
SHARD_CASES = CONFIGS / "shard_cases.json"   # one GPU's share of an H split over 8 GPUs
X_VIEWS = (None, "transpose12")

# optional keys of a case: (required Python type, default)
_OPTIONAL = {"seed": (int, 0), "noncontiguous": (bool, False), "memory_bound": (bool, False)}


def _check_case(case, seen):
    cid = case.get("case_id")
    if not (isinstance(cid, str) and cid):
        raise ValueError("case_id must be a unique non-empty string")
    if cid in seen:
        raise ValueError(f"case_id {cid!r} must be unique (case_id must be a unique non-empty string)")
    case_problem(case)
    for key, (kind, default) in _OPTIONAL.items():
        if type(case.get(key, default)) is not kind:
            raise ValueError(f"{cid}: {key} must be {'an integer' if kind is int else 'boolean'}")
    if case.get("x_view") not in X_VIEWS:
        raise ValueError(f"{cid}: x_view must be one of {X_VIEWS}")


def load_cases(path):
    """Parse and validate a workload file; raises ValueError on any schema violation."""
    doc = json.loads(Path(path).read_text())
    if not (isinstance(doc, dict) and doc.get("schema_version") == 1):
        raise ValueError("Expected case schema_version=1")
    cases = doc.get("cases")
    if not (isinstance(cases, list) and cases):
        raise ValueError("cases must be a non-empty list")
    seen = set()
    for case in cases:
        _check_case(case, seen)
        seen.add(case["case_id"])
    return cases


def case_problem(case):
    return problem_from_shapes(case["shape"], case["weight1_shape"], case["weight2_shape"],
                               case["dtype"], case.get("layout", "linear"))


def get_case(case_id, path=None):
    for source in ([path] if path else [BENCH_CASES, V1_CASES, SHARD_CASES]):
        hit = next((c for c in load_cases(source) if c["case_id"] == case_id), None)
        if hit is not None:
            return hit
    raise KeyError(case_id)


def _every_other(t):
    """Same values with stride 2 along the last dim: interleave with zeros, keep the evens."""
    import torch
    return torch.stack((t, torch.zeros_like(t)), dim=-1).flatten(-2)[..., 0::2]


def make_inputs(case, device="cpu"):
    """(x, weight1, weight2) of a case on `device`, from the seeded CPU draws above."""
    import torch
    p = case_problem(case)
    rng = torch.Generator(device="cpu")
    rng.manual_seed(case.get("seed", 0))
    dtype = getattr(torch, p.dtype)
    draws = ((p.input_shape, 1.0), ((p.h, p.k), p.k ** -0.5), ((p.n, p.h), p.h ** -0.5))
    x, w1, w2 = [(torch.randn(shape, generator=rng) * std).to(dtype).to(device) for shape, std in draws]
    if case.get("noncontiguous", False):
        x, w1, w2 = _every_other(x), _every_other(w1), _every_other(w2)
    if case.get("x_view") == "transpose12":
        x = x.transpose(1, 2).contiguous().transpose(1, 2)
    return x, w1, w2
