"""Case schema and deterministic inputs (restates common/cases.py).

A case is a JSON object {case_id, shape, weight1_shape, weight2_shape, dtype,
layout, seed, noncontiguous?, x_view?, memory_bound?}; files carry schema_version 1
(common/cases.py:7-25).  make_inputs draws the same seeded tensors as
common/cases.py:34-50; x_view='transpose12' additionally gives X the strides of
a dim-1/dim-2 transposed buffer with unchanged values (the unaligned 4-D case).
memory_bound marks a workload judged on HBM bandwidth, which is also timed with the caches
flushed between steps.
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


def load_cases(path):
    """Read and validate a case file (common/cases.py:7-25)."""
    data = json.loads(Path(path).read_text())
    if not isinstance(data, dict) or data.get("schema_version") != 1:
        raise ValueError("Expected case schema_version=1")
    cases = data.get("cases")
    if not isinstance(cases, list) or not cases:
        raise ValueError("cases must be a non-empty list")
    seen = set()
    for case in cases:
        name = case.get("case_id")
        if not isinstance(name, str) or not name or name in seen:
            raise ValueError("case_id must be a unique non-empty string")
        seen.add(name)
        case_problem(case)
        if type(case.get("seed", 0)) is not int:
            raise ValueError("seed must be an integer")
        if type(case.get("noncontiguous", False)) is not bool:
            raise ValueError("noncontiguous must be boolean")
        if case.get("x_view") not in X_VIEWS:
            raise ValueError(f"x_view must be one of {X_VIEWS}")
        if type(case.get("memory_bound", False)) is not bool:
            raise ValueError("memory_bound must be boolean")
    return cases


def case_problem(case):
    return problem_from_shapes(case["shape"], case["weight1_shape"], case["weight2_shape"],
                               case["dtype"], case.get("layout", "linear"))


def get_case(case_id, path=None):
    for path in ([path] if path else [BENCH_CASES, V1_CASES, SHARD_CASES]):
        for case in load_cases(path):
            if case["case_id"] == case_id:
                return case
    raise KeyError(case_id)


def make_inputs(case, device="cpu"):
    """Seeded inputs: one CPU generator, randn in the order x, w1, w2 (common/cases.py:34-50)."""
    import torch
    p = case_problem(case)
    generator = torch.Generator(device="cpu").manual_seed(case.get("seed", 0))
    dtype = getattr(torch, p.dtype)

    def sample(shape, scale=1.0):
        return (torch.randn(shape, generator=generator) * scale).to(dtype).to(device)

    x = sample(p.input_shape)
    w1 = sample((p.h, p.k), p.k ** -0.5)
    w2 = sample((p.n, p.h), p.h ** -0.5)
    if case.get("noncontiguous", False):
        def strided(t):
            buf = torch.empty((*t.shape[:-1], t.shape[-1] * 2), dtype=t.dtype, device=t.device)
            buf[..., ::2].copy_(t)
            return buf[..., ::2]
        x, w1, w2 = map(strided, (x, w1, w2))
    if case.get("x_view") == "transpose12":
        x = x.transpose(1, 2).contiguous().transpose(1, 2)
    return x, w1, w2
