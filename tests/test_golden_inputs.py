"""ffn_optim_amd.cases.make_inputs against the reference's own draws.

tests/golden/input_vectors.json was written by tests/golden/make_input_vectors.py,
which ran the reference's make_inputs (common/cases.py:34-50) on the reference's
smoke cases and on the five benchmark workloads.  Every tensor must match it in
shape, strides, dtype and the sha256 of its values, so "identical seeded inputs"
holds draw for draw.  Runs on the CPU (the full-size workloads draw ~250M values,
a few seconds).
"""
import hashlib
import json
from pathlib import Path

import pytest
import torch

from ffn_optim_amd.cases import load_cases, make_inputs, BENCH_CASES

FIXTURE = Path(__file__).resolve().parent / "golden" / "input_vectors.json"
ENTRIES = json.loads(FIXTURE.read_text())["entries"]


def _digest(t):
    return hashlib.sha256(t.contiguous().reshape(-1).view(torch.int16).numpy().tobytes()).hexdigest()


@pytest.mark.parametrize("entry", ENTRIES, ids=lambda e: e["case"]["case_id"])
def test_draws_match_the_reference(entry):
    tensors = dict(zip(("x", "weight1", "weight2"), make_inputs(entry["case"], "cpu")))
    for name, t in tensors.items():
        want = entry[name]
        assert list(t.shape) == want["shape"], name
        assert list(t.stride()) == want["stride"], name
        assert str(t.dtype).removeprefix("torch.") == want["dtype"], name
        flat = t.contiguous().reshape(-1)
        assert [float(v) for v in flat[:8]] == want["head"], name
        assert [float(v) for v in flat[-8:]] == want["tail"], name
        assert _digest(t) == want["sha256"], name


def test_fixture_covers_every_benchmark_workload():
    """The fixture was made from the committed workload file: same ids, shapes and seeds."""
    by_id = {e["case"]["case_id"]: e["case"] for e in ENTRIES}
    for case in load_cases(BENCH_CASES):
        ref = by_id[case["case_id"]]
        for key in ("shape", "weight1_shape", "weight2_shape", "dtype", "seed"):
            assert ref[key] == case[key], (case["case_id"], key)


def test_transposed_view_keeps_the_reference_values():
    """x_view only restrides X: its values are the reference's draws (C3's transposed view)."""
    case = next(c for c in load_cases(BENCH_CASES) if c.get("x_view") == "transpose12")
    entry = next(e for e in ENTRIES if e["case"]["case_id"] == case["case_id"])
    x, _, _ = make_inputs(case, "cpu")
    assert not x.is_contiguous()
    d0, d1, d2, d3 = x.shape
    assert x.stride() == (d1 * d2 * d3, d3, d1 * d3, 1)
    assert _digest(x) == entry["x"]["sha256"]
