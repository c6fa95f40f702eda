"""Writes tests/golden/input_vectors.json: the reference's own seeded draws.

Runs in the build container only (it reads /root/reference): imports the
reference's common/cases.py and calls its make_inputs (common/cases.py:34-50)
for the reference's smoke cases (configs/v1_cases.json) and for the five
benchmark workloads with the seeds this repository uses.  For every tensor it
records the shape, the strides, the dtype, the sha256 of its values in
row-major order, the float64 sum, and the first and last eight values.  The
fixture is data only; tests/test_golden_inputs.py checks
ffn_optim_amd.cases.make_inputs against it.

    python tests/golden/make_input_vectors.py
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

REFERENCE = Path("/root/reference")
HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
OUT = HERE / "input_vectors.json"

# keys of this repository's case schema that the reference's schema does not have;
# make_inputs of the reference ignores them, and they are stripped before the call
LOCAL_KEYS = ("x_view", "memory_bound")


def describe(t):
    import torch
    v = t.contiguous()
    flat = v.reshape(-1)
    raw = flat.view(torch.int16).numpy().tobytes()
    return {
        "shape": list(t.shape),
        "stride": list(t.stride()),
        "dtype": str(t.dtype).removeprefix("torch."),
        "sha256": hashlib.sha256(raw).hexdigest(),
        "sum_f64": float(flat.double().sum()),
        "head": [float(a) for a in flat[:8]],
        "tail": [float(a) for a in flat[-8:]],
    }


def main():
    sys.path.insert(0, str(REFERENCE))
    from common.cases import load_cases, make_inputs  # the reference's generator

    cases = [("reference:configs/v1_cases.json", c) for c in load_cases(REFERENCE / "configs/v1_cases.json")]
    bench = json.loads((REPO / "ffn_optim_amd/configs/benchmark_cases.json").read_text())["cases"]
    cases += [("ffn_optim_amd/configs/benchmark_cases.json", c) for c in bench]
    entries = []
    for source, case in cases:
        ref_case = {k: v for k, v in case.items() if k not in LOCAL_KEYS}
        x, w1, w2 = make_inputs(ref_case, "cpu")
        entries.append({"source": source, "case": ref_case,
                        "x": describe(x), "weight1": describe(w1), "weight2": describe(w2)})
        print(case["case_id"], entries[-1]["x"]["sha256"][:12], flush=True)
    import torch
    OUT.write_text(json.dumps({
        "generator": "reference common/cases.py:34-50 make_inputs, run on CPU",
        "torch": torch.__version__,
        "entries": entries,
    }, indent=1) + "\n")
    print(OUT)


if __name__ == "__main__":
    main()
