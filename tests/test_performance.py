"""Measurement/search harness: search ranking, checkpoints, profiler summaries, the CPU-only
default CLI and the tuning table (restates the SearchTests/ReportTests of
validation/test_ffn.py:186-330 for the gfx950 harness)."""
import ast
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_best_and_failure_filter():
    from ffn_optim_amd.performance.tune import search
    configs = [{"down_impl": k} for k in ("basic", "streamk", "full_load_a")]

    def evaluate(config):
        k = config["down_impl"]
        return {"status": "passed" if k != "full_load_a" else "unavailable",
                "device_median_us": {"basic": 8, "streamk": 4, "full_load_a": None}[k]}

    records, best = search(configs, evaluate)
    assert best["complete"]
    assert best["configuration"]["down_impl"] == "streamk"
    assert len(records) == 3


def test_dry_run_no_best():
    from ffn_optim_amd.performance.tune import search
    _, best = search([{}], lambda c: {"status": "planned"})
    assert best["configuration"] is None


def test_accuracy_failure_never_wins():
    from ffn_optim_amd.performance.tune import search

    def evaluate(c):
        return {"status": "accuracy_failed" if c["down_impl"] == "streamk" else "passed",
                "device_median_us": 1 if c["down_impl"] == "streamk" else 10}

    _, best = search([{"down_impl": "streamk"}, {"down_impl": "basic"}], evaluate)
    assert best["configuration"]["down_impl"] == "basic"


def test_non_finite_timing_never_wins():
    from ffn_optim_amd.performance.tune import search
    values = {"a": float("nan"), "b": 0.0, "c": 5.0}
    _, best = search([{"id": k} for k in values],
                     lambda c: {"status": "passed", "device_median_us": values[c["id"]]})
    assert best["configuration"] == {"id": "c"}


def test_refinement_finalists_and_ranking():
    """Tune mode re-times the distinct near-equal finalists side by side and keeps the
    fastest by that re-timing; without one, the one-run median decides."""
    from ffn_optim_amd.performance.tune import pick_fastest, refine_candidates

    def rec(up, down, us, status="passed", **extra):
        return dict({"status": status, "device_median_us": us,
                     "configuration": {"up_variant": up, "down_variant": down}}, **extra)

    rows = [rec(12, 10, 100.0), rec(12, 13, 101.0), rec(12, 10, 100.5), rec(0, 10, 104.9),
            rec(12, 11, 105.1), rec(12, 1, 99.0, status="accuracy_failed"), rec(12, 3, 130.0)]
    finalists = refine_candidates(rows)
    assert [(r["configuration"]["up_variant"], r["configuration"]["down_variant"]) for r in finalists] \
        == [(12, 10), (12, 13), (0, 10)]
    assert len(refine_candidates(rows, limit=2)) == 2
    assert pick_fastest(rows)["device_median_us"] == 100.0
    finalists[1]["refined_median_us"] = 95.0
    finalists[0]["refined_median_us"] = 97.0
    assert pick_fastest(rows)["configuration"]["down_variant"] == 13
    assert pick_fastest([rec(0, 0, 1.0, status="accuracy_failed")]) is None


def test_checkpoint_before_interruption():
    from ffn_optim_amd.performance.tune import search
    checkpoints = []

    def evaluate(c):
        if c["id"] == 2:
            raise KeyboardInterrupt()
        return {"status": "passed", "device_median_us": 10}

    with pytest.raises(KeyboardInterrupt):
        search([{"id": 1}, {"id": 2}], evaluate,
               lambda rows, best: checkpoints.append((list(rows), dict(best))))
    assert len(checkpoints[0][0]) == 1
    assert not checkpoints[0][1]["complete"]


def test_combinations_deduplicate_and_reject_empty():
    from ffn_optim_amd.performance.tune import combinations
    assert combinations(["basic", "basic"], ["basic", "streamk"]) == [
        {"up_impl": "basic", "down_impl": "basic"}, {"up_impl": "basic", "down_impl": "streamk"}]
    with pytest.raises(ValueError):
        combinations([], ["basic"])


def _write(path, text):
    path.parent.mkdir(parents=True, exist_ok=True)
    path.write_text(text)


def test_summary_reads_rocprof_outputs(tmp_path):
    from ffn_optim_amd.performance.collect import extract_summary
    # two FFN runs of two kernels each, plus an unrelated kernel that must be ignored
    _write(tmp_path / "kt" / "x_kernel_trace.csv",
           '"Kind","Dispatch_Id","Kernel_Name","Start_Timestamp","End_Timestamp"\n'
           '"K",1,"void ffn::ffn_gemm_kernel<1, A, 0, false>(ffn::GemmParams)",1000,11000\n'
           '"K",2,"void ffn::ffn_gemm_kernel<1, B, 2, false>(ffn::GemmParams)",12000,20000\n'
           '"K",3,"void other_kernel(int)",20000,900000\n'
           '"K",4,"void ffn::ffn_gemm_kernel<1, A, 0, false>(ffn::GemmParams)",30000,42000\n'
           '"K",5,"void ffn::ffn_gemm_kernel<1, B, 2, false>(ffn::GemmParams)",43000,53000\n')
    _write(tmp_path / "pmc" / "p_agent_info.csv",
           '"Agent_Type","Simd_Count","Num_Xcc","Cu_Count","Simd_Per_Cu"\n'
           '"CPU",0,1,16,0\n"GPU",1024,8,256,4\n')
    _write(tmp_path / "pmc" / "p_counter_collection.csv",
           '"Dispatch_Id","Kernel_Name","Counter_Name","Counter_Value"\n'
           '7,"void ffn::ffn_gemm_kernel<1, A, 0, false>(ffn::GemmParams)","SQ_VALU_MFMA_BUSY_CYCLES",300000\n'
           '7,"void ffn::ffn_gemm_kernel<1, A, 0, false>(ffn::GemmParams)","SQ_VALU_MFMA_BUSY_CYCLES",212000\n'
           '7,"void ffn::ffn_gemm_kernel<1, A, 0, false>(ffn::GemmParams)","GRBM_GUI_ACTIVE",8000\n'
           '8,"void other_kernel(int)","GRBM_GUI_ACTIVE",5\n')
    m = extract_summary(tmp_path)
    assert m["task_duration_us"] == pytest.approx((18.0 + 22.0) / 2)
    (key, busy), = m["pipeline_utilization"].items()
    assert "ffn_gemm_kernel<1, A, 0, false>" in key
    assert busy == pytest.approx(512000 / 1024 / (8000 / 8))
    assert not any("other_kernel" in k for k in m["counters"])


def test_summary_groups_runs_by_launch_count(tmp_path):
    """The up and down GEMMs can be the same kernel instantiation (a split up GEMM and a
    Stream-K down on one tile variant, both fast-DMA).  Grouping by name recurrence would count
    every FFN as two runs; grouping by the plan's launch count does not."""
    from ffn_optim_amd.performance.collect import extract_summary
    gemm = "void ffn::ffn_gemm_kernel<1, V8, 2, true, true>(ffn::GemmParams)"
    lines, t = [], 0
    for run in range(3):
        for name, dur in ((gemm, 14), (gemm, 12)):
            lines.append(f'"K",{len(lines) + 1},"{name}",{t},{t + dur * 1000}')
            t += dur * 1000 + 500
    _write(tmp_path / "kt" / "x_kernel_trace.csv",
           '"Kind","Dispatch_Id","Kernel_Name","Start_Timestamp","End_Timestamp"\n' + "\n".join(lines) + "\n")
    assert extract_summary(tmp_path, kernels_per_run=2)["task_duration_us"] == pytest.approx(26.0)
    assert extract_summary(tmp_path)["task_duration_us"] == pytest.approx(13.0)  # the miscount: halves of FFNs


def test_kernels_per_run_is_two_launches():
    """Split tiles (a split up GEMM, a Stream-K down) are finished inside their GEMM's launch."""
    from types import SimpleNamespace as NS
    from ffn_optim_amd.performance.collect import kernels_per_run
    assert kernels_per_run(NS(native=NS(up_sk_tiles=0, down_sk_tiles=0))) == 2
    assert kernels_per_run(NS(native=NS(up_sk_tiles=27, down_sk_tiles=80))) == 2


def test_summary_falls_back_to_kernel_stats(tmp_path):
    from ffn_optim_amd.performance.collect import extract_summary
    _write(tmp_path / "kt_kernel_stats.csv",
           '"Name","Calls","AverageNs"\n"void ffn::ffn_gemm_kernel<1, A, 0, false>(p)",3,40000\n'
           '"void ffn::ffn_gemm_kernel<1, A, 2, true>(p)",3,5000\n"void other(int)",1,99999999\n')
    assert extract_summary(tmp_path)["task_duration_us"] == pytest.approx(45.0)


def test_unknown_profiler_schema(tmp_path):
    from ffn_optim_amd.performance.collect import extract_summary
    _write(tmp_path / "op_summary_0.csv", "Op Name,Task Duration(us)\nffn,10\n")
    m = extract_summary(tmp_path)
    assert m["pipeline_utilization"] is None and m["task_duration_us"] is None


def test_task_duration_from_chrome_trace(tmp_path):
    from ffn_optim_amd.performance.collect import extract_task_duration
    trace = {"traceEvents": [
        {"ph": "X", "cat": "kernel", "name": "void ffn::ffn_gemm_kernel<1, A, 0, false>(p)", "dur": 30.5},
        {"ph": "X", "cat": "kernel", "name": "void ffn::ffn_gemm_kernel<1, B, 2, false>(p)", "dur": 20.0},
        {"ph": "X", "cat": "cuda_runtime", "name": "hipLaunchKernel ffn_gemm", "dur": 900.0},
        {"ph": "X", "cat": "kernel", "name": "void other(int)", "dur": 7.0}]}
    (tmp_path / "trace.json").write_text(json.dumps(trace))
    r = extract_task_duration(tmp_path / "trace.json")
    assert r["task_duration_us"] == pytest.approx(50.5)
    empty = tmp_path / "empty.json"
    empty.write_text(json.dumps({"traceEvents": []}))
    assert extract_task_duration(empty)["task_duration_us"] is None


def test_default_cli_is_cpu_only(tmp_path):
    script = """
import sys
import torch
from ffn_optim_amd.performance.run import main
assert main(['--mode', 'search', '--output-root', sys.argv[1]]) == 0
assert not torch.cuda.is_initialized()
"""
    result = subprocess.run([sys.executable, "-c", script, str(tmp_path)], cwd=ROOT,
                            capture_output=True, text=True, timeout=300)
    assert result.returncode == 0, result.stderr
    for message in ("case 1/3", "case 2/3", "case 3/3", "config 1/4",
                    "dry run: skipping the CPU golden", "all cases done"):
        assert message in result.stdout
    assert "computing the CPU FP32 golden" not in result.stdout
    run = next(tmp_path.iterdir())
    rows = json.loads((run / "accuracy.json").read_text())
    assert len(rows) == 12
    assert {r["status"] for r in rows} == {"planned", "unavailable"}
    assert not json.loads((run / "manifest.json").read_text())["device_executed"]
    best = json.loads((run / "best_configs.json").read_text())
    assert all(value["configuration"] is None for value in best.values())
    for name in ("performance.csv", "analysis.md"):
        assert (run / name).exists()


def test_runner_saves_case_preparation_interruption(tmp_path, capsys):
    from unittest.mock import patch
    from ffn_optim_amd.performance.run import PerformanceRunner, parser
    runner = PerformanceRunner(parser().parse_args(["--output-root", str(tmp_path)]))
    with patch.object(runner, "prepare_case", side_effect=KeyboardInterrupt()):
        with pytest.raises(KeyboardInterrupt):
            runner.run()
    info = json.loads((runner.root / "manifest.json").read_text())
    bests = json.loads((runner.root / "best_configs.json").read_text())
    assert not info["complete"] and not info["device_executed"]
    assert not bests[runner.cases[0]["case_id"]]["complete"]
    assert "run interrupted or failed" in capsys.readouterr().out
    with pytest.raises(RuntimeError):
        runner.run()


def test_bench_refuses_more_than_one_gpu():
    """bench.py --gpus N with N > 1 exits with a message before touching a device."""
    for n in ("2", "8"):
        proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", n],
                              capture_output=True, text=True, timeout=120, cwd=ROOT)
        assert proc.returncode != 0 and not proc.stdout.strip()
        assert "one GPU" in proc.stdout + proc.stderr


def test_runner_arguments_rejected():
    from ffn_optim_amd.performance.run import PerformanceRunner, parser
    for argv in (["--execute-gpu", "--dry-run"], ["--repeats", "0"], ["--write-tuned"],
                 ["--mode", "tune", "--write-tuned"]):
        with pytest.raises(ValueError):
            PerformanceRunner(parser().parse_args(argv))


def test_runner_methods_documented_and_flat():
    tree = ast.parse((ROOT / "ffn_optim_amd/performance/run.py").read_text())
    runner = next(n for n in tree.body if isinstance(n, ast.ClassDef) and n.name == "PerformanceRunner")
    doc = ast.get_docstring(runner)
    assert all(word in doc for word in ("Purpose", "Inputs", "Outputs"))
    for node in ast.walk(tree):
        if isinstance(node, ast.FunctionDef):
            assert not any(isinstance(child, (ast.FunctionDef, ast.AsyncFunctionDef))
                           for stmt in node.body for child in ast.walk(stmt)), node.name
    for method in runner.body:
        if isinstance(method, ast.FunctionDef):
            assert ast.get_docstring(method), method.name


def test_tune_space_covers_every_applicable_variant():
    from ffn_optim_amd import _lib
    from ffn_optim_amd.cases import case_problem, get_case
    from ffn_optim_amd.performance.tune import tile_space_down, tile_space_up
    nvar = _lib.load().ffn_mi355x_num_variants()
    p = case_problem(get_case("c2_aligned_bf16"))
    up = tile_space_up(p, "basic", 256)
    assert [c["up_variant"] for c in up] == list(range(nvar))
    assert len({c["down_variant"] for c in up}) == 1
    down = tile_space_down(p, ["basic", "streamk"], 0, 256)
    basic = [c for c in down if c["down_impl"] == "basic"]
    sk = [c for c in down if c["down_impl"] == "streamk"]
    assert len(basic) == nvar and 0 < len(sk) < nvar   # tile counts divisible by 256 have no SK
    assert all(c["up_variant"] == 0 for c in down)


def test_tuning_table_roundtrip_and_planner_use(tmp_path, monkeypatch):
    from ffn_optim_amd import tuning
    from ffn_optim_amd.host.dispatch import Selection
    from ffn_optim_amd.host.inputs import problem_from_shapes
    from ffn_optim_amd.host.tiling import make_plan
    table = tmp_path / "tuned.json"
    monkeypatch.setattr(tuning, "TABLE_PATH", table)
    p = problem_from_shapes([4096, 1024], [4096, 1024], [1024, 4096], "bfloat16")
    base = make_plan(p, Selection(), 256)
    key = tuning.make_key(p.m, base.mp, base.kp, base.hp, base.np, p.dtype, "basic", "erf", 256)
    assert tuning.lookup(key) is None
    up, down = (base.up.variant + 1) % 10, (base.down.variant + 2) % 10
    tuning.record(key, up, down, device_median_us=12.5, source="test")
    assert tuning.lookup(key) == (up, down)
    plan = make_plan(p, Selection(), 256)
    assert (plan.up.variant, plan.down.variant) == (up, down)
    assert make_plan(p, Selection(), 256, tuned=False).up.variant == base.up.variant
    forced = make_plan(p, Selection(), 256, up_variant=base.up.variant)
    assert forced.up.variant == base.up.variant          # a forced variant bypasses the table
    other = make_plan(p, Selection(), 128)               # another block_num is another key
    assert other.up.variant == make_plan(p, Selection(), 128, tuned=False).up.variant
    data = json.loads(table.read_text())
    assert data["schema_version"] == 1 and len(data["entries"]) == 1


def test_committed_tuning_table_plans_every_entry():
    """Every entry of the committed table names variants the library still accepts for its key,
    and the measured workloads find their entry (the planner then uses those variants)."""
    from ffn_optim_amd import _lib, tuning
    from ffn_optim_amd.cases import BENCH_CASES, SHARD_CASES, case_problem, load_cases
    from ffn_optim_amd.host.dispatch import Selection
    from ffn_optim_amd.host.tiling import make_plan
    entries = json.loads(tuning.TABLE_PATH.read_text())["entries"]
    assert entries
    for e in entries:
        k = e["key"]
        dtype = _lib.BF16 if k["dtype"] == "bfloat16" else _lib.FP16
        plan = _lib.make_plan(k["mp"], k["kp"], k["hp"], k["np"], dtype, k["down_impl"], k["gelu"],
                              k["block_num"], e["up_variant"], e["down_variant"], m=k["m"])
        assert (plan.up_variant, plan.down_variant) == (e["up_variant"], e["down_variant"])
    for path in (BENCH_CASES, SHARD_CASES):
        for case in load_cases(path):
            for down in ("basic", "streamk"):
                plan = make_plan(case_problem(case), Selection(down_impl=down), 256)
                key = tuning.make_key(plan.problem.m, plan.mp, plan.kp, plan.hp, plan.np,
                                      plan.problem.dtype, down, "erf", 256)
                assert tuning.lookup(key) == (plan.up.variant, plan.down.variant), (case["case_id"], down)


def test_tuning_table_rejects_bad_entries(tmp_path):
    from ffn_optim_amd import tuning
    bad = tmp_path / "bad.json"
    bad.write_text(json.dumps({"schema_version": 1, "entries": [
        {"key": {f: 1 for f in tuning.KEY_FIELDS}, "up_variant": -1, "down_variant": 0}]}))
    with pytest.raises(ValueError):
        tuning.load(bad)
    bad.write_text(json.dumps({"schema_version": 2, "entries": []}))
    with pytest.raises(ValueError):
        tuning.load(bad)


@pytest.mark.parametrize("gelu", ["erf", "rational"])
@pytest.mark.parametrize("staged", [False, True])
def test_harness_golden_matches_oracle(gelu, staged):
    """The harness's golden (plain and staged, erf and rational GELU) is the oracle's, bit for
    bit: the same torch CPU FP32 operations in the same order."""
    import torch
    from ffn_optim_amd.performance.accuracy import compare, golden
    from oracle.reference import compare as oracle_compare, ffn_torch
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 7, 40, generator=g).half()
    w1 = (torch.randn(72, 40, generator=g) * 40 ** -0.5).half()
    w2 = (torch.randn(24, 72, generator=g) * 72 ** -0.5).half()
    ours = golden(x, w1, w2, gelu=gelu, staged=staged)
    ref = ffn_torch(x, w1, w2, rational=(gelu == "rational"), staged=staged)
    assert ours.shape == ref.shape and ours.dtype == ref.dtype
    assert torch.equal(ours, ref)
    if staged:
        assert not torch.equal(ours, golden(x, w1, w2, gelu=gelu))
    noisy = (ref.float() * 1.2).to(ref.dtype)
    for a, b in ((ours, ref), (noisy, ref), (ref.float(), ref), (ref * float("nan"), ref)):
        ra, rb = compare(a, b), oracle_compare(a, b)
        assert ra["passed"] == rb["passed"]
