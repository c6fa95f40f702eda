"""Manual / search / tune entry of the FFN harness (restates performance/run.py).

The default is a CPU-only plan (dry run): cases are planned through the library,
nothing touches the GPU.  --execute-gpu authorises device preparation, validation
against the FP32 golden, event timing and (with --profile) a separate profiler pass.

    python -m ffn_optim_amd.performance.run --mode search --execute-gpu
    python -m ffn_optim_amd.performance.run --mode tune --execute-gpu --write-tuned \\
        --cases ffn_optim_amd/configs/benchmark_cases.json

Every run creates results/<run_id>/ with manifest.json, accuracy.json,
performance.csv, best_configs.json, analysis.md and profiler/; earlier runs are
never overwritten.  Modes: manual (one --up-impl/--down-impl), search (the
--up-candidates x --down-candidates product), tune (a coordinate search over the
compiled tile variants: every up variant with the planner's down, then every down
variant of each Basic/Stream-K candidate with the fastest up; --write-tuned records
the fastest pair per down implementation in the tuning table prepare_ffn consults).
"""
from __future__ import annotations

import argparse
import csv
import json
import platform
from datetime import datetime, timezone
from pathlib import Path
from time import perf_counter
from uuid import uuid4

from .. import _lib
from ..cases import V1_CASES, case_problem, load_cases, make_inputs
from ..host.dispatch import DependencyUnavailable, NotApplicable, Selection
from ..host.tiling import DEFAULT_BLOCK_NUM, make_plan
from .analyze import report
from .tune import (combinations, pick_fastest, refine_candidates, search, tile_space_down,
                   tile_space_up)

REPO_ROOT = Path(__file__).resolve().parents[2]


def parser():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--cases", default=str(V1_CASES))
    p.add_argument("--case-id", action="append", help="only the selected case IDs (repeatable)")
    p.add_argument("--mode", choices=("manual", "search", "tune"), default="manual")
    p.add_argument("--up-impl", default="basic")
    p.add_argument("--down-impl", default="basic")
    p.add_argument("--up-candidates", nargs="+", default=["basic"])
    p.add_argument("--down-candidates", nargs="+",
                   default=["basic", "full_load_a", "full_load_b", "streamk"])
    p.add_argument("--block-num", type=int, default=None,
                   help="persistent workgroups (default: every CU of the device; 256 in a dry run)")
    p.add_argument("--gelu", choices=("erf", "rational"), default="erf")
    p.add_argument("--device", default="cuda:0")
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--repeats", type=int, default=20)
    p.add_argument("--execute-gpu", action="store_true",
                   help="authorise device preparation, execution, validation and timing")
    p.add_argument("--profile", action="store_true", help="separate profiler pass after the timing")
    p.add_argument("--dry-run", action="store_true", help="explicit CPU-only mode (also the default)")
    p.add_argument("--write-tuned", action="store_true",
                   help="tune mode: record each case's fastest variants in the tuning table")
    p.add_argument("--tuned-table", default=None,
                   help="tuning table file to write (default: the package's configs/tuned_plans.json)")
    p.add_argument("--output-root", default="results")
    p.add_argument("--validate-only", action="store_true", help=argparse.SUPPRESS)
    return p


def _json(path, data):
    temporary = path.with_suffix(path.suffix + ".tmp")
    temporary.write_text(json.dumps(data, indent=2, allow_nan=False, default=str) + "\n")
    temporary.replace(path)


def manifest():
    """Provenance without initialising a device: interpreter, packages, library revision."""
    import importlib.metadata
    import subprocess
    versions = {}
    for package in ("torch", "numpy"):
        try:
            versions[package] = importlib.metadata.version(package)
        except importlib.metadata.PackageNotFoundError:
            versions[package] = None
    try:
        revision = subprocess.run(["git", "rev-parse", "HEAD"], cwd=REPO_ROOT, capture_output=True,
                                  text=True, timeout=10).stdout.strip() or None
    except (OSError, subprocess.SubprocessError):
        revision = None
    try:
        library = _lib.load().ffn_mi355x_version().decode()
    except OSError as exc:
        library = f"unloadable: {exc}"
    return {"created_utc": datetime.now(timezone.utc).isoformat(),
            "python": platform.python_version(), "platform": platform.platform(),
            "packages": versions, "project_commit": revision, "library": library,
            "device_executed": False, "target": "gfx950 (MI355X)",
            "limitations": ["timings hold for the device, clocks and library revision recorded here",
                            "hardware counters need a rocprofv3 --pmc run of the process"]}


class PerformanceRunner:
    """Purpose: run cases x candidate configurations serially: planning, validation against
    the FP32 golden, device timing and result files.

    Inputs: the Namespace from parser(); the case file must be readable and the output
    root writable.  Only a dry run (planning on the CPU) happens unless execute_gpu is set.
    Outputs: run() returns exit code 0 or 1 and leaves results/<run_id>/; on an exception
    the partial state is saved and the exception re-raised.  One run() per instance.
    """

    def __init__(self, args):
        """Validate arguments, load cases, create the run directory; no device work."""
        self.args = args
        self.validate_arguments()
        self.cases = load_cases(args.cases)
        if args.case_id:
            unknown = set(args.case_id) - {c["case_id"] for c in self.cases}
            if unknown:
                raise ValueError(f"Unknown case IDs: {sorted(unknown)}")
            self.cases = [c for c in self.cases if c["case_id"] in args.case_id]
        if args.mode == "search":
            self.configs = combinations(args.up_candidates, args.down_candidates)
        elif args.mode == "manual":
            self.configs = [{"up_impl": args.up_impl, "down_impl": args.down_impl}]
        else:
            self.configs = None  # per case, from the tile space
        for config in self.configs or []:
            Selection(config["up_impl"], config["down_impl"])
        self.info = manifest()
        run_id = datetime.now(timezone.utc).strftime("%Y%m%dT%H%M%S") + "_" + uuid4().hex[:8]
        self.root = Path(args.output_root) / run_id
        self.root.mkdir(parents=True, exist_ok=False)
        (self.root / "profiler").mkdir()
        self.info.update(arguments=vars(args), cases=self.cases, search_space=self.configs,
                         complete=False, device_executed=False)
        self.records, self.bests = [], {}
        self.case = None
        self.case_index = self.config_index = 0
        self.start_index = 0
        self.inputs = self.golden = None
        self.active_evaluation = None
        self.started = False
        self.case_configs = []
        _json(self.root / "manifest.json", self.info)

    def validate_arguments(self):
        """Reject contradictory modes and invalid counts with ValueError."""
        if self.args.execute_gpu and self.args.dry_run:
            raise ValueError("--execute-gpu and --dry-run are mutually exclusive")
        if self.args.warmup < 0 or self.args.repeats < 1:
            raise ValueError("Invalid timing counts")
        if self.args.write_tuned and (self.args.mode != "tune" or not self.args.execute_gpu):
            raise ValueError("--write-tuned needs --mode tune and --execute-gpu")

    def block_num(self):
        """The workgroup count of every candidate: the argument, the device CU count, or 256."""
        if self.args.block_num is not None:
            return self.args.block_num
        if self.args.execute_gpu:
            import torch
            device = torch.device(self.args.device)
            return _lib.query(device.index or 0)[0]
        return DEFAULT_BLOCK_NUM

    def log(self, message):
        """Print a progress line with the case and configuration position; never inside timing."""
        prefix = datetime.now().strftime("%H:%M:%S")
        if self.case is not None:
            prefix += f" case {self.case_index + 1}/{len(self.cases)} {self.case['case_id']}"
        if self.config_index:
            prefix += f" config {self.config_index}/{len(self.case_configs)}"
        print(f"[{prefix}] {message}", flush=True)

    def persist(self):
        """Write records, bests, CSV, report and manifest of the run so far."""
        _json(self.root / "accuracy.json", self.records)
        _json(self.root / "best_configs.json", self.bests)
        fields = ["case_id", "up_impl", "down_impl", "up_variant", "down_variant", "status",
                  "device_median_us", "refined_median_us", "task_duration_us",
                  "pipeline_utilization", "reason"]
        with (self.root / "performance.csv").open("w", newline="") as stream:
            writer = csv.DictWriter(stream, fieldnames=fields, extrasaction="ignore")
            writer.writeheader()
            for row in self.records:
                entry = {key: row.get(key) for key in fields}
                entry.update(row["configuration"])
                writer.writerow(entry)
        (self.root / "analysis.md").write_text(report(self.records, self.bests))
        _json(self.root / "manifest.json", self.info)

    def prepare_case(self):
        """Compute the CPU golden and fixed device inputs shared by every candidate of the case;
        a dry run skips both."""
        self.inputs = self.golden = None
        if not self.args.execute_gpu:
            self.log("dry run: skipping the CPU golden, device execution and timing")
            return
        import torch
        from .accuracy import golden
        self.log("computing the CPU FP32 golden")
        cpu_inputs = make_inputs(self.case, "cpu")
        self.golden = golden(*cpu_inputs, gelu=self.args.gelu)
        self.log(f"preparing device inputs on {self.args.device}")
        self.info["device_executed"] = True
        self.inputs = make_inputs(self.case, self.args.device)
        torch.cuda.synchronize(self.args.device)
        self.info.update(device_name=torch.cuda.get_device_name(self.args.device),
                         hip_version=getattr(torch.version, "hip", None))
        self.log("device inputs ready")

    def evaluate(self, config):
        """Plan, and on the device prepare, validate and time one configuration; returns the
        record (status planned / passed / not_applicable / unavailable / accuracy_failed /
        compile_failed).  Device preparation errors abort the search."""
        self.config_index += 1
        self.active_evaluation = {"case_id": self.case["case_id"], "configuration": config}
        self.log(f"evaluating {config}")
        row = {"case_id": self.case["case_id"]}
        forced = {k: config[k] for k in ("up_variant", "down_variant") if k in config}
        try:
            plan = make_plan(case_problem(self.case), Selection(config["up_impl"], config["down_impl"]),
                             self.block_num(), gelu=self.args.gelu, **forced)
        except DependencyUnavailable as exc:
            self.log(f"skipped, implementation unavailable: {exc}")
            return dict(row, status="unavailable", reason=str(exc))
        except NotApplicable as exc:
            self.log(f"skipped, not applicable to this case: {exc}")
            return dict(row, status="not_applicable", reason=str(exc))
        row.update(plan=plan.to_dict(), provenance={"library": self.info["library"]})
        if not self.args.execute_gpu:
            return dict(row, status="planned", reason="CPU planning only; not executed on the device")

        import torch
        from ..api import KernelCompilationError, prepare_ffn
        self.log("preparing buffers and binding kernels")
        before = perf_counter()
        try:
            prepared = prepare_ffn(*self.inputs, up_impl=config["up_impl"],
                                   down_impl=config["down_impl"], block_num=self.block_num(),
                                   layout=self.case.get("layout", "linear"), gelu=self.args.gelu,
                                   **forced)
        except KernelCompilationError as exc:
            self.log(f"kernel binding failed: {exc}")
            return dict(row, status="compile_failed", reason=str(exc))
        except Exception as exc:
            row.update(status="preparation_failed", reason=f"{type(exc).__name__}: {exc}")
            self.records.append(dict(row, configuration=config))
            self.persist()
            raise
        torch.cuda.synchronize(self.args.device)
        row["preparation_wall_ms"] = (perf_counter() - before) * 1000
        row.update(prepared.preparation)
        row.update(up_variant=prepared.plan.up.variant, down_variant=prepared.plan.down.variant)
        if not self.validate_prepared(prepared, row):
            return row
        if not self.args.validate_only:
            self.collect_performance(prepared, row, config)
        else:
            self.log("validate-only: no warm-up, timing or profiling")
        return dict(row, status="passed")

    def validate_prepared(self, prepared, row):
        """Run once and compare with the golden, then twice more (repeat invocation); updates
        row and returns whether the golden criterion passed."""
        from .accuracy import compare
        self.log("device run 1 and comparison with the golden")
        output = prepared.run().detach().cpu()
        row["accuracy"] = compare(output, self.golden)
        if not row["accuracy"]["passed"]:
            row.update(status="accuracy_failed", reason="FP32 golden comparison failed")
            self.log(f"accuracy failed: {row['accuracy']}")
            return False
        self.log(f"accuracy passed: mean_rel={row['accuracy']['mean_rel']:.6g}")
        for repeat in range(2):
            if not compare(prepared.run().detach().cpu(), self.golden)["passed"]:
                row.update(status="accuracy_failed", reason="Repeated invocation failed")
                self.log(f"repeat {repeat + 1}/2 failed")
                return False
        self.log("repeat invocations passed")
        return True

    def collect_performance(self, prepared, row, config):
        """Event-time the prepared FFN and, with --profile, run a separate profiler pass."""
        from .collect import time_prepared
        row.update(time_prepared(prepared, self.args.warmup, self.args.repeats, progress=self.log))
        self.log(f"device timing done: median={row['device_median_us']:.3f} us")
        if self.args.profile:
            self.collect_profile(prepared, row, config)

    def collect_profile(self, prepared, row, config):
        """One traced run (torch.profiler) and the FFN kernel durations read from its trace."""
        from .collect import capture_profile, extract_task_duration
        tag = "_".join(str(config.get(k)) for k in ("down_impl", "up_variant", "down_variant") if k in config)
        directory = self.root / "profiler" / f"case_{self.case_index}_{tag}"
        self.log("profiler pass")
        try:
            info = capture_profile(prepared, directory)
            info["profiler_path"] = str(directory.relative_to(self.root))
            row.update(info)
            row.update(extract_task_duration(directory / "trace.json"))
        except (AttributeError, ImportError, RuntimeError) as exc:
            row["profiler_note"] = f"Profiler unavailable: {exc}"
            self.log(f"profiler unavailable: {exc}")

    def checkpoint(self, current, best):
        """Replace this case's records with the search's current list and persist."""
        self.records[self.start_index:] = current
        self.bests[self.case["case_id"]] = dict(
            best, measured=bool(self.args.execute_gpu and not self.args.validate_only))
        self.active_evaluation = None
        self.persist()

    def record_tuned(self):
        """Tune mode: record the fastest passed (up, down) variant pair per down implementation."""
        from .. import tuning
        problem = case_problem(self.case)
        rows = [r for r in self.records[self.start_index:] if r["status"] == "passed"]
        for down in dict.fromkeys(r["configuration"]["down_impl"] for r in rows):
            fastest = pick_fastest([r for r in rows if r["configuration"]["down_impl"] == down])
            p = fastest["plan"]
            key = tuning.make_key(problem.m, p["mp"], p["kp"], p["hp"], p["np"], problem.dtype, down,
                                  self.args.gelu, self.block_num())
            cfg = fastest["configuration"]
            tuning.record(key, cfg["up_variant"], cfg["down_variant"],
                          device_median_us=fastest["device_median_us"], source=self.root.name,
                          path=self.args.tuned_table)
            self.log(f"tuned {down}: up v{cfg['up_variant']} down v{cfg['down_variant']} "
                     f"({fastest['device_median_us']:.2f} us)")

    def run_case(self, index, case):
        """Evaluate every candidate of one case; exceptions propagate to run()."""
        self.case_index, self.case = index, case
        self.config_index = 0
        self.start_index = len(self.records)
        self.bests[case["case_id"]] = {"configuration": None, "complete": False}
        self.log(f"case start: shape={case['shape']} dtype={case['dtype']}")
        self.persist()
        self.prepare_case()
        if self.args.mode == "tune":
            self.tune_case(case)
        else:
            self.case_configs = self.configs
            search(self.case_configs, self.evaluate, self.checkpoint)
        if self.args.write_tuned:
            self.record_tuned()
        self.log("case done")

    def tune_case(self, case):
        """Tune mode: the up variants with the planner's down, then every down variant of each
        down candidate with the fastest up; bests cover both phases."""
        problem = case_problem(case)
        case_start = self.start_index
        downs = [d for d in self.args.down_candidates if d in ("basic", "streamk")]
        self.case_configs = tile_space_up(problem, downs[0], self.block_num(), self.args.gelu)
        self.log(f"tune phase 1: {len(self.case_configs)} up variants")
        _, best = search(self.case_configs, self.evaluate, self.checkpoint)
        up = best["configuration"]["up_variant"] if best["configuration"] else None
        self.start_index = len(self.records)
        self.config_index = 0
        self.case_configs = tile_space_down(problem, downs, up, self.block_num(), self.args.gelu)
        self.log(f"tune phase 2: {len(self.case_configs)} down variants with up v{up}")
        search(self.case_configs, self.evaluate, self.checkpoint)
        self.start_index = case_start
        if self.args.execute_gpu and not self.args.validate_only:
            self.refine(case_start)
        passed = [r for r in self.records[case_start:] if r["status"] == "passed"]
        fastest = pick_fastest(passed)
        self.bests[case["case_id"]] = {
            "configuration": fastest["configuration"] if fastest else None,
            "device_median_us": fastest["device_median_us"] if fastest else None,
            "refined_median_us": fastest.get("refined_median_us") if fastest else None,
            "complete": True, "ranking_metric": "unprofiled_device_event_median_us",
            "measured": bool(self.args.execute_gpu and not self.args.validate_only)}
        self.persist()

    def refine(self, case_start):
        """Tune mode: re-time each down implementation's near-equal finalists side by side
        (collect.time_interleaved) and store the result in their records as refined_median_us."""
        import torch
        from ..api import prepare_ffn
        from .collect import time_interleaved
        rows = [r for r in self.records[case_start:] if r["status"] == "passed"]
        for down in dict.fromkeys(r["configuration"]["down_impl"] for r in rows):
            finalists = refine_candidates([r for r in rows if r["configuration"]["down_impl"] == down])
            if len(finalists) < 2:
                continue
            self.log(f"refining {down}: " + ", ".join(
                f"up v{r['configuration']['up_variant']} down v{r['configuration']['down_variant']}"
                for r in finalists) + " interleaved")
            prepared = [prepare_ffn(*self.inputs, up_impl="basic", down_impl=down,
                                    block_num=self.block_num(), layout=self.case.get("layout", "linear"),
                                    gelu=self.args.gelu, up_variant=r["configuration"]["up_variant"],
                                    down_variant=r["configuration"]["down_variant"]) for r in finalists]
            for r, value in zip(finalists, time_interleaved(prepared)):
                r["refined_median_us"] = value
                self.log(f"  up v{r['configuration']['up_variant']} down v{r['configuration']['down_variant']}: "
                         f"{value:.2f} us per run (back-to-back)")
            del prepared
            torch.cuda.synchronize(self.args.device)
        self.persist()

    def save_failure(self, exc):
        """Save the interrupted state and the active candidate's reason; never marks success."""
        reason = f"{type(exc).__name__}: {exc}"
        self.info["interrupted_or_failed"] = reason
        if self.active_evaluation is not None and not any(
                r["case_id"] == self.active_evaluation["case_id"]
                and r["configuration"] == self.active_evaluation["configuration"] for r in self.records):
            self.records.append(dict(self.active_evaluation, status="interrupted_or_failed", reason=reason))
        self.log(f"run interrupted or failed: {reason}; saving state")
        self.persist()

    def run(self):
        """All cases in order, then the final report; 0 on success, 1 on an accuracy failure or
        when a device run produced no passing candidate."""
        if self.started:
            raise RuntimeError("PerformanceRunner.run() may only be called once")
        self.started = True
        mode = "device execution" if self.args.execute_gpu else "dry run, no device execution"
        self.log(f"run start: {len(self.cases)} cases, mode {self.args.mode}, {mode}")
        try:
            for index, case in enumerate(self.cases):
                self.run_case(index, case)
            self.info["complete"] = True
        except BaseException as exc:
            self.save_failure(exc)
            raise
        self.case = None
        self.config_index = 0
        self.persist()
        self.log(f"all cases done; results in {self.root}")
        if self.args.execute_gpu and any(r["status"] == "accuracy_failed" for r in self.records):
            return 1
        if self.args.execute_gpu and not any(r["status"] == "passed" for r in self.records):
            return 1
        return 0


def main(argv=None):
    """Parse the arguments and run; returns the exit code."""
    return PerformanceRunner(parser().parse_args(argv)).run()


if __name__ == "__main__":
    raise SystemExit(main())
