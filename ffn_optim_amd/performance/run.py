"""Command-line entry of the FFN measurement harness (the counterpart of performance/run.py).

    python -m ffn_optim_amd.performance.run --mode search --execute-gpu
    python -m ffn_optim_amd.performance.run --mode tune --execute-gpu --write-tuned \\
        --cases ffn_optim_amd/configs/benchmark_cases.json

Without --execute-gpu the run is a plan-only pass: every candidate is planned through the library
on the CPU and nothing touches a GPU.  --execute-gpu authorises device work per candidate:
preparation (prepare_ffn), validation of three runs against the FP32 golden, event timing and,
with --profile, a separate profiler pass.

Modes: manual (one --up-impl/--down-impl), search (the --up-candidates x --down-candidates
product) and tune (the compiled tile variants, one GEMM at a time: every up variant with the
planner's down, then every down variant of each Basic/Stream-K candidate with the fastest up, the
near-equal finalists re-timed side by side; --write-tuned stores each down implementation's
fastest pair in the tuning table prepare_ffn consults).

Each run writes results/<run_id>/ (run id: UTC timestamp and 8 hex digits) and never reuses one:
manifest.json, accuracy.json (one record per evaluated candidate, with the golden comparison in
``accuracy`` and the staged rational-GELU comparison in ``staged_accuracy``), performance.csv,
best_configs.json, analysis.md and profiler/.  The files are rewritten after every candidate, so
an interrupted run keeps what it measured; the manifest then records the interruption.
"""
from __future__ import annotations

import argparse
import csv
import json
import platform
from dataclasses import dataclass
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
CSV_FIELDS = ["case_id", "up_impl", "down_impl", "up_variant", "down_variant", "status",
              "device_median_us", "refined_median_us", "task_duration_us",
              "pipeline_utilization", "reason"]


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


def check_arguments(args):
    """ValueError for contradictory flags or impossible timing counts."""
    problems = []
    if args.execute_gpu and args.dry_run:
        problems.append("--execute-gpu and --dry-run are mutually exclusive")
    if args.warmup < 0 or args.repeats < 1:
        problems.append("Invalid timing counts: --warmup >= 0 and --repeats >= 1")
    if args.write_tuned and not (args.mode == "tune" and args.execute_gpu):
        problems.append("--write-tuned needs --mode tune and --execute-gpu")
    if problems:
        raise ValueError("; ".join(problems))


def select_cases(args):
    """The case list of the run: the file's cases, restricted to --case-id when given."""
    cases = load_cases(args.cases)
    if not args.case_id:
        return cases
    known = [c["case_id"] for c in cases]
    missing = sorted(set(args.case_id) - set(known))
    if missing:
        raise ValueError(f"Unknown case IDs: {missing}")
    return [c for c in cases if c["case_id"] in args.case_id]


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


class RunDirectory:
    """results/<run_id>/: created empty, then rewritten as a whole after every candidate.

    JSON files are replaced atomically (written aside, then renamed), so a reader or an
    interruption never sees a half-written file.
    """

    def __init__(self, output_root):
        run_id = datetime.now(timezone.utc).strftime("%Y%m%dT%H%M%S") + "_" + uuid4().hex[:8]
        self.root = Path(output_root) / run_id
        self.root.mkdir(parents=True, exist_ok=False)
        (self.root / "profiler").mkdir()

    def write_json(self, name, data):
        target = self.root / name
        aside = target.with_name(target.name + ".tmp")
        aside.write_text(json.dumps(data, indent=2, allow_nan=False, default=str) + "\n")
        aside.replace(target)

    def write_all(self, info, records, bests):
        """Every artefact from the run's current state."""
        self.write_json("accuracy.json", records)
        self.write_json("best_configs.json", bests)
        with (self.root / "performance.csv").open("w", newline="") as stream:
            out = csv.DictWriter(stream, fieldnames=CSV_FIELDS, extrasaction="ignore")
            out.writeheader()
            out.writerows({**{f: r.get(f) for f in CSV_FIELDS}, **r["configuration"]} for r in records)
        (self.root / "analysis.md").write_text(report(records, bests))
        self.write_json("manifest.json", info)


class CandidateStop(Exception):
    """Ends the evaluation of one candidate with a final status (not an error of the run)."""

    def __init__(self, status, reason):
        super().__init__(reason)
        self.status, self.reason = status, reason


@dataclass
class CaseData:
    """What every candidate of one case shares: the FP32 golden, the staged rational-GELU golden
    and the device inputs (all None in a plan-only run)."""

    golden: object = None
    staged: object = None
    inputs: tuple | None = None


class PerformanceRunner:
    """Purpose: evaluate every case of a case file against a list of candidate configurations,
    one candidate at a time, and keep the evidence in results/<run_id>/.

    Inputs: the Namespace of parser(); the case file must be readable and --output-root
    writable.  Device work happens only with --execute-gpu.
    Outputs: run() returns 0, or 1 when a device run had an accuracy failure or no passing
    candidate; the run directory holds every record.  An exception is recorded in the run
    directory and re-raised.  run() may be called once per instance.
    """

    def __init__(self, args):
        """Check the arguments, select the cases and create the run directory; no device work."""
        check_arguments(args)
        self.args = args
        self.cases = select_cases(args)
        self.fixed_space = None
        if args.mode == "search":
            self.fixed_space = combinations(args.up_candidates, args.down_candidates)
        elif args.mode == "manual":
            self.fixed_space = [{"up_impl": args.up_impl, "down_impl": args.down_impl}]
        for candidate in self.fixed_space or []:
            Selection(candidate["up_impl"], candidate["down_impl"])
        self.store = RunDirectory(args.output_root)
        self.root = self.store.root
        self.info = manifest()
        self.info.update(arguments=vars(args), cases=self.cases, search_space=self.fixed_space,
                         complete=False, device_executed=False)
        self.records, self.bests = [], {}
        self.case = None
        self.case_index = 0
        self.case_first = 0          # index in self.records of the current case's first record
        self.space = []              # candidates of the current sweep (for progress lines)
        self.position = 0            # 1-based position in that sweep, 0 between candidates
        self.data = CaseData()
        self.pending = None          # (case_id, configuration) being evaluated
        self.used = False
        self.store.write_json("manifest.json", self.info)

    # -- progress and persistence ---------------------------------------------------------------

    def log(self, message):
        """One progress line: wall time, case and candidate position, message.  Never called
        inside a timed region."""
        where = [datetime.now().strftime("%H:%M:%S")]
        if self.case is not None:
            where.append(f"case {self.case_index + 1}/{len(self.cases)} {self.case['case_id']}")
        if self.position:
            where.append(f"config {self.position}/{len(self.space)}")
        print(f"[{' '.join(where)}] {message}", flush=True)

    def persist(self):
        """Write every artefact from the current state."""
        self.store.write_all(self.info, self.records, self.bests)

    def block_num(self):
        """Workgroups of every candidate: --block-num, else the device's CU count (256 in a
        plan-only run)."""
        if self.args.block_num is not None:
            return self.args.block_num
        if not self.args.execute_gpu:
            return DEFAULT_BLOCK_NUM
        import torch
        return _lib.query(torch.device(self.args.device).index or 0)[0]

    def measured(self):
        """Whether records of this run carry device timings."""
        return bool(self.args.execute_gpu and not self.args.validate_only)

    # -- one case -------------------------------------------------------------------------------

    def prepare_case(self):
        """The case's shared data: the FP32 golden, the staged rational-GELU golden (the kernel's
        own form: rational GELU, hidden rounded to the input dtype) and the device inputs.  A
        plan-only run computes none of them."""
        self.data = CaseData()
        if not self.args.execute_gpu:
            self.log("dry run: skipping the CPU golden, device execution and timing")
            return
        import torch
        from .accuracy import golden
        self.log("computing the CPU FP32 golden and the staged rational-GELU golden")
        host_inputs = make_inputs(self.case, "cpu")
        self.data.golden = golden(*host_inputs, gelu=self.args.gelu)
        self.data.staged = golden(*host_inputs, gelu="rational", staged=True)
        self.log(f"preparing device inputs on {self.args.device}")
        self.data.inputs = make_inputs(self.case, self.args.device)
        torch.cuda.synchronize(self.args.device)
        self.info.update(device_executed=True, device_name=torch.cuda.get_device_name(self.args.device),
                         hip_version=getattr(torch.version, "hip", None))
        self.log("device inputs ready")

    def sweep(self, candidates):
        """Evaluate a candidate list of the current case; returns search()'s (records, best)."""
        self.space, self.position = candidates, 0
        return search(candidates, self.evaluate, self.checkpoint, progress=None)

    def checkpoint(self, case_records, best):
        """search()'s callback: the current sweep's records replace the case's tail, then persist."""
        self.records[self.case_first:] = case_records
        self.bests[self.case["case_id"]] = dict(best, measured=self.measured())
        self.pending = None
        self.persist()

    def run_case(self, index, case):
        """Evaluate every candidate of one case (exceptions propagate to run())."""
        self.case_index, self.case, self.position = index, case, 0
        self.case_first = len(self.records)
        self.bests[case["case_id"]] = {"configuration": None, "complete": False}
        self.log(f"case start: shape={case['shape']} dtype={case['dtype']}")
        self.persist()
        self.prepare_case()
        if self.args.mode == "tune":
            self.tune_case()
        else:
            self.sweep(self.fixed_space)
        if self.args.write_tuned:
            self.record_tuned()
        self.log("case done")

    # -- one candidate --------------------------------------------------------------------------

    def evaluate(self, config):
        """The record of one candidate.  Its status is the step where it stopped: planned (plan
        only), unavailable, not_applicable, compile_failed, accuracy_failed -- or passed after
        validation and timing.  A device preparation error aborts the run after it is recorded."""
        self.position += 1
        self.pending = (self.case["case_id"], config)
        self.log(f"evaluating {config}")
        record = {"case_id": self.case["case_id"]}
        try:
            self.plan_step(config, record)
            prepared = self.prepare_step(config, record)
            self.validate_step(prepared, record)
            if self.args.validate_only:
                self.log("validate-only: no warm-up, timing or profiling")
            else:
                self.measure_step(prepared, record, config)
        except CandidateStop as stop:
            record.update(status=stop.status, reason=stop.reason)
            self.log(f"{stop.status}: {stop.reason}")
            return record
        record["status"] = "passed"
        return record

    def plan_step(self, config, record):
        """Plan on the CPU; a plan-only run stops here with status 'planned'."""
        forced = {k: config[k] for k in ("up_variant", "down_variant") if k in config}
        try:
            plan = make_plan(case_problem(self.case), Selection(config["up_impl"], config["down_impl"]),
                             self.block_num(), gelu=self.args.gelu, **forced)
        except DependencyUnavailable as exc:
            raise CandidateStop("unavailable", str(exc)) from exc
        except NotApplicable as exc:
            raise CandidateStop("not_applicable", str(exc)) from exc
        record.update(plan=plan.to_dict(), provenance={"library": self.info["library"]})
        if not self.args.execute_gpu:
            raise CandidateStop("planned", "CPU planning only; not executed on the device")

    def prepare_step(self, config, record):
        """prepare_ffn on the case's device inputs; a binding failure ends the candidate
        (compile_failed), any other failure is recorded and re-raised."""
        import torch
        from ..api import KernelCompilationError, prepare_ffn
        forced = {k: config[k] for k in ("up_variant", "down_variant") if k in config}
        self.log("preparing buffers and binding kernels")
        started = perf_counter()
        try:
            prepared = prepare_ffn(*self.data.inputs, up_impl=config["up_impl"],
                                   down_impl=config["down_impl"], block_num=self.block_num(),
                                   layout=self.case.get("layout", "linear"), gelu=self.args.gelu,
                                   **forced)
        except KernelCompilationError as exc:
            raise CandidateStop("compile_failed", str(exc)) from exc
        except Exception as exc:
            self.records.append(dict(record, configuration=config, status="preparation_failed",
                                     reason=f"{type(exc).__name__}: {exc}"))
            self.persist()
            raise
        torch.cuda.synchronize(self.args.device)
        record.update(prepared.preparation, preparation_wall_ms=(perf_counter() - started) * 1000,
                      up_variant=prepared.plan.up.variant, down_variant=prepared.plan.down.variant)
        return prepared

    def validate_step(self, prepared, record):
        """Three runs against the FP32 golden (the first also against the staged rational-GELU
        golden, recorded, not judged); any failure ends the candidate (accuracy_failed)."""
        from .accuracy import compare
        self.log("device run 1 and comparison with the golden")
        first = prepared.run().detach().cpu()
        record["accuracy"] = compare(first, self.data.golden)
        record["staged_accuracy"] = compare(first, self.data.staged)
        if not record["accuracy"]["passed"]:
            raise CandidateStop("accuracy_failed", "FP32 golden comparison failed")
        self.log(f"accuracy passed: mean_rel={record['accuracy']['mean_rel']:.6g} "
                 f"(staged rational: {record['staged_accuracy']['mean_rel']:.6g})")
        for attempt in (2, 3):
            if not compare(prepared.run().detach().cpu(), self.data.golden)["passed"]:
                raise CandidateStop("accuracy_failed", f"Repeated invocation failed (run {attempt})")
        self.log("repeat invocations passed")

    def measure_step(self, prepared, record, config):
        """Event timing; with --profile, one separate profiler pass whose numbers never rank."""
        from .collect import capture_profile, extract_task_duration, time_prepared
        record.update(time_prepared(prepared, self.args.warmup, self.args.repeats, progress=self.log))
        self.log(f"device timing done: median={record['device_median_us']:.3f} us")
        if not self.args.profile:
            return
        label = "_".join(str(config[k]) for k in ("down_impl", "up_variant", "down_variant") if k in config)
        folder = self.root / "profiler" / f"case_{self.case_index}_{label}"
        self.log("profiler pass")
        try:
            record.update(capture_profile(prepared, folder), profiler_path=str(folder.relative_to(self.root)))
            record.update(extract_task_duration(folder / "trace.json"))
        except (AttributeError, ImportError, RuntimeError) as exc:
            record["profiler_note"] = f"Profiler unavailable: {exc}"
            self.log(f"profiler unavailable: {exc}")

    # -- tune mode ------------------------------------------------------------------------------

    def tune_case(self):
        """Tile variants one GEMM at a time: the up variants with the planner's down, then the down
        variants of each Basic/Stream-K candidate with the fastest up; then the near-equal
        finalists are re-timed side by side and the case's best covers both phases."""
        problem = case_problem(self.case)
        downs = [d for d in self.args.down_candidates if d in ("basic", "streamk")]
        first = self.case_first
        phase1 = tile_space_up(problem, downs[0], self.block_num(), self.args.gelu)
        self.log(f"tune phase 1: {len(phase1)} up variants")
        _, best = self.sweep(phase1)
        up = (best["configuration"] or {}).get("up_variant")
        self.case_first = len(self.records)
        phase2 = tile_space_down(problem, downs, up, self.block_num(), self.args.gelu)
        self.log(f"tune phase 2: {len(phase2)} down variants with up v{up}")
        self.sweep(phase2)
        self.case_first = first
        if self.measured():
            self.refine(first)
        winner = pick_fastest([r for r in self.records[first:] if r["status"] == "passed"])
        self.bests[self.case["case_id"]] = {
            "configuration": winner["configuration"] if winner else None,
            "device_median_us": winner["device_median_us"] if winner else None,
            "refined_median_us": winner.get("refined_median_us") if winner else None,
            "complete": True, "ranking_metric": "unprofiled_device_event_median_us",
            "measured": self.measured()}
        self.persist()

    def refine(self, first):
        """Re-time each down implementation's near-equal finalists side by side
        (collect.time_interleaved) and store the result as their refined_median_us."""
        import torch
        from ..api import prepare_ffn
        from .collect import time_interleaved
        passed = [r for r in self.records[first:] if r["status"] == "passed"]
        for down in dict.fromkeys(r["configuration"]["down_impl"] for r in passed):
            finalists = refine_candidates([r for r in passed if r["configuration"]["down_impl"] == down])
            if len(finalists) < 2:
                continue
            pairs = [(r["configuration"]["up_variant"], r["configuration"]["down_variant"]) for r in finalists]
            self.log(f"refining {down}: " + ", ".join(f"up v{u} down v{d}" for u, d in pairs) + " interleaved")
            prepared = [prepare_ffn(*self.data.inputs, up_impl="basic", down_impl=down,
                                    block_num=self.block_num(), layout=self.case.get("layout", "linear"),
                                    gelu=self.args.gelu, up_variant=u, down_variant=d) for u, d in pairs]
            for r, (u, d), value in zip(finalists, pairs, time_interleaved(prepared)):
                r["refined_median_us"] = value
                self.log(f"  up v{u} down v{d}: {value:.2f} us per run (back-to-back)")
            del prepared
            torch.cuda.synchronize(self.args.device)
        self.persist()

    def record_tuned(self):
        """Tune mode with --write-tuned: the fastest passed (up, down) variant pair of each down
        implementation goes into the tuning table."""
        from .. import tuning
        problem = case_problem(self.case)
        passed = [r for r in self.records[self.case_first:] if r["status"] == "passed"]
        for down in dict.fromkeys(r["configuration"]["down_impl"] for r in passed):
            winner = pick_fastest([r for r in passed if r["configuration"]["down_impl"] == down])
            plan, cfg = winner["plan"], winner["configuration"]
            key = tuning.make_key(problem.m, plan["mp"], plan["kp"], plan["hp"], plan["np"], problem.dtype,
                                  down, self.args.gelu, self.block_num())
            tuning.record(key, cfg["up_variant"], cfg["down_variant"],
                          device_median_us=winner["device_median_us"], source=self.root.name,
                          path=self.args.tuned_table)
            self.log(f"tuned {down}: up v{cfg['up_variant']} down v{cfg['down_variant']} "
                     f"({winner['device_median_us']:.2f} us)")

    # -- the run --------------------------------------------------------------------------------

    def save_failure(self, exc):
        """Record an interruption or failure: the manifest names it, the candidate being
        evaluated gets an interrupted_or_failed record unless it already has one; the run is
        never marked complete."""
        reason = f"{type(exc).__name__}: {exc}"
        self.info["interrupted_or_failed"] = reason
        if self.pending is not None:
            case_id, config = self.pending
            if not any(r["case_id"] == case_id and r["configuration"] == config for r in self.records):
                self.records.append({"case_id": case_id, "configuration": config,
                                     "status": "interrupted_or_failed", "reason": reason})
        self.log(f"run interrupted or failed: {reason}; saving state")
        self.persist()

    def exit_code(self):
        """1 when a device run had an accuracy failure or produced no passing candidate."""
        if not self.args.execute_gpu:
            return 0
        statuses = {r["status"] for r in self.records}
        return 1 if "accuracy_failed" in statuses or "passed" not in statuses else 0

    def run(self):
        """Every case in order, then the final artefacts; returns the exit code."""
        if self.used:
            raise RuntimeError("PerformanceRunner.run() may only be called once")
        self.used = True
        kind = "device execution" if self.args.execute_gpu else "dry run, no device execution"
        self.log(f"run start: {len(self.cases)} cases, mode {self.args.mode}, {kind}")
        try:
            for index, case in enumerate(self.cases):
                self.run_case(index, case)
        except BaseException as exc:
            self.save_failure(exc)
            raise
        self.info["complete"] = True
        self.case, self.position = None, 0
        self.persist()
        self.log(f"all cases done; results in {self.root}")
        return self.exit_code()


def main(argv=None):
    """Parse the arguments and run; returns the exit code."""
    return PerformanceRunner(parser().parse_args(argv)).run()


if __name__ == "__main__":
    raise SystemExit(main())
