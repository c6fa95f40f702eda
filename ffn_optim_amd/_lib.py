"""ctypes binding of ``libffn_mi355x.so`` (declarations in include/ffn_mi355x.h).

Loading the library touches no GPU; only the run entry points and
``ffn_mi355x_query`` talk to the HIP runtime.  Return codes are mapped onto the
reference's exception taxonomy (ops/api.py:9-14, ops/host/dispatch.py:22-39).
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().parent / "libffn_mi355x.so"

FP16, BF16 = 0, 1
DOWN_CODES = {"basic": 0, "streamk": 1, "full_load_a": 2, "full_load_b": 3}
GELU_CODES = {"erf": 0, "rational": 1}
# activation of the up epilogue (the GELU codes above, then SiLU and SwiGLU)
ACTIVATION_CODES = {"gelu:erf": 0, "gelu:rational": 1, "silu": 2, "swiglu": 3}

OK, EINVAL, ENOT_APPLICABLE, EUNAVAILABLE, EHIP, EDEVICE = 0, -1, -2, -3, -4, -5
# FFN_MI355X_MAX_PITCH: the largest operand row pitch (elements) ffn_mi355x_set_operands accepts
MAX_PITCH = 4_000_000
# FFN_MI355X_SPLIT_COUNTER_WORDS: words from one split tile's arrival counters to the next, when
# both GEMMs' split tiles fit the counter region that way (else one word per tile wave)
SPLIT_COUNTER_WORDS = 32


class PlanStruct(ctypes.Structure):
    """Mirror of ``ffn_mi355x_plan``."""

    _fields_ = [(name, ctypes.c_int) for name in (
        "m", "mp", "kp", "hp", "np", "dtype", "down_impl", "activation", "block_num",
        "up_variant", "down_variant", "up_bm", "up_bn", "up_bk",
        "down_bm", "down_bn", "down_bk", "up_tiles", "up_grid",
        "down_tiles", "down_grid", "down_k_iters", "down_dp_tiles",
        "down_sk_tiles", "down_slots_per_wg")] + [("workspace_bytes", ctypes.c_size_t)] + [
        (name, ctypes.c_int) for name in ("k", "h", "n", "ldx", "ldw1", "ldw2",
                                          "up_k_iters", "up_sk_tiles", "up_slots_per_wg",
                                          "x_d1", "x_d2", "x_s0", "x_s1", "x_s2",
                                          "single_launch")] + [
        ("stamp", ctypes.c_ulonglong)]

    def to_dict(self):
        return {name: getattr(self, name) for name, _ in self._fields_}


_P = ctypes.POINTER
_vp = ctypes.c_void_p
_i = ctypes.c_int
# Entry points that load, query and plan: a library lacking one of them cannot serve this host
# at all (load() raises LibraryMismatch, which prepare_ffn reports as DependencyUnavailable).
CORE_SIGNATURES = {
    "ffn_mi355x_query": (_i, [_i, _P(_i), ctypes.c_char_p, _i]),
    "ffn_mi355x_make_plan": (_i, [_i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _P(PlanStruct)]),
    "ffn_mi355x_workspace_bytes": (_i, [_P(PlanStruct), _P(ctypes.c_size_t)]),
    "ffn_mi355x_workspace_counter_bytes": (_i, [_P(PlanStruct), _P(ctypes.c_size_t)]),
    "ffn_mi355x_set_operands": (_i, [_P(PlanStruct), _i, _i, _i, _i, _i, _i]),
    "ffn_mi355x_set_x_rows": (_i, [_P(PlanStruct), _i, _i, _i, _i, _i]),
    "ffn_mi355x_set_single_launch": (_i, [_P(PlanStruct), _i]),
    "ffn_mi355x_num_variants": (_i, []),
    "ffn_mi355x_variant_info": (_i, [_i, _P(_i), _P(_i), _P(_i), _P(_i), _P(_i), _P(_i)]),
    "ffn_mi355x_variant_refill_waves": (_i, [_i]),
    "ffn_mi355x_variant_mfma_edge": (_i, [_i]),
    "ffn_mi355x_last_error": (ctypes.c_char_p, []),
    "ffn_mi355x_strerror": (ctypes.c_char_p, [_i]),
    "ffn_mi355x_version": (ctypes.c_char_p, []),
}
# Launch entry points, bound when present: compile_kernel requires those a plan launches
# through (require_entry_points), and a library without them fails there, the counterpart of
# the reference's compile step failing (KernelCompilationError, ops/api.py:82-88).
LAUNCH_SIGNATURES = {
    "ffn_mi355x_run": (_i, [_P(PlanStruct), _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "ffn_mi355x_run_noalloc": (_i, [_P(PlanStruct), _vp, _vp, _vp, _vp, _vp, _vp]),
    "ffn_mi355x_run_ex": (_i, [_P(PlanStruct), _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "ffn_mi355x_up_ex": (_i, [_P(PlanStruct), _vp, _vp, _vp, _vp, _vp, _vp]),
    "ffn_mi355x_down_ex": (_i, [_P(PlanStruct), _vp, _vp, _vp, _vp, _vp, _vp]),
    "ffn_mi355x_up": (_i, [_P(PlanStruct), _vp, _vp, _vp, _vp, _vp]),
    "ffn_mi355x_down": (_i, [_P(PlanStruct), _vp, _vp, _vp, _vp, _vp]),
}
SIGNATURES = {**CORE_SIGNATURES, **LAUNCH_SIGNATURES}


class LibraryMismatch(OSError):
    """The shared object loads but lacks entry points this host calls (a stale or foreign
    build)."""


def _bind(lib) -> list[str]:
    """Set restype/argtypes of every entry point the library exports; returns the names of
    the missing launch entry points.  A missing core entry point raises LibraryMismatch."""
    missing_core, missing_launch = [], []
    for table, missing in ((CORE_SIGNATURES, missing_core), (LAUNCH_SIGNATURES, missing_launch)):
        for name, (res, args) in table.items():
            try:
                fn = getattr(lib, name)
            except AttributeError:
                missing.append(name)
                continue
            fn.restype, fn.argtypes = res, args
    if missing_core:
        raise LibraryMismatch(f"{lib._name} does not export {', '.join(missing_core)}; "
                              "rebuild it with `python -m ffn_optim_amd.build`")
    lib._ffn_missing_launch = tuple(missing_launch)
    return missing_launch


_lock = threading.Lock()
_lib = None


def load(path: Path | str | None = None):
    """Load (once) and return the library; raises OSError if it cannot be loaded, and
    LibraryMismatch (an OSError) if it lacks a core entry point.

    torch is imported first: it loads its own copy of the HIP runtime by path, and the
    library's libamdhip64.so.7 dependency must then resolve (by soname) to that same copy.
    Loaded the other way round, the process holds two HIP runtimes and the library's sees
    no device once torch's owns it.  Importing torch initialises no GPU.
    """
    global _lib
    import torch  # noqa: F401  (HIP runtime load order, see above)
    with _lock:
        if _lib is None or path is not None:
            lib = ctypes.CDLL(str(path or LIBRARY_PATH), mode=ctypes.RTLD_LOCAL)
            _bind(lib)
            if path is not None:
                return lib
            _lib = lib
        return _lib


def require_entry_points(lib, names) -> None:
    """RuntimeError naming the launch entry points of `names` that `lib` does not export."""
    absent = [n for n in names if n in getattr(lib, "_ffn_missing_launch", ())]
    if absent:
        raise RuntimeError(f"{lib._name} does not export the launch entry point(s) "
                           f"{', '.join(absent)}")


def last_error() -> str:
    return load().ffn_mi355x_last_error().decode()


def check(rc: int) -> None:
    """Raise the reference-equivalent exception for a non-zero return code."""
    if rc == OK:
        return
    from .host.dispatch import DependencyUnavailable, NotApplicable
    msg = last_error() or load().ffn_mi355x_strerror(rc).decode()
    if rc == EINVAL:
        raise ValueError(msg)
    if rc == ENOT_APPLICABLE:
        raise NotApplicable(msg)
    if rc == EUNAVAILABLE:
        raise DependencyUnavailable(msg)
    raise RuntimeError(msg)


def query(device: int) -> tuple[int, str]:
    """(CU count, gcnArchName) of a device; RuntimeError unless it is gfx950."""
    lib = load()
    cus = ctypes.c_int(0)
    arch = ctypes.create_string_buffer(64)
    check(lib.ffn_mi355x_query(device, ctypes.byref(cus), arch, len(arch)))
    return cus.value, arch.value.decode()


def activation_code(activation="gelu", gelu="erf") -> int:
    """Code of the up epilogue: a GELU form, SiLU or SwiGLU."""
    key = f"gelu:{gelu}" if activation == "gelu" else activation
    if key not in ACTIVATION_CODES:
        raise ValueError(f"activation must be gelu, silu or swiglu and gelu erf or rational "
                         f"(got {activation!r}, {gelu!r})")
    return ACTIVATION_CODES[key]


def make_plan(mp, kp, hp, np_, dtype, down_impl, gelu, block_num, up_variant=-1,
              down_variant=-1, m=None, activation="gelu") -> PlanStruct:
    """Native plan; `m` is the logical row count (default: all mp rows hold data); `gelu` is the
    GELU form when activation is 'gelu'."""
    plan = PlanStruct()
    check(load().ffn_mi355x_make_plan(mp if m is None else m, mp, kp, hp, np_, dtype,
                                      DOWN_CODES[down_impl],
                                      activation_code(activation, gelu), block_num, up_variant,
                                      down_variant, ctypes.byref(plan)))
    return plan


def set_operands(plan: PlanStruct, k, h, n, ldx, ldw1, ldw2) -> None:
    """Point a native plan at operands of their logical widths (ffn_mi355x_set_operands)."""
    check(load().ffn_mi355x_set_operands(ctypes.byref(plan), k, h, n, ldx, ldw1, ldw2))


def workspace_counter_bytes(plan: PlanStruct) -> int:
    """Leading workspace bytes (arrival counters) that must be zero before first use."""
    n = ctypes.c_size_t()
    check(load().ffn_mi355x_workspace_counter_bytes(ctypes.byref(plan), ctypes.byref(n)))
    return n.value


def set_single_launch(plan: PlanStruct, on: bool) -> None:
    """Run the plan's FFN as one launch or as two (ffn_mi355x_set_single_launch)."""
    check(load().ffn_mi355x_set_single_launch(ctypes.byref(plan), 1 if on else 0))


def set_x_rows(plan: PlanStruct, d1, d2, s0, s1, s2) -> None:
    """Read X as gathered rows of a strided view (ffn_mi355x_set_x_rows); d1 = 0 undoes it."""
    check(load().ffn_mi355x_set_x_rows(ctypes.byref(plan), d1, d2, s0, s1, s2))


def variants() -> list[dict]:
    lib = load()
    out = []
    for v in range(lib.ffn_mi355x_num_variants()):
        vals = [ctypes.c_int(0) for _ in range(6)]
        check(lib.ffn_mi355x_variant_info(v, *map(ctypes.byref, vals)))
        refill = lib.ffn_mi355x_variant_refill_waves(v)
        check(min(refill, 0))
        edge = lib.ffn_mi355x_variant_mfma_edge(v)
        check(min(edge, 0))
        out.append(dict(zip(("bm", "bn", "bk", "waves", "stages", "lds_bytes"),
                            (x.value for x in vals)), variant=v, refill_waves=refill, mfma_edge=edge))
    return out
