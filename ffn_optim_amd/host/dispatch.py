"""Implementation selection and library loading: no silent fallbacks.

Restates the selection half of ops/host/dispatch.py (DOWN_IMPLS :15,
KERNEL_ENTRIES :16-19, DependencyUnavailable :22-29, NotApplicable :32-39,
Selection :42-66).  The CATLASS pinning (verify_dependency :69-83) and the JIT
``tla.compile`` (compile_kernel :97-116) become a check of the prebuilt gfx950
library and a load of its C entry points.
"""
from __future__ import annotations

import ctypes
import hashlib
from dataclasses import dataclass

DOWN_IMPLS = ("basic", "full_load_a", "full_load_b", "streamk")
GELU_FORMS = ("erf", "rational")
# C-ABI entry point and the down-projection role it runs
KERNEL_ENTRIES = {
    "basic": "ffn_mi355x_run[down=basic]",
    "streamk": "ffn_mi355x_run[down=streamk]",
}


class DependencyUnavailable(RuntimeError):
    """A dependency is missing or the selected implementation is not provided (no fallback)."""


class NotApplicable(ValueError):
    """An existing implementation does not apply to this shape / block_num."""


@dataclass(frozen=True)
class Selection:
    """Up/down implementation of one FFN, never switched automatically (dispatch.py:42-66).

    up_impl must be 'basic'; down_impl is one of DOWN_IMPLS.  require_available()
    raises DependencyUnavailable for the full-load variants, which have no gfx950
    kernel.
    """

    up_impl: str = "basic"
    down_impl: str = "basic"

    def __post_init__(self):
        if self.up_impl != "basic":
            raise ValueError("up_impl must be basic")
        if self.down_impl not in DOWN_IMPLS:
            raise ValueError(f"Unknown down_impl: {self.down_impl}")

    def require_available(self):
        if self.down_impl in ("full_load_a", "full_load_b"):
            raise DependencyUnavailable(
                f"{self.down_impl}: no gfx950 kernel is provided for this down variant; no fallback")
        return self


def verify_dependency():
    """Check that the prebuilt gfx950 library is present and loadable; return its provenance."""
    from .. import _lib

    path = _lib.LIBRARY_PATH
    if not path.exists():
        raise DependencyUnavailable(
            f"{path.name} is not built; run `python -m ffn_optim_amd.build` first")
    try:
        lib = _lib.load()
    except OSError as exc:
        raise DependencyUnavailable(f"cannot load {path.name}: {exc}") from exc
    return {"library": str(path),
            "library_sha256": hashlib.sha256(path.read_bytes()).hexdigest(),
            "version": lib.ffn_mi355x_version().decode()}


def compile_kernel(plan):
    """Resolve the launch entry point for a plan; returns (artifact, provenance).

    The counterpart of the reference's compile step: the kernels are already
    compiled for gfx950, so this loads the library and binds the plan.  The
    artifact launches up + down on the stream it is given.  Raises RuntimeError when
    the library lacks a launch entry point or the plan's tile variants (prepare_ffn
    reports it as KernelCompilationError).
    """
    Selection(plan.selection.up_impl, plan.selection.down_impl).require_available()
    provenance = verify_dependency()
    from .. import _lib

    lib = _lib.load()
    native = plan.native
    # binding: the entry points this artifact launches through, and the plan's tile variants
    _lib.require_entry_points(lib, ("ffn_mi355x_run", "ffn_mi355x_run_ex"))
    for variant in (native.up_variant, native.down_variant):
        if not 0 <= variant < lib.ffn_mi355x_num_variants():
            raise RuntimeError(f"tile variant {variant} is not compiled into {_lib.LIBRARY_PATH.name}")
    plan_ref = ctypes.byref(native)
    run, run_ex = lib.ffn_mi355x_run, lib.ffn_mi355x_run_ex

    def artifact(x, w1, w2, hidden, out, ws, *rest):
        """Launch on the stream given last; bias1 and bias2 (device addresses) may come
        before it (the EagleFFN form with biases)."""
        if len(rest) == 1:
            rc = run(plan_ref, x, w1, w2, hidden, out, ws, rest[0])
        else:
            b1, b2, stream = rest
            rc = run_ex(plan_ref, x, w1, b1, w2, b2, hidden, out, ws, stream)
        if rc:
            _lib.check(rc)

    provenance.update(down_impl=plan.selection.down_impl,
                      entry_point=KERNEL_ENTRIES[plan.selection.down_impl],
                      up_variant=native.up_variant, down_variant=native.down_variant)
    return artifact, provenance
