"""Padding, tile choice and Stream-K applicability (restates ops/host/tiling.py).

Padding units are the reference's (M/H/N to 64, K to 16, tiling.py:63-64).  The
tile geometry and the Stream-K schedule are decided by the native library
(``ffn_mi355x_make_plan``) so that the C ABI plans exactly as this host does;
this module mirrors its result into the reference's Plan/Tile shape.
"""
from __future__ import annotations

from dataclasses import asdict, dataclass

from .dispatch import Selection
from .inputs import Problem

MI355X_CU_COUNT = 256
DEFAULT_BLOCK_NUM = MI355X_CU_COUNT


def align(value, unit):
    return (value + unit - 1) // unit * unit


@dataclass(frozen=True)
class Tile:
    """Macro tile of one GEMM (elements): bm x bn output, bk deep per LDS stage.

    waves is the number of 64-lane wavefronts per workgroup, stages the number of
    LDS buffers, variant the id of the compiled kernel variant.
    """

    bm: int
    bn: int
    bk: int
    waves: int
    stages: int
    variant: int

    # The reference's names for the LDS-staged macro tile (its L1 tile, ops/host/tiling.py:11-25).
    # Its L0 tile (the cube unit's operand buffers) has no counterpart: a wave feeds the MFMA
    # from registers, 32x32 outputs and 16 of K per instruction.
    @property
    def l1_tm(self):
        return self.bm

    @property
    def l1_tn(self):
        return self.bn

    @property
    def l1_tk(self):
        return self.bk


@dataclass(frozen=True)
class Plan:
    """Everything one FFN launch sequence needs (reference Plan, tiling.py:28-55).

    block_num is the persistent-workgroup count of both launches; mp/kp/hp/np are
    the padded extents; workspace_shape is the FP32 scratch of the Stream-K down and of
    a split up GEMM ((1, 1) and unused when neither splits).  native is the C plan handed
    to the library.

    workspace_shape keeps the reference's form, FP32 rows of 64 (ops/host/tiling.py:71),
    with a row count of its own: the reference holds two 64x64 partial tiles per core,
    (128 * block_num, 64); here a slot is one macro tile of the chosen variant (up to
    256x256) and a workgroup holds as many slots as its split range touches tiles, so the
    shape is (workspace_bytes / 256, 64).
    """

    problem: Problem
    selection: Selection
    block_num: int
    mp: int
    kp: int
    hp: int
    np: int
    up: Tile
    down: Tile
    workspace_shape: tuple[int, int]
    gelu: str = "erf"
    native: object = None

    @property
    def activation(self):
        """gelu (with the `gelu` form), silu or swiglu: the problem's activation."""
        return self.problem.activation

    @property
    def workspace_bytes(self):
        return self.workspace_shape[0] * self.workspace_shape[1] * 4

    def schedule(self):
        """Launch shapes, the down GEMM's Stream-K split and the up GEMM's K split (from the
        native plan)."""
        n = self.native
        return {"up_tiles": n.up_tiles, "up_grid": n.up_grid, "up_k_iters": n.up_k_iters,
                "up_sk_tiles": n.up_sk_tiles, "up_slots_per_wg": n.up_slots_per_wg,
                "down_tiles": n.down_tiles, "down_grid": n.down_grid, "down_k_iters": n.down_k_iters,
                "down_dp_tiles": n.down_dp_tiles, "down_sk_tiles": n.down_sk_tiles,
                "down_slots_per_wg": n.down_slots_per_wg}

    def to_dict(self):
        d = {k: v for k, v in asdict(self).items() if k != "native"}
        d["schedule"] = self.schedule() if self.native is not None else None
        return d


def _tile(bm, bn, bk, variant):
    from .. import _lib
    info = _lib.variants()[variant]
    return Tile(bm, bn, bk, info["waves"], info["stages"], variant)


def make_plan(problem, selection=Selection(), block_num=DEFAULT_BLOCK_NUM, *, gelu="erf",
              up_variant=None, down_variant=None, tuned=True):
    """Plan one FFN (ops/host/tiling.py:58-74).

    Raises DependencyUnavailable for full_load_*, ValueError for a block_num outside
    [1, 65535], NotApplicable when Stream-K has no remainder tiles for this
    block_num or H spans fewer than two K iterations.  With neither variant forced
    and tuned=True, a measured choice from the tuning table (ffn_optim_amd.tuning)
    replaces the library planner's for the shapes it covers.
    """
    from .. import _lib
    from .dispatch import GELU_FORMS

    selection.require_available()
    if type(block_num) is not int or not 1 <= block_num <= 65535:
        raise ValueError("block_num must be a positive integer; hardware limit checked before launch")
    if gelu not in GELU_FORMS:
        raise ValueError(f"gelu must be one of {GELU_FORMS}")
    mp, kp = align(problem.m, 64), align(problem.k, 16)
    hp, np_ = align(problem.h, 64), align(problem.n, 64)
    dtype = _lib.BF16 if problem.dtype == "bfloat16" else _lib.FP16
    activation = getattr(problem, "activation", "gelu")
    if tuned and up_variant is None and down_variant is None:
        from .. import tuning
        # the key's epilogue field: the GELU form, or the other activation's name
        epilogue = gelu if activation == "gelu" else activation
        hit = tuning.lookup(tuning.make_key(problem.m, mp, kp, hp, np_, problem.dtype,
                                            selection.down_impl, epilogue, block_num))
        if hit is not None:
            up_variant, down_variant = hit
    native = _lib.make_plan(mp, kp, hp, np_, dtype, selection.down_impl, gelu, block_num,
                            -1 if up_variant is None else up_variant,
                            -1 if down_variant is None else down_variant, m=problem.m,
                            activation=activation)
    up = _tile(native.up_bm, native.up_bn, native.up_bk, native.up_variant)
    down = _tile(native.down_bm, native.down_bn, native.down_bk, native.down_variant)
    if native.workspace_bytes:   # Stream-K down and/or split up GEMM
        workspace = (native.workspace_bytes // 256, 64)
    else:
        workspace = (1, 1)  # unused argument: Basic down, one workgroup per up tile
    return Plan(problem, selection, block_num, mp, kp, hp, np_, up, down, workspace, gelu, native)
