"""Input contract shared by the oracle checks, planning and device execution.

Restates ops/host/inputs.py of the reference: the same shape/dtype rules
(`problem_from_shapes`, ops/host/inputs.py:38-53), tensor checks
(`validate_tensors`, :56-71) and contiguise + zero-pad storage
(`prepare_storage`, :74-90).  The device check asks for a ROCm GPU tensor
(torch's ``cuda`` device type on ROCm) instead of an Ascend NPU tensor.
"""
from __future__ import annotations

from dataclasses import dataclass
from math import prod

MAX_DIM = 65535
MAX_ROWS = 2 ** 31 - 16


@dataclass(frozen=True)
class Problem:
    """Logical FFN shape and type (ops/host/inputs.py:6-26).

    input_shape is the 2-8-D shape of X, m the product of its leading dims, k its
    last dim; h and n are the hidden and output widths.  Built by
    problem_from_shapes, which validates; direct construction does not.
    """

    input_shape: tuple[int, ...]
    m: int
    k: int
    h: int
    n: int
    dtype: str
    layout: str
    activation: str = "gelu"   # gelu (the reference's operator), silu or swiglu

    @property
    def output_shape(self):
        return (*self.input_shape[:-1], self.n)

    @property
    def up_width(self):
        """Rows of weight1: H, or 2H for SwiGLU (gate rows, then up rows)."""
        return 2 * self.h if self.activation == "swiglu" else self.h


def _shape(value, name, ranks):
    result = tuple(value)
    if len(result) not in ranks:
        raise ValueError(f"{name}: unsupported rank {len(result)}")
    if any(type(d) is not int or d <= 0 for d in result):
        raise ValueError(f"{name}: dimensions must be positive integers")
    return result


ACTIVATIONS = ("gelu", "silu", "swiglu")


def problem_from_shapes(x_shape, w1_shape, w2_shape, dtype="float16", layout="linear", activation="gelu"):
    """Validate shapes (ops/host/inputs.py:38-53): X rank 2-8, W1 [H,K], W2 [N,H].

    activation 'silu' keeps these shapes; 'swiglu' takes W1 [2H,K], gate rows then up rows
    (the EagleFFN paths, spec/MindIE-SD EagleFFN算子实现分析.md:17-71, :76-86)."""
    x = _shape(x_shape, "x", range(2, 9))
    w1 = _shape(w1_shape, "weight1", (2,))
    w2 = _shape(w2_shape, "weight2", (2,))
    if dtype not in ("float16", "bfloat16"):
        raise ValueError("dtype must be float16 or bfloat16")
    if layout != "linear":
        raise ValueError("Only explicit layout='linear' is enabled in this implementation")
    if activation not in ACTIVATIONS:
        raise ValueError(f"activation must be one of {ACTIVATIONS}")
    u, k = w1
    n, h = w2
    if x[-1] != k or u != (2 * h if activation == "swiglu" else h):
        raise ValueError("Expected x[..., K], weight1[2H,K], weight2[N,H]" if activation == "swiglu"
                         else "Expected x[..., K], weight1[H,K], weight2[N,H]")
    if max(k, h, n) > MAX_DIM or prod(x[:-1]) > MAX_ROWS:
        raise ValueError("Shape exceeds the supported bounds (K, H, N <= 65535; M <= 2**31-16)")
    return Problem(x, prod(x[:-1]), k, h, n, dtype, layout, activation)


def validate_tensors(x, weight1, weight2, layout="linear", require_device=False, require_npu=None,
                     activation="gelu", bias1=None, bias2=None):
    """Tensor checks of ops/host/inputs.py:56-71; `require_device` asks for ROCm GPU tensors.

    require_npu is the reference's name of the same switch (ops/host/inputs.py:56), accepted
    so that its callers run unchanged; it asks for the device the library runs on.  bias1
    ([H], or [2H] for SwiGLU) and bias2 ([N]) are given together or not at all, like the
    operands (same dtype and device, dense, no grad)."""
    import torch
    if require_npu is not None:
        require_device = bool(require_npu)
    if (bias1 is None) != (bias2 is None):
        raise ValueError("bias1 and bias2 must be given together or not at all")

    tensors = (x, weight1, weight2) + (() if bias1 is None else (bias1, bias2))
    if any(not isinstance(t, torch.Tensor) for t in tensors):
        raise TypeError("x, weight1 and weight2 must be torch.Tensor")
    if any(t.dtype != x.dtype or t.device != x.device for t in tensors):
        raise ValueError("All tensors must have the same dtype and device")
    if any(t.layout != torch.strided for t in tensors):
        raise ValueError("Only dense strided tensors are supported")
    if any(t.requires_grad for t in tensors):
        raise ValueError("Inference-only operator; detach inputs explicitly")
    if require_device and x.device.type != "cuda":
        raise ValueError("FFN execution requires ROCm GPU tensors; no torch fallback is used")
    p = problem_from_shapes(x.shape, weight1.shape, weight2.shape,
                            str(x.dtype).removeprefix("torch."), layout, activation)
    if bias1 is not None and (tuple(bias1.shape) != (p.up_width,) or tuple(bias2.shape) != (p.n,)):
        raise ValueError(f"Expected bias1[{p.up_width}] and bias2[{p.n}]")
    return p


def _in_place(t, width):
    """A [rows, width] operand the kernels can read where it lies: contiguous rows of a
    multiple of 8 elements on a 16-byte boundary (whole 16-byte chunks per row)."""
    return t.is_contiguous() and width % 8 == 0 and t.data_ptr() % 16 == 0


# Gathered rows are addressed with 32-bit byte offsets below 2^31 (ffn_mi355x_set_x_rows).
MAX_GATHER_SPAN = 2 ** 31


def row_grid(x, k):
    """How the up GEMM can read X [..., k] where it lies, as rows of k contiguous elements.

    Leading dims of size 1 are dropped and neighbours whose strides chain (outer stride =
    inner size * inner stride) are merged.  Returns ("pitch", ldx) when one dim is left (a
    contiguous X or one sliced from wider rows: rows at one pitch), ("grid", (d1, d2, s0, s1,
    s2)) when two or three are left (a permuted view such as a [B, S, K] tensor read as
    [S, B, K]: row (i0, i1, i2) of a [m / (d1*d2), d1, d2] grid starts at i0*s0 + i1*s1 + i2*s2),
    or None when the view must be copied: K not contiguous or not a multiple of 8, a stride or
    the base off a 16-byte boundary, more than three dims left, rows spread over 2^31 bytes
    or more, or a single pitch above the library's largest (_lib.MAX_PITCH).  No counterpart
    in the reference, which copies every X (ops/host/inputs.py:74-90).
    """
    from .._lib import MAX_PITCH
    if k % 8 != 0 or x.stride(-1) != 1 or (x.data_ptr() % 16) != 0:
        return None
    dims = [(n, st) for n, st in zip(x.shape[:-1], x.stride()[:-1]) if n != 1]
    merged = []
    for n, st in reversed(dims):
        if merged and st == merged[-1][0] * merged[-1][1]:
            merged[-1] = (n * merged[-1][0], merged[-1][1])
        else:
            merged.append((n, st))
    merged.reverse()
    if any(st % 8 != 0 for _, st in merged) or len(merged) > 3:
        return None
    if not merged:
        return ("pitch", k)
    span = (sum((n - 1) * st for n, st in merged) + k) * x.element_size()
    if span > MAX_GATHER_SPAN:
        return None
    if len(merged) == 1 and merged[0][1] >= k:
        return ("pitch", merged[0][1]) if merged[0][1] <= MAX_PITCH else None
    merged = [(1, 0)] * (3 - len(merged)) + merged
    (_, s0), (d1, s1), (d2, s2) = merged
    return ("grid", (d1, d2, s0, s1, s2))


def operands_aligned(x, weight1, weight2, plan):
    """True when X, W1 and W2 can all be used in place at the padded widths: contiguous, K,
    H and N already at their padded extents.  M needs no padding: the kernels never read
    rows of X past m."""
    p = plan.problem
    return (p.k == plan.kp and p.h == plan.hp and p.n == plan.np and x.is_contiguous()
            and weight1.is_contiguous() and weight2.is_contiguous())


def interleave_gate_up(weight, h, hp):
    """SwiGLU weight1 [2h, K] (gate rows, then up rows) or bias1 [2h] -> the [2hp, ...] layout the
    up GEMM reads: 32-row blocks alternate, block 2b holding gate rows 32b..32b+31 and block 2b+1
    the up rows of the same hidden columns; zero past h."""
    import torch
    tail = tuple(weight.shape[1:])
    out = torch.zeros((hp // 32, 2, 32) + tail, device=weight.device, dtype=weight.dtype)
    flat = out.view((hp // 32, 2 * 32) + tail)
    gate = torch.zeros((hp,) + tail, device=weight.device, dtype=weight.dtype)
    up = torch.zeros_like(gate)
    gate[:h].copy_(weight[:h])
    up[:h].copy_(weight[h:2 * h])
    out[:, 0].copy_(gate.view((hp // 32, 32) + tail))
    out[:, 1].copy_(up.view((hp // 32, 32) + tail))
    return flat.reshape((2 * hp,) + tail)


def prepare_storage(x, weight1, weight2, plan, alias_aligned=False, bias1=None, bias2=None):
    """Contiguise and zero-pad into [mp,kp], [hp,kp], [np,hp]; allocate hidden, out, workspace.

    Same buffers as ops/host/inputs.py:74-90; the FP32 workspace holds the arrival counters and
    partial tiles of the Stream-K down and of a split up GEMM (allocated zero-filled; every
    partial slot is written before it is read).
    Returns the six buffers, the operand layout (k, h, n, ldx, ldw1, ldw2) for
    ffn_mi355x_set_operands and X's row grid (d1, d2, s0, s1, s2) for ffn_mi355x_set_x_rows,
    or None when X is read as rows at pitch ldx.

    With alias_aligned, every operand the kernels can read where it lies is the caller's
    tensor itself, at its logical width, and only the others are copied: for a launch that
    runs before the caller can modify them.  X needs K % 8 == 0 and K contiguous, and is read
    in place even as a permuted or sliced view (row_grid); W1 needs K % 8 == 0 and W2
    H % 8 == 0, both contiguous (a transposed weight is copied).  X read in place is kept as
    an [m, k] view at pitch ldx, or as the caller's tensor itself when its rows form a grid.
    """
    import torch

    p = plan.problem
    hidden = torch.empty((plan.mp, plan.hp), device=x.device, dtype=x.dtype)
    out = torch.empty((plan.mp, plan.np), device=x.device, dtype=x.dtype)
    # zero-filled: its leading bytes are the split tiles' arrival counters, which every launch
    # leaves zero again
    ws = torch.zeros(plan.workspace_shape, device=x.device, dtype=torch.float32)
    grid = row_grid(x, p.k) if alias_aligned else None
    x_rows = None
    if grid is not None and grid[0] == "pitch":
        ldx = grid[1]
        xs = x.as_strided((p.m, p.k), (ldx, 1))
    elif grid is not None:
        xs, ldx, x_rows = x, p.k, grid[1]
    else:
        xs = torch.zeros((plan.mp, plan.kp), device=x.device, dtype=x.dtype)
        xs[:p.m, :p.k].copy_(x.reshape(p.m, p.k))
        ldx = plan.kp
    if p.activation == "swiglu":
        # always a copy: the gate and up rows are interleaved for the up GEMM
        wk = torch.zeros((2 * p.h, plan.kp), device=x.device, dtype=x.dtype)
        wk[:, :p.k].copy_(weight1)
        w1s, ldw1 = interleave_gate_up(wk, p.h, plan.hp), plan.kp
    elif alias_aligned and _in_place(weight1, p.k):
        w1s, ldw1 = weight1, p.k
    else:
        w1s = torch.zeros((plan.hp, plan.kp), device=x.device, dtype=x.dtype)
        w1s[:p.h, :p.k].copy_(weight1)
        ldw1 = plan.kp
    if alias_aligned and _in_place(weight2, p.h):
        w2s, ldw2 = weight2, p.h
    else:
        w2s = torch.zeros((plan.np, plan.hp), device=x.device, dtype=x.dtype)
        w2s[:p.n, :p.h].copy_(weight2)
        ldw2 = plan.hp
    # the reduction runs to the logical K when both up operands hold whole chunks up to it
    k = p.k if p.k % 8 == 0 else plan.kp
    layout = (k, p.h, p.n, ldx, ldw1, ldw2)
    storage = (xs, w1s, w2s, hidden, out, ws)
    if bias1 is not None:
        # copies: 16-byte aligned; SwiGLU's bias1 interleaved like its weight rows
        b1s = (interleave_gate_up(bias1, p.h, plan.hp) if p.activation == "swiglu"
               else bias1.detach().clone().contiguous())
        storage += (b1s, bias2.detach().clone().contiguous())
    return storage, layout, x_rows


