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

    @property
    def output_shape(self):
        return (*self.input_shape[:-1], self.n)


def _shape(value, name, ranks):
    result = tuple(value)
    if len(result) not in ranks:
        raise ValueError(f"{name}: unsupported rank {len(result)}")
    if any(type(d) is not int or d <= 0 for d in result):
        raise ValueError(f"{name}: dimensions must be positive integers")
    return result


def problem_from_shapes(x_shape, w1_shape, w2_shape, dtype="float16", layout="linear"):
    """Validate shapes (ops/host/inputs.py:38-53): X rank 2-8, W1 [H,K], W2 [N,H]."""
    x = _shape(x_shape, "x", range(2, 9))
    w1 = _shape(w1_shape, "weight1", (2,))
    w2 = _shape(w2_shape, "weight2", (2,))
    if dtype not in ("float16", "bfloat16"):
        raise ValueError("dtype must be float16 or bfloat16")
    if layout != "linear":
        raise ValueError("Only explicit layout='linear' is enabled in this implementation")
    h, k = w1
    n, h2 = w2
    if x[-1] != k or h != h2:
        raise ValueError("Expected x[..., K], weight1[H,K], weight2[N,H]")
    if max(k, h, n) > MAX_DIM or prod(x[:-1]) > MAX_ROWS:
        raise ValueError("Shape exceeds the supported bounds (K, H, N <= 65535; M <= 2**31-16)")
    return Problem(x, prod(x[:-1]), k, h, n, dtype, layout)


def validate_tensors(x, weight1, weight2, layout="linear", require_device=False, require_npu=None):
    """Tensor checks of ops/host/inputs.py:56-71; `require_device` asks for ROCm GPU tensors.

    require_npu is the reference's name of the same switch (ops/host/inputs.py:56), accepted
    so that its callers run unchanged; it asks for the device this build runs on."""
    import torch
    if require_npu is not None:
        require_device = bool(require_npu)

    tensors = (x, weight1, weight2)
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
    return problem_from_shapes(x.shape, weight1.shape, weight2.shape,
                               str(x.dtype).removeprefix("torch."), layout)


def _in_place(t, width):
    """A [rows, width] operand the kernels can read where it lies: contiguous rows of a
    multiple of 8 elements on a 16-byte boundary (whole 16-byte chunks per row)."""
    return t.is_contiguous() and width % 8 == 0 and t.data_ptr() % 16 == 0


def operands_aligned(x, weight1, weight2, plan):
    """True when X, W1 and W2 can all be used in place at the padded widths: contiguous, K,
    H and N already at their padded extents.  M needs no padding: the kernels never read
    rows of X past m."""
    p = plan.problem
    return (p.k == plan.kp and p.h == plan.hp and p.n == plan.np and x.is_contiguous()
            and weight1.is_contiguous() and weight2.is_contiguous())


def prepare_storage(x, weight1, weight2, plan, alias_aligned=False):
    """Contiguise and zero-pad into [mp,kp], [hp,kp], [np,hp]; allocate hidden, out, workspace.

    Same buffers as ops/host/inputs.py:74-90; the FP32 workspace holds the partial tiles of
    the Stream-K down and of a split up GEMM (every slot is written before it is read).
    Returns the six buffers and
    the operand layout (k, h, n, ldx, ldw1, ldw2) for ffn_mi355x_set_operands.

    With alias_aligned, every operand the kernels can read where it lies (_in_place) is
    the caller's tensor itself, at its logical width, and only the others are copied:
    for a launch that runs before the caller can modify them.  X needs K % 8 == 0, W1 the
    same, W2 H % 8 == 0; a non-contiguous operand (a transposed view) is always copied.
    """
    import torch

    p = plan.problem
    hidden = torch.empty((plan.mp, plan.hp), device=x.device, dtype=x.dtype)
    out = torch.empty((plan.mp, plan.np), device=x.device, dtype=x.dtype)
    ws = torch.empty(plan.workspace_shape, device=x.device, dtype=torch.float32)
    xv = x.reshape(p.m, p.k) if x.is_contiguous() else None
    if alias_aligned and xv is not None and _in_place(xv, p.k):
        xs, ldx = xv, p.k
    else:
        xs = torch.zeros((plan.mp, plan.kp), device=x.device, dtype=x.dtype)
        xs[:p.m, :p.k].copy_(x.reshape(p.m, p.k))
        ldx = plan.kp
    if alias_aligned and _in_place(weight1, p.k):
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
    return (xs, w1s, w2s, hidden, out, ws), layout


