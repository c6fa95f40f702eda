"""Workspace helpers of the GPU tests: a workspace whose partial slots hold NaN (so a slot read
before it is written shows in the result) and whose leading arrival counters are zero, as the
library requires before a workspace's first use."""
import torch

from ffn_optim_amd import _lib


def poisoned_workspace(plan):
    ws = torch.full((max(1, plan.workspace_bytes // 4),), float("nan"), dtype=torch.float32, device="cuda")
    ws[: _lib.workspace_counter_bytes(plan) // 4] = 0.0
    return ws


def counters_are_zero(plan, ws):
    """Every launch leaves the counters zero for the next one."""
    n = _lib.workspace_counter_bytes(plan) // 4
    return not bool(ws[:n].view(torch.int32).any())
