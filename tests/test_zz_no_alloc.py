"""ffn_mi355x_run_noalloc: the entry point that allocates nothing, against ffn_mi355x_run.

Both run the same kernels in the same order, so the outputs must agree bit for bit.  The
no-allocation entry point keeps its partial tiles in the library's own device scratch, which
every call on the GPU shares: three calls in a row, each smaller than the one before, must
each match ffn_mi355x_run on a workspace of its own (a stale partial of the previous call
would show).  The calls cover the Stream-K down (partials) and a split up GEMM (partials, the
GELU applied by the last piece of each tile); a call that left the scratch's arrival counters
nonzero would break the next.
"""
import ctypes

import pytest
import torch

from ffn_optim_amd import _lib, prepare_ffn
from ffn_optim_amd.cases import get_case, make_inputs

pytestmark = pytest.mark.gpu

# (case, down path), inputs from largest to smallest
SEQUENCE = (("c4_decode_bf16", "streamk"), ("c4_tp8_shard_bf16", "streamk"), ("c1_smoke_fp16", "streamk"),
            ("c1_smoke_fp16", "basic"))


def _bits(t):
    return t.contiguous().view(torch.int16).cpu()


def test_noalloc_matches_run_call_after_call():
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    sizes, inputs = [], []
    for case_id, down in SEQUENCE:
        x, w1, w2 = make_inputs(get_case(case_id), "cuda")
        prepared = prepare_ffn(x, w1, w2, down_impl=down)
        plan = prepared.plan.native
        xs, w1s, w2s, hid, out, ws = prepared.tensors
        expected = prepared.run().clone()          # ffn_mi355x_run, torch-allocated workspace
        torch.cuda.synchronize()
        prepared.storage[3].fill_(float("nan"))    # hidden and out poisoned between the two
        prepared.storage[4].fill_(float("nan"))
        torch.cuda.synchronize()
        print(f"[no-alloc] {case_id} {down} workspace={plan.workspace_bytes} "
              f"up_sk_tiles={plan.up_sk_tiles} down_sk_tiles={plan.down_sk_tiles}", flush=True)
        rc = lib.ffn_mi355x_run_noalloc(ctypes.byref(plan), xs, w1s, w2s, hid, out, stream)
        assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
        got = prepared.storage[4][:prepared.plan.problem.m, :prepared.plan.problem.n]
        assert torch.equal(_bits(got.reshape(expected.shape)), _bits(expected)), (case_id, down)
        sizes.append(plan.workspace_bytes)
        inputs.append(x.numel() + w1.numel() + w2.numel())
    # each call's input no larger than the one before; scratch use never grows
    assert inputs[0] > inputs[1] > inputs[2] == inputs[3]
    assert sizes[0] >= sizes[1] > sizes[2] > sizes[3] == 0 and sizes[0] <= 32 << 20


def test_noalloc_refuses_a_plan_beyond_its_scratch():
    """The DiT-size Stream-K plan needs 128 MiB of partials: refused, nothing launched."""
    lib = _lib.load()
    plan = _lib.make_plan(8192, 3072, 12288, 3072, _lib.BF16, "streamk", "erf", 256, 12, 6)
    assert plan.workspace_bytes > 32 << 20
    fake = [ctypes.c_void_p(4096 * (i + 1)) for i in range(5)]
    rc = lib.ffn_mi355x_run_noalloc(ctypes.byref(plan), *fake, None)
    assert rc == _lib.EINVAL and "scratch" in _lib.last_error()
