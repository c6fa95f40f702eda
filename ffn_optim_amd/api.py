"""Drop-in FFN API: ``ffn``, ``prepare_ffn``, ``PreparedFFN.run`` (restates ops/api.py).

    Y = GELU(X @ weight1.T) @ weight2.T       no bias, no autograd

X is 2-8-D [..., K], weight1 [H, K], weight2 [N, H], all float16 or bfloat16 on
one ROCm GPU (gfx950).  Inputs are contiguised and zero-padded on entry (M/H/N to
64, K to 16), the output is cropped and the leading dims restored.  Differences
from the reference, by design of the target:
  * block_num is the number of persistent workgroups (<= the device CU count);
    its default None means "every CU" instead of the reference's 8 AI cores.
  * gelu='erf' (exact GELU, the reference's golden) or 'rational' (the
    reference's P5/Q5 kernel approximation) selects the up-projection epilogue.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from time import perf_counter

from .host.dispatch import Selection, verify_dependency
from .host.inputs import prepare_storage, validate_tensors
from .host.tiling import make_plan


class KernelCompilationError(RuntimeError):
    """Binding the prebuilt kernels to a plan failed (ops/api.py:9-14): the library lacks a
    launch entry point or a tile variant the plan needs.

    Raised before any FFN launch and before the input copies.  The original exception is
    chained.  (A library that is missing, unloadable or lacks a planning entry point is
    reported earlier, as DependencyUnavailable.)
    """


@dataclass
class PreparedFFN:
    """Prepared inputs, buffers and bound kernels; run() may be called repeatedly.

    storage is (X[mp,kp], W1[hp,kp], W2[np,hp], hidden[mp,hp], out[mp,np], ws) on
    one device (for ffn(), operands read in place keep their own shapes); tensors
    holds their device addresses; provenance and preparation record the library and
    the preparation timings; stream is the preparation stream (ops/api.py:17-35).
    """

    plan: object
    storage: tuple
    tensors: tuple
    artifact: object
    provenance: dict
    preparation: dict
    stream: object
    _output: object = field(default=None, init=False, repr=False)

    def run(self):
        """One FFN launch sequence; the returned view is overwritten by the next run().

        Must be called on the preparation stream; returns without synchronising
        (ops/api.py:37-45).  The host work per call is one stream check and one C call:
        the plan and buffers were validated at preparation, and the output view is
        built once (the same [:m, :n] view of the out buffer every call).
        """
        import torch
        device = self.stream.device_index
        if torch.cuda.current_device() != device:
            with torch.cuda.device(device):
                return self.run()
        if _current_stream_handle(device) != self.stream.cuda_stream:
            raise RuntimeError(
                "PreparedFFN must run on its preparation stream; concurrent reuse is unsupported")
        self.artifact(*self.tensors, self.stream.cuda_stream)
        if self._output is None:
            p = self.plan.problem
            self._output = self.storage[4][:p.m, :p.n].view(p.output_shape)
        return self._output


def _current_stream_handle(device):
    """Raw handle of torch's current stream on `device` (the cheap form of
    torch.cuda.current_stream(device).cuda_stream)."""
    import torch
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    return raw(device) if raw is not None else torch.cuda.current_stream(device).cuda_stream


def prepare_ffn(x, weight1, weight2, *, up_impl="basic", down_impl="basic", block_num=None,
                layout="linear", gelu="erf", up_variant=None, down_variant=None, activation="gelu",
                bias1=None, bias2=None, single_launch=None, _alias=False):
    """Validate, plan, check the device, pad/contiguise and bind the kernels; no FFN launch.

    Follows ops/api.py:48-89.  Padding and contiguisation are auxiliary device
    operations timed outside the FFN.  up_variant/down_variant force a compiled
    tile variant (tuning); None lets the library choose.  The prepared storage is a
    snapshot of the inputs (later changes to x, weight1, weight2 do not reach run());
    ffn() alone, which runs at once, may use aligned inputs in place (_alias).

    activation 'silu' or 'swiglu' (weight1 [2H, K]: gate rows, then up rows) and the
    biases bias1 ([H] or [2H]) and bias2 ([N]), given together, select the other EagleFFN
    paths, Y = act(X W1^T + b1) W2^T + b2 (spec/MindIE-SD EagleFFN算子实现分析.md:17-71); the
    defaults are the reference's operator.  storage then ends with the two bias buffers.

    single_launch: True runs the FFN as one launch (NotApplicable where no single-launch kernel
    is compiled for the plan's tile pair); None and False keep the two launches, which measured
    faster on every workload the single launch serves.
    """
    from .host.dispatch import compile_kernel
    from . import _lib

    p = validate_tensors(x, weight1, weight2, layout=layout, require_device=True,
                         activation=activation, bias1=bias1, bias2=bias2)
    selection = Selection(up_impl, down_impl)
    selection.require_available()
    import torch
    verify_dependency()
    device = x.device.index if x.device.index is not None else torch.cuda.current_device()
    cu_count, _arch = _lib.query(device)
    if block_num is None:
        block_num = cu_count
    plan = make_plan(p, selection, block_num, gelu=gelu, up_variant=up_variant,
                     down_variant=down_variant)
    if block_num > cu_count:
        raise ValueError(f"block_num must not exceed the device CU count ({cu_count})")
    if single_launch is not None:
        _lib.set_single_launch(plan.native, bool(single_launch))
    # Binding needs the plan only, so it runs before any device work: a library that cannot
    # launch this plan fails here, ahead of the input copies.
    before = perf_counter()
    try:
        artifact, provenance = compile_kernel(plan)
    except Exception as exc:
        raise KernelCompilationError(f"{type(exc).__name__}: {exc}") from exc
    compile_ms = (perf_counter() - before) * 1000
    with torch.cuda.device(x.device):
        stream = torch.cuda.current_stream()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        storage, layout, x_rows = prepare_storage(x, weight1, weight2, plan, alias_aligned=_alias,
                                                  bias1=bias1, bias2=bias2)
        end.record()
        _lib.set_operands(plan.native, *layout)
        if x_rows is not None:
            _lib.set_x_rows(plan.native, *x_rows)
        end.synchronize()
        auxiliary_ms = start.elapsed_time(end)
        tensors = tuple(t.data_ptr() for t in storage)
        preparation = {"auxiliary_device_interval_ms": auxiliary_ms,
                       "compile_wall_ms": compile_ms}
    return PreparedFFN(plan, storage, tensors, artifact, provenance, preparation, stream)


def ffn(x, weight1, weight2, **configuration):
    """Y = GELU(X @ weight1.T) @ weight2.T; no bias, no autograd (ops/api.py:92-94).

    Operands the kernels can read where they lie (contiguous, rows a multiple of 8
    elements: K for X and weight1, H for weight2) are used in place for this single
    launch instead of being copied into padded buffers; the result is identical (the
    kernels zero-fill past the logical widths and mask ragged tiles).
    """
    return prepare_ffn(x, weight1, weight2, **configuration, _alias=True).run()
