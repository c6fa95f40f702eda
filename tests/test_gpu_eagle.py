"""GPU parity of the EagleFFN paths (bias, SiLU, SwiGLU, the Canonical layout) against the oracle.

The paths are those of the reference's analysis of the EagleFFN baseline
(spec/MindIE-SD EagleFFN算子实现分析.md:17-71): act(X W1^T + b1) W2^T + b2.  Random cases run
through eagle_ffn_linear / prepare_ffn under the reference criterion and the tripwires of the
GELU operator's tests; integer-valued cases pin the epilogues through the C ABI exactly.
"""
import ctypes

import pytest
import torch

from ffn_optim_amd import _lib, eagle_ffn_linear, prepare_eagle_ffn
from ffn_optim_amd.host.inputs import interleave_gate_up
from oracle.reference import compare, ffn_torch
from gpu_workspace import counters_are_zero, poisoned_workspace

pytestmark = pytest.mark.gpu

UNSTAGED_BOUND = {torch.float16: 2e-3, torch.bfloat16: 1.2e-2}
STAGED_BOUND = 1e-3


def say(*args):
    print("[gpu-eagle]", *args, flush=True)


def _inputs(shape, k, h, n, dtype, activation, bias, seed):
    g = torch.Generator().manual_seed(seed)
    u = 2 * h if activation == "swiglu" else h
    x = torch.randn((*shape, k), generator=g).to(dtype)
    w1 = (torch.randn(u, k, generator=g) * k ** -0.5).to(dtype)
    w2 = (torch.randn(n, h, generator=g) * h ** -0.5).to(dtype)
    b1 = (torch.randn(u, generator=g) * 0.5).to(dtype) if bias else None
    b2 = (torch.randn(n, generator=g) * 0.5).to(dtype) if bias else None
    return x, w1, w2, b1, b2


def _check(out, x, w1, w2, b1, b2, activation, tag):
    kw = dict(activation=activation, bias1=b1, bias2=b2)
    golden = ffn_torch(x, w1, w2, **kw)
    staged = ffn_torch(x, w1, w2, staged=True, **kw)
    res, res_staged = compare(out.cpu(), golden), compare(out.cpu(), staged)
    say(tag, "unstaged", res, "staged", res_staged)
    assert res["passed"], res
    assert res["mean_rel"] <= UNSTAGED_BOUND[x.dtype], res
    assert res_staged["mean_rel"] <= STAGED_BOUND, res_staged


@pytest.mark.parametrize("down", ["basic", "streamk"])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("activation", ["gelu", "silu", "swiglu"])
def test_eagle_paths_ragged(activation, bias, down):
    """Ragged M, K, H, N (padding on every dimension), fp16 and bf16."""
    for dtype, seed in ((torch.float16, 1), (torch.bfloat16, 2)):
        x, w1, w2, b1, b2 = _inputs((3, 97), 200, 320, 136, dtype, activation, bias, seed)
        dev = [t.cuda() if t is not None else None for t in (x, w1, w2, b1, b2)]
        try:
            out = eagle_ffn_linear(dev[0], dev[1], dev[2], dev[3], dev[4], activation=activation, down_impl=down)
        except ValueError as exc:   # Stream-K refused for this tile count
            assert down == "streamk", exc
            continue
        torch.cuda.synchronize()
        assert out.shape == (3, 97, 136) and out.dtype == dtype
        _check(out, x, w1, w2, b1, b2, activation, f"{activation} bias={bias} {down} {dtype}")


@pytest.mark.parametrize("down", ["basic", "streamk"])
@pytest.mark.parametrize("activation", ["silu", "swiglu"])
def test_eagle_paths_mid_size(activation, down):
    """A DiT-block-like size with biases: X [2, 1024, 1024] bf16, H 2048, N 1024."""
    x, w1, w2, b1, b2 = _inputs((2, 1024), 1024, 2048, 1024, torch.bfloat16, activation, True, 7)
    prepared = prepare_eagle_ffn(x.cuda(), w1.cuda(), w2.cuda(), b1.cuda(), b2.cuda(), activation=activation,
                                 down_impl=down)
    out = prepared.run()
    torch.cuda.synchronize()
    say("mid", activation, down, prepared.plan.up, prepared.plan.down)
    _check(out, x, w1, w2, b1, b2, activation, f"mid {activation} {down}")
    again = prepared.run().clone()
    torch.cuda.synchronize()
    assert torch.equal(again.view(torch.int16), out.view(torch.int16))


def test_canonical_layout_matches_linear():
    """Canonical weights (W1 [K,H], W2 [H,N]) are the same operator: bit-identical output."""
    x, w1, w2, b1, b2 = _inputs((64,), 256, 384, 192, torch.bfloat16, "silu", True, 5)
    xd, w1d, w2d, b1d, b2d = (t.cuda() for t in (x, w1, w2, b1, b2))
    lin = eagle_ffn_linear(xd, w1d, w2d, b1d, b2d, activation="silu").clone()
    can = eagle_ffn_linear(xd, w1d.t().contiguous(), w2d.t().contiguous(), b1d, b2d, activation="silu",
                           layout="canonical")
    torch.cuda.synchronize()
    assert torch.equal(lin.view(torch.int16), can.view(torch.int16))


def _ordinal(bits16):
    b = bits16.int() & 0xFFFF
    return torch.where(b >= 0x8000, -(b & 0x7FFF), b)


def _int_tensor(shape, gen, lo=-2, hi=2):
    return torch.randint(lo, hi + 1, shape, generator=gen).float()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("activation", ["silu", "swiglu"])
def test_up_integer_activation_all_variants(dtype, activation):
    """With integer X, W1 and bias1, z + b1 is exact, so hidden must be the activation of it
    rounded once: within one unit in the last place of the float64 SiLU (SwiGLU: of the float64
    SiLU(gate) * up), for every tile variant that the activation can use."""
    lib = _lib.load()
    gen = torch.Generator().manual_seed(3)
    mp, kp, hp = 320, 80, 448
    u = 2 * hp if activation == "swiglu" else hp
    x = _int_tensor((mp, kp), gen).to(dtype)
    w1 = _int_tensor((u, kp), gen).to(dtype)
    b1 = _int_tensor((u,), gen).to(dtype)
    z64 = x.double() @ w1.double().T + b1.double()
    silu64 = lambda z: z / (1 + torch.exp(-z))
    truth = (silu64(z64) if activation == "silu" else silu64(z64[:, :hp]) * z64[:, hp:]).to(dtype)
    w1k = interleave_gate_up(w1, hp, hp) if activation == "swiglu" else w1
    b1k = interleave_gate_up(b1, hp, hp) if activation == "swiglu" else b1
    xd, w1d, b1d = x.cuda(), w1k.contiguous().cuda(), b1k.contiguous().cuda()
    stream = torch.cuda.current_stream().cuda_stream
    code = _lib.BF16 if dtype == torch.bfloat16 else _lib.FP16
    tested = 0
    for variant in range(lib.ffn_mi355x_num_variants()):
        try:
            plan = _lib.make_plan(mp, kp, hp, 64, code, "basic", "erf", 256, variant, -1, activation=activation)
        except ValueError:
            assert activation == "swiglu"   # a tile without whole 64-column block pairs
            continue
        hidden = torch.full((mp, hp), float("nan"), dtype=dtype, device="cuda")
        ws = poisoned_workspace(plan)
        _lib.check(lib.ffn_mi355x_up_ex(ctypes.byref(plan), xd.data_ptr(), w1d.data_ptr(), b1d.data_ptr(),
                                        hidden.data_ptr(), ws.data_ptr(), stream))
        torch.cuda.synchronize()
        assert counters_are_zero(plan, ws), (activation, variant)
        ulps = (_ordinal(hidden.cpu().view(torch.int16)) - _ordinal(truth.view(torch.int16))).abs()
        say("up-act", activation, dtype, variant, plan.up_sk_tiles, int(ulps.max()), int((ulps > 0).sum()))
        assert int(ulps.max()) <= 1, (activation, variant)
        tested += 1
    assert tested >= 8


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_down_integer_bias_bit_exact(dtype):
    """Integer hidden, W2 and bias2: out = hidden W2^T + b2 is exact in FP32 and rounded once, for
    Basic and Stream-K on every variant (the bias enters the register, staged-store and split-tile
    finish epilogues alike)."""
    lib = _lib.load()
    gen = torch.Generator().manual_seed(13)
    mp, hp, np_ = 320, 1024, 448
    hid = _int_tensor((mp, hp), gen).to(dtype)
    w2 = _int_tensor((np_, hp), gen).to(dtype)
    b2 = _int_tensor((np_,), gen, -8, 8).to(dtype)
    golden = (hid.double() @ w2.double().T + b2.double()).float().to(dtype)
    hid_d, w2_d, b2_d = hid.cuda(), w2.cuda(), b2.cuda()
    stream = torch.cuda.current_stream().cuda_stream
    code = _lib.BF16 if dtype == torch.bfloat16 else _lib.FP16
    for variant in range(lib.ffn_mi355x_num_variants()):
        for down, block_num in (("basic", 256), ("streamk", 256), ("streamk", 37)):
            try:
                plan = _lib.make_plan(mp, 64, hp, np_, code, down, "erf", block_num, 0, variant)
            except ValueError:
                continue
            out = torch.full((mp, np_), float("nan"), dtype=dtype, device="cuda")
            ws = poisoned_workspace(plan)
            _lib.check(lib.ffn_mi355x_down_ex(ctypes.byref(plan), hid_d.data_ptr(), w2_d.data_ptr(),
                                              b2_d.data_ptr(), out.data_ptr(), ws.data_ptr(), stream))
            torch.cuda.synchronize()
            assert counters_are_zero(plan, ws), (variant, down, block_num)
            say("down-bias", dtype, variant, down, block_num)
            assert torch.equal(out.cpu().view(torch.int16), golden.view(torch.int16)), (variant, down, block_num)


@pytest.mark.parametrize("activation", ["gelu", "silu", "swiglu"])
def test_eagle_permuted_x_read_in_place(activation):
    """eagle_ffn_linear on a permuted X (a [97, 3, 200] view of a [3, 97, 200] tensor) reads its
    rows in place through the row grid, biases and every activation included: bit-identical to
    the same call on a contiguous copy of X, and within the criterion of the golden."""
    from ffn_optim_amd.host.inputs import row_grid
    x, w1, w2, b1, b2 = _inputs((3, 97), 200, 320, 136, torch.bfloat16, activation, True, 7)
    dev = [t.cuda() for t in (x, w1, w2, b1, b2)]
    xt = dev[0].transpose(0, 1)
    assert row_grid(xt, 200)[0] == "grid"
    out = eagle_ffn_linear(xt, *dev[1:], activation=activation)
    ref = eagle_ffn_linear(xt.contiguous(), *dev[1:], activation=activation)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), activation
    _check(out, x.transpose(0, 1), w1, w2, b1, b2, activation, f"{activation} permuted X")
