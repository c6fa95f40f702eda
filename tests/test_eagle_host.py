"""Host side of the EagleFFN paths (CPU): shapes, biases, the SwiGLU row interleave, the
Canonical layout and the plans (spec/MindIE-SD EagleFFN算子实现分析.md:17-94)."""
import ctypes

import pytest
import torch

from ffn_optim_amd import _lib, eagle_ffn_linear, prepare_eagle_ffn
from ffn_optim_amd.host.dispatch import Selection
from ffn_optim_amd.host.inputs import interleave_gate_up, problem_from_shapes, validate_tensors
from ffn_optim_amd.host.tiling import make_plan


def test_swiglu_shapes():
    p = problem_from_shapes((4, 96), (2 * 160, 96), (48, 160), "bfloat16", activation="swiglu")
    assert (p.k, p.h, p.n, p.up_width, p.activation) == (96, 160, 48, 320, "swiglu")
    with pytest.raises(ValueError, match="weight1\\[2H,K\\]"):
        problem_from_shapes((4, 96), (160, 96), (48, 160), "bfloat16", activation="swiglu")
    with pytest.raises(ValueError):
        problem_from_shapes((4, 96), (320, 96), (48, 160), "bfloat16", activation="gelu")
    with pytest.raises(ValueError, match="activation"):
        problem_from_shapes((4, 96), (160, 96), (48, 160), "bfloat16", activation="relu")
    # the reference's contract is unchanged: canonical is refused by the shape check itself
    with pytest.raises(ValueError):
        problem_from_shapes([2, 3], [4, 3], [3, 4], layout="canonical")


def test_biases_together_and_shaped():
    x, w1, w2 = torch.zeros(2, 8).half(), torch.zeros(16, 8).half(), torch.zeros(4, 16).half()
    b1, b2 = torch.zeros(16).half(), torch.zeros(4).half()
    assert validate_tensors(x, w1, w2, bias1=b1, bias2=b2).h == 16
    with pytest.raises(ValueError, match="together"):
        validate_tensors(x, w1, w2, bias1=b1)
    with pytest.raises(ValueError, match="bias1\\[16\\]"):
        validate_tensors(x, w1, w2, bias1=torch.zeros(15).half(), bias2=b2)
    with pytest.raises(ValueError):
        validate_tensors(x, w1, w2, bias1=b1.float(), bias2=b2)
    with pytest.raises(ValueError, match="bias1\\[32\\]"):   # SwiGLU: bias1 covers gate and up
        validate_tensors(x, torch.zeros(32, 8).half(), w2, activation="swiglu", bias1=b1, bias2=b2)


def test_interleave_gate_up_layout():
    """Rows 64b..64b+31 hold gate rows 32b.., rows 64b+32.. the up rows of the same hidden
    columns; zero past h; a vector (bias1) interleaves the same way."""
    h, hp, k = 70, 128, 3
    w = torch.arange(2 * h * k, dtype=torch.float32).reshape(2 * h, k) + 1
    out = interleave_gate_up(w, h, hp)
    assert out.shape == (2 * hp, k)
    for hid in range(hp):
        blk, c = divmod(hid, 32)
        gate, up = out[64 * blk + c], out[64 * blk + 32 + c]
        if hid < h:
            assert torch.equal(gate, w[hid]) and torch.equal(up, w[h + hid])
        else:
            assert not gate.any() and not up.any()
    b = torch.arange(2 * h, dtype=torch.float32) + 1
    ib = interleave_gate_up(b, h, hp)
    assert ib[64 + 5] == b[32 + 5] and ib[64 + 32 + 5] == b[h + 32 + 5] and ib[63] == 0 + b[h + 31]


def test_swiglu_plans_use_block_pair_tiles():
    """The SwiGLU up GEMM runs over 2 hp interleaved rows on tiles whose wave tiles hold whole
    64-column block pairs, never split; a tile without them is refused when forced."""
    lib = _lib.load()
    code = _lib.BF16
    for (m, kp, hp) in ((8192, 3072, 8192), (16, 5120, 13824), (1005, 1024, 3008)):
        mp = -(-m // 64) * 64
        plan = _lib.make_plan(mp, kp, hp, 1024, code, "basic", "erf", 256, m=m, activation="swiglu")
        assert plan.activation == 3 and plan.up_sk_tiles == 0
        assert plan.up_tiles == -(-m // plan.up_bm) * -(-2 * hp // plan.up_bn)
        assert plan.up_bn % 64 == 0, (m, hp, plan.up_variant)
    for v in _lib.variants():
        try:
            _lib.make_plan(1024, 1024, 1024, 1024, code, "basic", "erf", 256, v["variant"], -1,
                           activation="swiglu")
        except ValueError as exc:
            assert "SwiGLU" in str(exc)
            # only the narrow tiles and the 256x192 tile (96-column wave tiles) lack block pairs
            assert v["bn"] <= 64 or v["bn"] % 128 != 0
    # SiLU splits like the GELU: the decode shard's up
    plan = _lib.make_plan(64, 5120, 1728, 5120, code, "basic", "erf", 256, 8, -1, m=16, activation="silu")
    assert plan.up_sk_tiles > 0


def test_run_ex_needs_both_biases():
    """Both biases or neither, refused before any device call."""
    lib = _lib.load()
    plan = _lib.make_plan(128, 256, 1024, 256, _lib.FP16, "basic", "erf", 256, activation="silu")
    fake = [ctypes.c_void_p(4096 * (i + 1)) for i in range(8)]
    rc = lib.ffn_mi355x_run_ex(ctypes.byref(plan), fake[0], fake[1], fake[2], fake[3], None, fake[4],
                               fake[5], fake[6], None)
    assert rc == _lib.EINVAL and "together" in _lib.last_error()


def test_eagle_entry_refusals():
    x, w1, w2 = torch.zeros(2, 8).half(), torch.zeros(8, 32).half(), torch.zeros(32, 4).half()
    with pytest.raises(ValueError, match="linear weight layout"):
        eagle_ffn_linear(x, torch.zeros(8, 64).half(), w2, activation="swiglu", layout="canonical")
    with pytest.raises(ValueError, match="no unfused fallback"):
        eagle_ffn_linear(x, w1, w2, fused=False, layout="canonical")
    with pytest.raises(ValueError, match="layout"):
        prepare_eagle_ffn(x, w1, w2, layout="columns")
    # a canonical call reaches the device check with the weights transposed to [H,K], [N,H]
    with pytest.raises(ValueError, match="requires ROCm GPU tensors"):
        eagle_ffn_linear(x, w1, w2, layout="canonical")


def test_activation_enters_the_tuning_key():
    """A SiLU or SwiGLU problem never takes a GELU entry of the tuning table."""
    p = problem_from_shapes((8192, 3072), (12288, 3072), (3072, 12288), "bfloat16", activation="silu")
    plan = make_plan(p, Selection(), 256)
    gelu = make_plan(problem_from_shapes((8192, 3072), (12288, 3072), (3072, 12288), "bfloat16"), Selection(), 256)
    assert plan.activation == "silu" and plan.native.activation == 2
    assert gelu.native.activation == 0
    untuned = make_plan(p, Selection(), 256, tuned=False)
    assert (plan.up.variant, plan.down.variant) == (untuned.up.variant, untuned.down.variant)
