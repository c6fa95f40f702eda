"""Pins the oracle (CPU only): reference KATs, closed forms, brute force, the C restatement.

Each check is chosen so a plausible slip (tanh GELU instead of erf, a transposed
weight, a dropped rounding stage, a wrong rounding mode) fails one of them.
"""
import math
import ctypes

import numpy as np
import pytest
import torch

from oracle import build as oracle_build
from oracle.reference import compare, ffn_rows, ffn_torch, gelu_erf, gelu_rational


@pytest.fixture(scope="module")
def cref():
    return oracle_build.load()


def _fptr(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def test_rational_gelu_bound_vs_erf():
    """Reference KAT (validation/test_ffn.py:91-96): |rational - erf GELU| < 2e-5 on [-10, 10]."""
    x = torch.linspace(-10, 10, 10001)
    d = (gelu_rational(x) - torch.nn.functional.gelu(x, approximate="none")).abs()
    assert d.max().item() < 2e-5


def test_erf_gelu_closed_form():
    """GELU is the exact-erf form (not tanh): compare with math.erf in double."""
    pts = [i / 8 for i in range(-64, 65)]
    got = gelu_erf(torch.tensor(pts, dtype=torch.float32)).double()
    for z, g in zip(pts, got.tolist()):
        exact = 0.5 * z * (1 + math.erf(z / math.sqrt(2)))
        assert abs(g - exact) <= 2e-6 * max(1.0, abs(z)), z
    tanh = torch.nn.functional.gelu(torch.tensor([1.0]), approximate="tanh").item()
    assert abs(gelu_erf(torch.tensor([1.0])).item() - tanh) > 1e-4  # the two forms differ


def test_rational_gelu_invariants(cref):
    """Odd symmetry of the erf part, the clamp at |t| = 3.92, and op-by-op agreement with C."""
    z = torch.linspace(-12, 12, 4801)
    g = gelu_rational(z)
    # GELU(z) - GELU(-z) = z for an odd erf approximation
    assert torch.allclose(g - gelu_rational(-z), z, atol=2e-5)
    # beyond the clamp the approximated erf is a constant
    big = torch.tensor([6.0, 8.0, 11.0])
    ratio = gelu_rational(big) / (0.5 * big)
    assert torch.allclose(ratio, ratio[0].expand(3), rtol=0, atol=1e-6)
    c = np.array([cref.ffn_ref_gelu_rational(float(v)) for v in z.tolist()], dtype=np.float32)
    assert np.max(np.abs(c - g.numpy())) <= 4e-6


def test_compare_rejects_bad_results():
    """Reference KAT (validation/test_ffn.py:84-89)."""
    a = torch.ones(2, 3).half()
    assert compare(a, a)["passed"]
    for bad in (a.float(), a.T, a * float("nan"), a * float("inf"), a * 2):
        assert not compare(bad, a)["passed"]
    r = compare(a * 1.01, a)
    assert r["passed"] and abs(r["max_abs"] - 0.01) < 2e-3 and r["rms"] > 0


def _brute_ffn(x, w1, w2, gelu):
    m, k = len(x), len(x[0])
    h, n = len(w1), len(w2)
    out = []
    for i in range(m):
        hid = [gelu(sum(x[i][l] * w1[j][l] for l in range(k))) for j in range(h)]
        out.append([sum(hid[j] * w2[c][j] for j in range(h)) for c in range(n)])
    return out


def test_ffn_torch_brute_force_orientation():
    """Non-square integer case in pure Python: pins X@W1^T, W2^T orientation and reshape."""
    g = torch.Generator().manual_seed(3)
    x = torch.randint(-2, 3, (2, 3, 5), generator=g).float()
    w1 = torch.randint(-2, 3, (7, 5), generator=g).float()
    w2 = torch.randint(-2, 3, (4, 7), generator=g).float()
    gelu = lambda z: 0.5 * z * (1 + math.erf(z / math.sqrt(2)))
    exact = _brute_ffn(x.reshape(6, 5).tolist(), w1.tolist(), w2.tolist(), gelu)
    got = ffn_torch(x, w1, w2)
    assert got.shape == (2, 3, 4)
    assert np.allclose(got.reshape(6, 4).numpy(), np.array(exact), atol=1e-4)


@pytest.mark.parametrize("dtype,code", [(torch.float16, 0), (torch.bfloat16, 1)])
@pytest.mark.parametrize("rational", [False, True])
def test_ffn_torch_matches_c_restatement(cref, dtype, code, rational):
    g = torch.Generator().manual_seed(5)
    m, k, h, n = 9, 40, 70, 33
    x = torch.randn(m, k, generator=g).to(dtype)
    w1 = (torch.randn(h, k, generator=g) * k ** -0.5).to(dtype)
    w2 = (torch.randn(n, h, generator=g) * h ** -0.5).to(dtype)
    xs, a, b = (t.float().numpy().copy() for t in (x, w1, w2))
    for staged in (False, True):
        out = np.zeros((m, n), np.float32)
        hid = np.zeros((m, h), np.float32)
        cref.ffn_ref_run(_fptr(xs), _fptr(a), _fptr(b), _fptr(hid), _fptr(out), m, k, h, n,
                         int(rational), code if staged else -1)
        got = ffn_torch(x, w1, w2, staged=staged, rational=rational).float().numpy()
        cref_cast = torch.from_numpy(out).to(dtype).float().numpy()
        # the two differ only by FP32 summation order before one rounding to dtype
        ulp = np.abs(cref_cast) * (2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10)
        assert np.all(np.abs(got - cref_cast) <= ulp + 1e-5)


@pytest.mark.parametrize("dtype,code", [(torch.float16, 0), (torch.bfloat16, 1)])
def test_torch_casts_are_rne(cref, dtype, code):
    """The oracle's casts (torch .to) equal an explicit round-to-nearest-even: ties, overflow,
    subnormals, NaN."""
    vals = [0.0, -0.0, 1.0, 1.0009765625, 1.00048828125, 1.00146484375, 65504.0, 65519.0, 65520.0,
            1e-7, 6e-8, 3e-5, -2.5, 1 + 2 ** -8, 1 + 3 * 2 ** -9, float("inf"), 1e30]
    rng = np.random.default_rng(0)
    arr = np.concatenate([np.array(vals, np.float32),
                          rng.standard_normal(4096).astype(np.float32) * 100]).astype(np.float32)
    out = np.zeros_like(arr)
    cref.ffn_ref_round(_fptr(arr), _fptr(out), arr.size, code)
    t = torch.from_numpy(arr).to(dtype).float().numpy()
    assert np.array_equal(t, out)
    nan_in = np.array([np.nan], np.float32)
    nan_out = np.zeros(1, np.float32)
    cref.ffn_ref_round(_fptr(nan_in), _fptr(nan_out), 1, code)
    assert np.isnan(nan_out[0])


def test_staged_rounding_changes_result():
    """staged=True really rounds the hidden activation (a dropped stage would pass unnoticed)."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(32, 64, generator=g).half()
    w1 = torch.randn(128, 64, generator=g).half()
    w2 = torch.randn(48, 128, generator=g).half()
    a = ffn_torch(x, w1, w2).float()
    b = ffn_torch(x, w1, w2, staged=True).float()
    assert not torch.equal(a, b)
    assert compare(b.half(), a.half())["passed"]


def test_row_sampling_equals_full():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 8, 24, generator=g).bfloat16()
    w1 = torch.randn(40, 24, generator=g).bfloat16()
    w2 = torch.randn(16, 40, generator=g).bfloat16()
    rows = torch.tensor([0, 5, 11, 15])
    full = ffn_torch(x, w1, w2).reshape(16, 16)
    assert torch.equal(ffn_rows(x, w1, w2, rows), full[rows])


# ---- the EagleFFN paths (spec/MindIE-SD EagleFFN算子实现分析.md:17-71) ------------------------

def test_silu_closed_form_and_identity():
    """SiLU is z / (1 + e^-z) (math.exp in double), not z * tanh or the GELU; SiLU(z) - SiLU(-z) = z."""
    from oracle.reference import silu
    pts = [i / 8 for i in range(-96, 97)]
    got = silu(torch.tensor(pts, dtype=torch.float32)).double()
    for z, g in zip(pts, got.tolist()):
        exact = z / (1 + math.exp(-z))
        assert abs(g - exact) <= 2e-6 * max(1.0, abs(z)), z
    z = torch.linspace(-20, 20, 801)
    assert torch.allclose(silu(z) - silu(-z), z, atol=2e-5)
    assert torch.allclose(silu(z), torch.nn.functional.silu(z), atol=1e-6, rtol=1e-6)
    assert abs(silu(torch.tensor([1.0])).item() - gelu_erf(torch.tensor([1.0])).item()) > 1e-2


def _brute_eagle(x, w1, w2, b1, b2, act):
    """act(x W1^T + b1) W2^T + b2 in pure Python; act maps the list of up outputs of one row to
    the hidden row (SwiGLU: the first half gated by the second)."""
    out = []
    for row in x:
        z = [sum(a * b for a, b in zip(row, w)) + bb for w, bb in zip(w1, b1)]
        hid = act(z)
        out.append([sum(hh * w for hh, w in zip(hid, wr)) + bb for wr, bb in zip(w2, b2)])
    return out


@pytest.mark.parametrize("activation", ["gelu", "silu", "swiglu"])
def test_ffn_torch_eagle_paths_brute_force(activation):
    """Integer operands and biases: the bias goes into the up sum before the activation and into
    the down sum before the cast; SwiGLU gates with the first H columns of the up output (swapping
    the halves, or adding bias1 after the activation, changes the result)."""
    g = torch.Generator().manual_seed(11)
    m, k, h, n = 3, 5, 4, 2
    u = 2 * h if activation == "swiglu" else h
    x = torch.randint(-2, 3, (m, k), generator=g).float()
    w1 = torch.randint(-2, 3, (u, k), generator=g).float()
    w2 = torch.randint(-2, 3, (n, h), generator=g).float()
    b1 = torch.randint(-2, 3, (u,), generator=g).float()
    b2 = torch.randint(-2, 3, (n,), generator=g).float()
    gelu1 = lambda v: 0.5 * v * (1 + math.erf(v / math.sqrt(2)))
    silu1 = lambda v: v / (1 + math.exp(-v))
    act = {"gelu": lambda z: [gelu1(v) for v in z], "silu": lambda z: [silu1(v) for v in z],
           "swiglu": lambda z: [silu1(a) * b for a, b in zip(z[:h], z[h:])]}[activation]
    want = torch.tensor(_brute_eagle(x.tolist(), w1.tolist(), w2.tolist(), b1.tolist(), b2.tolist(), act))
    got = ffn_torch(x, w1, w2, activation=activation, bias1=b1, bias2=b2)
    assert torch.allclose(got, want, atol=1e-4, rtol=1e-5)
    # the slips this pins: no bias, bias after the activation, swapped SwiGLU halves
    assert not torch.allclose(ffn_torch(x, w1, w2, activation=activation), want, atol=1e-3)
    late = torch.tensor(_brute_eagle(x.tolist(), w1.tolist(), w2.tolist(), [0.0] * u, b2.tolist(),
                                     lambda z: [a + b for a, b in zip(act(z), b1.tolist())]
                                     if activation != "swiglu" else act(z)))
    if activation != "swiglu":
        assert not torch.allclose(got, late, atol=1e-3)
    else:
        swapped = ffn_torch(x, torch.cat([w1[h:], w1[:h]]), w2, activation=activation,
                            bias1=torch.cat([b1[h:], b1[:h]]), bias2=b2)
        assert not torch.allclose(swapped, want, atol=1e-3)
