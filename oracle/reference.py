"""Oracle -- TEST INFRASTRUCTURE ONLY, never part of the product path.

CPU restatement of the reference's golden FFN and its error metric:

  gelu_rational  validation/reference.py:5-13   rational erf GELU (FP32)
  gelu_erf       validation/reference.py:19     F.gelu(approximate='none')
  ffn_torch      validation/reference.py:16-23  FP32 matmul -> GELU -> [stage] -> matmul -> cast
  compare        validation/test_ffn.py:6-21    mean(|o-g|/(|g|+1e-3)) < 0.05 (+ max_abs, rms)
  silu, biases,  spec/MindIE-SD EagleFFN算子实现分析.md:17-71, :88-94   the EagleFFN paths the
  swiglu         reference's analysis describes (FP32 up + bias -> activation or gating ->
                 [stage] -> FP32 down + bias -> cast)

Pinning (tests/test_oracle.py): the reference's own KATs (rational-vs-erf bound
< 2e-5 on linspace(-10,10,10001); compare's bad-result cases), closed forms
(math.erf), brute-force integer FFNs in pure Python, the independent C
restatement oracle/ffn_ref.c (double accumulation), invariants (padding,
odd symmetry, the clamp).  Nothing here is imported by ffn_optim_amd/.
"""
from __future__ import annotations

from math import prod

SQRT1_2 = 0.70710678118654752


def gelu_rational(z):
    """Rational erf GELU of the reference kernel, FP32 (validation/reference.py:5-13)."""
    t = (z.float() * SQRT1_2).clamp(-3.92, 3.92)
    t2 = t * t
    p = (((((t2 * 0.053443748819 + 7.5517016694) * t2 + 101.62808918)
            * t2 + 1393.8061484) * t2 + 5063.7915060) * t2 + 29639.384698) * t
    q = ((((t2 + 31.212858877) * t2 + 398.56963806) * t2 + 3023.1248150)
         * t2 + 13243.365831) * t2 + 26267.224157
    return 0.5 * z.float() * (1 + p / q)


def gelu_erf(z):
    """Exact GELU 0.5*z*(1+erf(z/sqrt2)) in FP32 (validation/reference.py:19)."""
    import torch.nn.functional as F
    return F.gelu(z.float(), approximate="none")


def silu(z):
    """SiLU(z) = z / (1 + exp(-z)) in FP32 (analysis doc :52-56)."""
    import torch
    z = z.float()
    return z / (1 + torch.exp(-z))


def shapes(x_shape, w1_shape, w2_shape, activation="gelu"):
    """(m, k, h, n, output_shape) of an FFN, without the product's validation; SwiGLU's w1 has
    2H rows."""
    u, k = w1_shape
    n, h = w2_shape
    assert x_shape[-1] == k and u == (2 * h if activation == "swiglu" else h), "x[...,K], w1[H|2H,K], w2[N,H]"
    return prod(x_shape[:-1]), k, h, n, (*x_shape[:-1], n)


def ffn_torch(x, weight1, weight2, *, staged=False, rational=False, activation="gelu", bias1=None,
              bias2=None):
    """Torch FP32 golden (validation/reference.py:16-23), widened to the EagleFFN paths.

    z = X[m,k].float() @ W1.float().T (+ bias1); hidden = GELU(z) (erf, or the rational
    form), SiLU(z), or for SwiGLU SiLU(z[:, :H]) * z[:, H:] (gate columns first);
    staged rounds hidden to the input dtype before the second matmul; the down product
    (+ bias2) is cast once to the input dtype and reshaped to [..., N].
    """
    m, k, h, _, out_shape = shapes(tuple(x.shape), tuple(weight1.shape), tuple(weight2.shape), activation)
    z = x.reshape(m, k).float() @ weight1.float().T
    if bias1 is not None:
        z = z + bias1.float()
    if activation == "gelu":
        hidden = gelu_rational(z) if rational else gelu_erf(z)
    elif activation == "silu":
        hidden = silu(z)
    elif activation == "swiglu":
        hidden = silu(z[:, :h]) * z[:, h:]
    else:
        raise ValueError(activation)
    if staged:
        hidden = hidden.to(x.dtype).float()
    y = hidden @ weight2.float().T
    if bias2 is not None:
        y = y + bias2.float()
    return y.to(x.dtype).reshape(out_shape)


def ffn_rows(x, weight1, weight2, rows, **kw):
    """ffn_torch on a subset of the rows of X (each output row depends on its X row only)."""
    m, k, _, n, _ = shapes(tuple(x.shape), tuple(weight1.shape), tuple(weight2.shape),
                           kw.get("activation", "gelu"))
    xs = x.reshape(m, k)[rows]
    return ffn_torch(xs, weight1, weight2, **kw)


def compare(output, golden):
    """Pass criterion of validation/test_ffn.py:6-21 (shape, dtype, finiteness, mean_rel < 0.05)."""
    import torch
    result = {"passed": False, "shape_ok": tuple(output.shape) == tuple(golden.shape),
              "dtype_ok": output.dtype == golden.dtype, "finite": False,
              "max_abs": None, "rms": None, "mean_rel": None}
    if not result["shape_ok"] or not result["dtype_ok"]:
        return result
    a, b = output.detach().float(), golden.detach().float()
    result["finite"] = bool(torch.isfinite(a).all() and torch.isfinite(b).all())
    if not result["finite"] or not a.numel():
        return result
    d = (a - b).abs()
    result.update(max_abs=d.max().item(), rms=d.square().mean().sqrt().item(),
                  mean_rel=(d / (b.abs() + 1e-3)).mean().item())
    result["passed"] = result["mean_rel"] < 0.05
    return result
