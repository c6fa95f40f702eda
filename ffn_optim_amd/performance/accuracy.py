"""FP32 golden and the error criterion the harness validates candidates with.

golden() composes torch CPU FP32 ops in the order of validation/reference.py:16-23
(X reshaped to [m, k] @ W1^T -> exact or rational GELU -> [staged: cast to the input dtype and
back] -> @ W2^T -> cast to the input dtype -> leading dims restored); compare() is validation/test_ffn.py:6-21:
shape/dtype/finiteness, max_abs, rms and mean(|a-b|/(|b|+1e-3)) < 0.05.
"""
from __future__ import annotations

TOLERANCE = 0.05


def gelu_rational(x):
    """Rational erf GELU, coefficients and order of validation/reference.py:5-13."""
    import torch
    t = torch.clamp(x * 0.70710678118654752, -3.92, 3.92)
    t2 = t * t
    p = t2 * 0.053443748819 + 7.5517016694
    p = p * t2 + 101.62808918
    p = p * t2 + 1393.8061484
    p = p * t2 + 5063.7915060
    p = p * t2 + 29639.384698
    p = p * t
    q = t2 + 31.212858877
    q = q * t2 + 398.56963806
    q = q * t2 + 3023.1248150
    q = q * t2 + 13243.365831
    q = q * t2 + 26267.224157
    return x * 0.5 * (p / q + 1.0)


def golden(x, w1, w2, gelu="erf", staged=False):
    """CPU FP32 reference output in the input dtype.  staged rounds the hidden activation to the
    input dtype before the second product, as the kernels store it (the reference's staged
    golden, validation/reference.py:16-23)."""
    import torch
    m, k = x.numel() // x.shape[-1], x.shape[-1]
    xs = x.detach().cpu().reshape(m, k).float()
    z = xs @ w1.detach().cpu().float().T
    h = torch.nn.functional.gelu(z, approximate="none") if gelu == "erf" else gelu_rational(z)
    if staged:
        h = h.to(x.dtype).float()
    y = h @ w2.detach().cpu().float().T
    return y.to(x.dtype).reshape(*x.shape[:-1], w2.shape[0])


def golden_rows(x, w1, w2, rows, gelu="erf"):
    """golden() on a subset of the rows of X (each output row depends on its own X row only);
    returns [len(rows), N]."""
    m, k = x.numel() // x.shape[-1], x.shape[-1]
    xs = x.detach().reshape(m, k)[rows.to(x.device)]
    return golden(xs, w1, w2, gelu)


def sample_rows(m, count=384, seed=7):
    """A seeded sample of `count` row indices of an m-row problem (all rows when m <= count)."""
    import torch
    if m <= count:
        return torch.arange(m)
    return torch.randperm(m, generator=torch.Generator().manual_seed(seed))[:count]


def compare(actual, expected):
    """The reference's pass/fail criterion with its diagnostics."""
    import torch
    res = {"shape_ok": tuple(actual.shape) == tuple(expected.shape),
           "dtype_ok": actual.dtype == expected.dtype}
    a, b = actual.detach().cpu().float(), expected.detach().cpu().float()
    res["finite"] = bool(torch.isfinite(a).all() and torch.isfinite(b).all())
    if not (res["shape_ok"] and res["dtype_ok"] and res["finite"]):
        res.update(passed=False, max_abs=None, rms=None, mean_rel=None)
        return res
    d = (a - b).abs()
    res["max_abs"] = float(d.max()) if d.numel() else 0.0
    res["rms"] = float(torch.sqrt((d * d).mean())) if d.numel() else 0.0
    res["mean_rel"] = float((d / (b.abs() + 1e-3)).mean()) if d.numel() else 0.0
    res["passed"] = res["mean_rel"] < TOLERANCE
    return res
