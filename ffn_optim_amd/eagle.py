"""EagleFFN entry: Y = act(X W1 + b1) W2 + b2 with GELU, SiLU or SwiGLU, in either weight layout.

The operator the reference optimises is the bias-free GELU FFN; its analysis of the MindIE-SD
EagleFFN baseline (spec/MindIE-SD EagleFFN算子实现分析.md:17-140) describes the wider operator
this entry serves on the same kernels:

* activation 'gelu', 'silu' or 'swiglu' -- three alternative paths, not a chain (:17-44);
  SwiGLU's weight1 holds 2H rows, gate rows then up rows, and SiLU applies to the gate half
  only (:58-71);
* bias1 (H, or 2H for SwiGLU) and bias2 (N), given together or not at all (:84-86);
* layout 'linear' (weight1 [H,K], weight2 [N,H], nn.Linear's storage) or 'canonical'
  (weight1 [K,H], weight2 [H,N], the same weights transposed); SwiGLU is linear only (:76-86).

Canonical weights are read through their transposed views and copied into the kernels'
K-contiguous layout at preparation, like every operand that cannot be read in place.  There is
no unfused fallback: fused=False is refused.
"""
from __future__ import annotations

from .api import ffn, prepare_ffn

LAYOUTS = ("linear", "canonical")


def _linear_weights(weight1, weight2, activation, layout):
    if layout not in LAYOUTS:
        raise ValueError(f"layout must be one of {LAYOUTS}")
    if layout == "linear":
        return weight1, weight2
    if activation == "swiglu":
        raise ValueError("SwiGLU takes the linear weight layout only")
    if weight1.dim() != 2 or weight2.dim() != 2:
        raise ValueError("Expected weight1[K,H] and weight2[H,N] in the canonical layout")
    return weight1.t(), weight2.t()


def prepare_eagle_ffn(x, weight1, weight2, bias1=None, bias2=None, *, activation="gelu",
                      layout="linear", fused=True, **configuration):
    """Prepare the EagleFFN launch (prepare_ffn with the activation, biases and layout)."""
    if not fused:
        raise ValueError("only the fused operator is provided; there is no unfused fallback")
    w1, w2 = _linear_weights(weight1, weight2, activation, layout)
    return prepare_ffn(x, w1, w2, activation=activation, bias1=bias1, bias2=bias2, **configuration)


def eagle_ffn_linear(x, weight1, weight2, bias1=None, bias2=None, activation="gelu", fused=True,
                     layout="linear", **configuration):
    """Y = act(X . W1^T + b1) . W2^T + b2 for x [..., K]; returns [..., N] in x's dtype.

    Same argument order as the EagleFFN baseline's Python entry (analysis doc :124-133):
    x, the up and down weights, their biases, the activation.  Extra keywords are
    prepare_ffn's (down_impl, block_num, ...)."""
    if not fused:
        raise ValueError("only the fused operator is provided; there is no unfused fallback")
    w1, w2 = _linear_weights(weight1, weight2, activation, layout)
    return ffn(x, w1, w2, activation=activation, bias1=bias1, bias2=bias2, **configuration)
