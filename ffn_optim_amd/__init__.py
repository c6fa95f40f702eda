"""MI355X-native fused FFN operator, Y = GELU(X @ W1.T) @ W2.T (FP16/BF16, gfx950)."""
from .api import KernelCompilationError, PreparedFFN, ffn, prepare_ffn

__all__ = ["ffn", "prepare_ffn", "PreparedFFN", "KernelCompilationError"]
