"""MI355X-native fused FFN operator, Y = GELU(X @ W1.T) @ W2.T (FP16/BF16, gfx950), and the
EagleFFN form act(X @ W1.T + b1) @ W2.T + b2 with GELU, SiLU or SwiGLU."""
from .api import KernelCompilationError, PreparedFFN, ffn, prepare_ffn
from .eagle import eagle_ffn_linear, prepare_eagle_ffn

__all__ = ["ffn", "prepare_ffn", "PreparedFFN", "KernelCompilationError", "eagle_ffn_linear",
           "prepare_eagle_ffn"]
