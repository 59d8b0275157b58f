"""mlc for MI355X: a static-shape PyTorch inference compiler whose fused
kernels, arena and replay run natively on CDNA4 through HIP."""

from .api import compile
from .config import ELEMENTWISE_ONLY, NO_FUSION, Config

__version__ = "0.1.0"
__all__ = ["compile", "Config", "ELEMENTWISE_ONLY", "NO_FUSION"]
