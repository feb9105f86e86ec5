"""TurboQuant KV-cache compression and compressed-cache attention for AMD
MI355X (gfx950), with the public API of mlx-turboquant
(mlx_turboquant/__init__.py:45-59): apply_turboquant, enable_turboquant,
TurboQuantKVCache, TurboQuantMSE, TurboQuantProd.

All compute runs in the hand-written HIP kernels of ``libtq_hip.so``; there is
no CPU fallback.
"""

__version__ = "0.1.0"

from .cache import TurboQuantKVCache
from .patch import apply_turboquant, detect_outlier_layers, enable_turboquant
from .quantizer import QuantizedTensor, TurboQuantMSE, TurboQuantProd

__all__ = [
    "__version__",
    "apply_turboquant",
    "enable_turboquant",
    "TurboQuantKVCache",
    "TurboQuantMSE",
    "TurboQuantProd",
    "QuantizedTensor",
    "detect_outlier_layers",
]
