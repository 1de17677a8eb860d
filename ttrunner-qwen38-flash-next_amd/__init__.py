"""qwen4mix: the qwen4exp token-mixing path (QSA + Gated DeltaNet) for MI355X.

Drop-in for the token-mixing methods of the reference engine's PyTorch model
(``_linear_attention``, ``_full_attention``, ``_indexer_mask``), backed by
hand-written gfx950 HIP kernels behind the C ABI of libqwen4mix.so
(include/qwen4mix.h). Importing this package never falls back to a CPU path: the
native library must be built (``build.build()``) before any layer is used.
"""

from . import native
from .cache import MixHybridCache, MixLayerCache
from .config import MixConfig
from .decoder import MixDecoder
from .model import Qwen4MixModel
from .pages import PagePool, PoolExhausted

__all__ = ["native", "MixHybridCache", "MixLayerCache", "MixConfig", "MixDecoder", "Qwen4MixModel", "PagePool",
           "PoolExhausted"]
