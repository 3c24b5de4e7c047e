"""MI355X-native TurboPolar compressed-KV decode attention.

Drop-in for the reference's TurboPolar decode path (the
``TurboPolarKVCacheRuntime`` append/attend API, its page layout and the
``MetalKernelBridge`` methods), implemented as hand-written gfx950 HIP kernels
behind the C ABI of ``include/turbopolar.h`` (``libturbopolar_hip.so``).
"""

from .bridge import HipKernelBridge
from .codecs import GroupedVQuantizer, PolarQuantDecoder, PolarQuantEncoder
from .config import TurboPolarConfig
from .fast_attention import TurboPolarFastCache, make_turbo_caches
from .payload import PolarKeyBlock, QuantizedVBlock
from .runtime import TurboPolarKVCacheRuntime
from .storage import PolarKBlockStorage, QuantVBlockStorage

__all__ = [
    "GroupedVQuantizer",
    "HipKernelBridge",
    "PolarKBlockStorage",
    "PolarKeyBlock",
    "PolarQuantDecoder",
    "PolarQuantEncoder",
    "QuantVBlockStorage",
    "QuantizedVBlock",
    "TurboPolarConfig",
    "TurboPolarFastCache",
    "TurboPolarKVCacheRuntime",
    "make_turbo_caches",
]
