"""MI355X-native TriAttention KV-cache compression behind method API v1.

Python mirror of the reference plugin's method boundary
(``vllm_ascend_kvcompress``) whose compute runs in hand-written HIP kernels
for gfx950, reached through the C ABI of ``libkvcompress_mi355x.so``.
"""

from .config import KERNEL_BLOCK_SIZE, PROVIDER_NAME
from .methods import METHOD_API_VERSION, available_methods, create_method, register_method

__all__ = [
    "KERNEL_BLOCK_SIZE",
    "METHOD_API_VERSION",
    "PROVIDER_NAME",
    "available_methods",
    "create_method",
    "register_method",
]
__version__ = "0.1.0"
