"""infrared_amd — MI355X-native (gfx950) paged-attention hot path.

Drop-in for the paged-attention seam of the infrared inference engine:
``PagedKVPool`` / ``PagedContext`` / ``paged_attention`` keep the reference's
names and call contracts, and run hand-written HIP kernels through a C ABI
(``include/infrared_amd.h``, ``libinfrared_amd.so``).
"""

from infrared_amd.paged_attention import paged_attention, rope_paged_attention
from infrared_amd.paged_kv_cache import PagedContext, PagedKVPool

__all__ = ["PagedContext", "PagedKVPool", "paged_attention", "rope_paged_attention"]
__version__ = "0.1.0"
