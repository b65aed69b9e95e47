"""MI355X-native sparse shared-KV attention (gfx950 HIP kernels behind a C ABI).

Drop-in for the reference operator's Python interface:

* :func:`sparse_attn_sharedkv` (reference ``api.py``)
* :func:`sparse_attn_sharedkv_metadata` (reference ``metadata.py``)
"""

from .api import DEFAULT_BLOCK_I, DEFAULT_CORE_NUM, _get_kernel, sparse_attn_sharedkv  # noqa: F401
from .metadata import SAS_META_SIZE, sparse_attn_sharedkv_metadata  # noqa: F401

__all__ = ["sparse_attn_sharedkv", "sparse_attn_sharedkv_metadata", "SAS_META_SIZE",
           "DEFAULT_BLOCK_I", "DEFAULT_CORE_NUM"]
