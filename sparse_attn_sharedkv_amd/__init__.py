"""MI355X (gfx950) sparse shared-KV attention decode.

Drop-in for the reference's ``api.sparse_attn_sharedkv``,
``sparse_flash_mla_api.sparse_flash_mla`` and
``metadata.sparse_attn_sharedkv_metadata``; compute runs in the HIP library
``_lib/libsas_mi355x.so`` (C ABI in ``include/sas_mi355x.h``).
"""

from .api import DEFAULT_BLOCK_I, sparse_attn_sharedkv  # noqa: F401
from .kv_fp8 import append_kv_fp8, quantize_kv_fp8  # noqa: F401
from .metadata import (AIC_CORE_NUM, AIV_CORE_NUM, DEFAULT_CORE_NUM, FA_METADATA_SIZE,  # noqa: F401
                       FD_METADATA_SIZE, SAS_META_SIZE, sparse_attn_sharedkv_metadata)
from .sparse_flash_mla_api import sparse_flash_mla  # noqa: F401

__all__ = ["sparse_attn_sharedkv", "sparse_flash_mla", "sparse_attn_sharedkv_metadata",
           "append_kv_fp8", "quantize_kv_fp8",
           "SAS_META_SIZE", "AIC_CORE_NUM", "AIV_CORE_NUM", "FA_METADATA_SIZE",
           "FD_METADATA_SIZE", "DEFAULT_CORE_NUM", "DEFAULT_BLOCK_I"]
