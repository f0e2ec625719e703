"""CPU control plane of the paged KV cache (block tables, free-block queue, request types)."""

from mini_infra_qwen3_amd.core.block_manager import (
    NULL_BLOCK_ID,
    FreeKVCacheBlockQueue,
    KVCacheManager,
    num_blocks_for_tokens,
    required_pool_blocks,
)
from mini_infra_qwen3_amd.core.types import PagedCacheConfig, Request

__all__ = [
    "FreeKVCacheBlockQueue",
    "KVCacheManager",
    "NULL_BLOCK_ID",
    "PagedCacheConfig",
    "Request",
    "num_blocks_for_tokens",
    "required_pool_blocks",
]
