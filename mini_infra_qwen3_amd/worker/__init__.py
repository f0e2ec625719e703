"""GPU data plane of the paged KV cache: block pool, runners, host metadata packing, block swap."""

from mini_infra_qwen3_amd.worker.base_runner import BaseModelRunner, PrefillOutput
from mini_infra_qwen3_amd.worker.block_tables import DeviceBlockTables
from mini_infra_qwen3_amd.worker.kv_cache import KVCache
from mini_infra_qwen3_amd.worker.kv_swap import HostSwapPool, KVBlockHeader, load_kv_blocks, save_kv_blocks
from mini_infra_qwen3_amd.worker.paged_kv_cache import PagedKVCachePool
from mini_infra_qwen3_amd.worker.paged_runner import MixedStepOutput, PagedDecodeOutput, PagedRunner
from mini_infra_qwen3_amd.worker.sampler import greedy_sample

__all__ = [
    "DeviceBlockTables",
    "BaseModelRunner",
    "HostSwapPool",
    "KVBlockHeader",
    "KVCache",
    "MixedStepOutput",
    "PagedDecodeOutput",
    "PagedKVCachePool",
    "PagedRunner",
    "PrefillOutput",
    "greedy_sample",
    "load_kv_blocks",
    "save_kv_blocks",
]
