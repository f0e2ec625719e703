"""GPU data plane of the paged KV cache: block pool, runners, host metadata packing."""

from mini_infra_qwen3_amd.worker.base_runner import BaseModelRunner, PrefillOutput
from mini_infra_qwen3_amd.worker.kv_cache import KVCache
from mini_infra_qwen3_amd.worker.paged_kv_cache import PagedKVCachePool
from mini_infra_qwen3_amd.worker.paged_runner import PagedDecodeOutput, PagedRunner
from mini_infra_qwen3_amd.worker.sampler import greedy_sample

__all__ = [
    "BaseModelRunner",
    "KVCache",
    "PagedDecodeOutput",
    "PagedKVCachePool",
    "PagedRunner",
    "PrefillOutput",
    "greedy_sample",
]
