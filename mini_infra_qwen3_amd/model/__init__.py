"""Qwen3 whose attention runs on the paged-KV data plane (dense GEMMs on PyTorch-ROCm)."""

from mini_infra_qwen3_amd.model.config import Qwen3Config, qwen3_0_6b
from mini_infra_qwen3_amd.model.qwen3 import (
    PagedAttentionMetadata,
    PagedMixedMetadata,
    PagedPrefillMetadata,
    Qwen3ForCausalLM,
    Qwen3Model,
    init_random_,
)

__all__ = [
    "PagedAttentionMetadata",
    "PagedMixedMetadata",
    "PagedPrefillMetadata",
    "Qwen3Config",
    "Qwen3ForCausalLM",
    "Qwen3Model",
    "init_random_",
    "qwen3_0_6b",
]
