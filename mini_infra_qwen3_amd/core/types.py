"""Control-plane value types the paged path needs (no torch, CPU only)."""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class Request:
    """Immutable request payload on the logical timeline. Reference src/mini_infra/core/request.py:28-49."""

    request_idx: int
    token_ids: tuple[int, ...]
    max_new_tokens: int
    arrival_ms: float = 0.0

    def __post_init__(self) -> None:
        if self.request_idx < 0:
            raise ValueError("request_idx must be non-negative")
        if not self.token_ids:
            raise ValueError("prompt must not be empty")
        if self.max_new_tokens < 1:
            raise ValueError("max_new_tokens must be positive")
        if self.arrival_ms < 0:
            raise ValueError("arrival_ms must be non-negative")

    @property
    def prompt_len(self) -> int:
        return len(self.token_ids)


@dataclass(frozen=True)
class PagedCacheConfig:
    """Paged KV cache settings. Reference src/mini_infra/core/types.py:47-66.

    block_size: tokens per block; num_blocks: pool size including the null block (None: derive
    it from the workload with ``required_pool_blocks``).
    """

    block_size: int = 16
    num_blocks: int | None = None

    def __post_init__(self) -> None:
        if self.block_size < 1:
            raise ValueError("block_size must be positive")
        if self.num_blocks is not None and self.num_blocks < 2:
            raise ValueError("num_blocks must be at least 2 (block 0 is the null block)")


__all__ = ["PagedCacheConfig", "Request"]
