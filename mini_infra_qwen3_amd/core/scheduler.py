"""Iteration-level scheduler of the continuous-batching paged run: arrival / waiting / running
queues and the chunked-prefill policy.

Behaviour of the reference's IterationScheduler under ``continuous-batching`` + ``paged-kv-cache``
+ ``chunked-prefill`` (src/mini_infra/core/scheduler.py:39-485, request state
src/mini_infra/core/request.py:52-110):

* a step is either PREFILL or DECODE, never both;
* after a PREFILL step, if any request is decoding, the next step is DECODE (decode protection);
* otherwise the in-flight chunked prefills plus newly admissible waiting requests (FCFS, limited by
  free batch slots and by free blocks after reserving the unwritten prompt blocks of in-flight
  prefills) share the token budget: each gets ``token_budget // n`` prompt tokens at most;
* with nothing to prefill, decode every request whose prompt is fully cached; else idle.

``mixed=True`` is the mixed chunk + decode batching the reference lists as its next step
(src/mini_infra/core/scheduler.py:310-311, src/mini_infra/core/types.py:108): every step decodes
all requests whose prompt is cached and spends what is left of the token budget (one token per
decoding request) on prefill chunks, split as above, in one MIXED step; a step with only one kind
of work is a plain DECODE or PREFILL step.  There is no decode protection: decoding never waits.
``mixed_chunk_tokens`` caps the prompt tokens of a MIXED step below that remainder (stall-free
batching as in Sarathi-Serve: a smaller chunk bounds the step's time and so the inter-token gap of
every decoding request, at the cost of more steps per prompt); PREFILL steps keep the full budget.

Pure CPU logic: no tensors, no device.
"""

from __future__ import annotations

import heapq
from collections import deque
from collections.abc import Iterable, Sequence
from dataclasses import dataclass, field
from enum import Enum

from mini_infra_qwen3_amd.core.block_manager import KVCacheManager, num_blocks_for_tokens
from mini_infra_qwen3_amd.core.types import Request


class RequestStatus(str, Enum):
    WAITING = "waiting"
    RUNNING = "running"
    FINISHED = "finished"


class SchedulePhase(str, Enum):
    PREFILL = "prefill"
    DECODE = "decode"
    MIXED = "mixed"


@dataclass
class RequestState:
    """Mutable run state of one request (reference request.py:52-110).

    ``cache_length`` counts the tokens whose K/V are scheduled into the cache: prompt chunks move
    it to ``chunk.end``, each decode step adds one.
    """

    request: Request
    status: RequestStatus = RequestStatus.WAITING
    generated: list[int] = field(default_factory=list)
    batch_slot_idx: int | None = None
    cache_length: int = 0
    admitted_ms: float | None = None
    first_token_ms: float | None = None
    completion_ms: float | None = None
    token_times_ms: list[float] = field(default_factory=list)
    finish_reason: str = "max_tokens"

    @property
    def is_prefilling(self) -> bool:
        return self.status is RequestStatus.RUNNING and self.cache_length < self.request.prompt_len

    def append_token(self, token_id: int, clock_ms: float, eos_token_id: int | None = None,
                     stop_on_eos: bool = True) -> bool:
        """Records a generated token; True when the request is done (EOS or output budget)."""
        self.generated.append(token_id)
        self.token_times_ms.append(clock_ms)
        if self.first_token_ms is None:
            self.first_token_ms = clock_ms
        hit_eos = stop_on_eos and eos_token_id is not None and token_id == eos_token_id
        if hit_eos or len(self.generated) >= self.request.max_new_tokens:
            self.completion_ms = clock_ms
            self.finish_reason = "stop" if hit_eos else "max_tokens"
            return True
        return False


class ArrivalQueue:
    """Requests not yet arrived, in arrival order (stable: equal times keep submission order)."""

    def __init__(self, states: Iterable[RequestState]):
        self._queue = deque(sorted(states, key=lambda s: s.request.arrival_ms))

    def __len__(self) -> int:
        return len(self._queue)

    def pop_arrived(self, clock_ms: float) -> list[RequestState]:
        out = []
        while self._queue and self._queue[0].request.arrival_ms <= clock_ms:
            out.append(self._queue.popleft())
        return out

    def next_arrival_ms(self) -> float:
        return self._queue[0].request.arrival_ms


@dataclass(frozen=True)
class PrefillChunk:
    """Prompt positions ``[start, end)`` of one request prefilled in one step (reference scheduler.py:228-246)."""

    state: RequestState
    start: int
    end: int

    @property
    def num_tokens(self) -> int:
        return self.end - self.start

    @property
    def is_last(self) -> bool:
        return self.end == self.state.request.prompt_len


@dataclass(frozen=True)
class SchedulerOutput:
    """One step's plan.  ``num_scheduled_tokens``: padded chunk tokens (rows x longest chunk) for
    PREFILL, the number of rows for DECODE (reference scheduler.py:249-264), their sum for MIXED.
    ``scheduled_requests`` lists a MIXED step's decoding requests first, then its chunks' requests."""

    phase: SchedulePhase
    scheduled_requests: tuple[RequestState, ...]
    num_scheduled_tokens: int
    prefill_chunks: tuple[PrefillChunk, ...] = ()

    @property
    def decode_requests(self) -> tuple[RequestState, ...]:
        """The requests that decode one token in this step (all of them for DECODE, none for PREFILL)."""
        return self.scheduled_requests[:len(self.scheduled_requests) - len(self.prefill_chunks)]


class IterationScheduler:
    """Continuous batching with chunked prefill over a paged KV cache.

    ``token_budget``: padded prompt tokens per PREFILL step (hard cap); ``max_running_requests``:
    batch slots; ``kv_cache_manager``: the block allocator this scheduler allocates and frees with;
    ``mixed_chunk_tokens`` (with ``mixed``): at most this many prompt tokens in a MIXED step.
    """

    def __init__(self, token_budget: int, max_running_requests: int, kv_cache_manager: KVCacheManager,
                 mixed: bool = False, mixed_chunk_tokens: int | None = None):
        if max_running_requests < 1:
            raise ValueError("max_running_requests must be positive")
        if token_budget < max_running_requests:
            raise ValueError("token_budget must be at least max_running_requests (every running prefill "
                             "advances by at least one token per step)")
        if mixed_chunk_tokens is not None and (not mixed or mixed_chunk_tokens < max_running_requests):
            raise ValueError("mixed_chunk_tokens needs mixed batching and at least max_running_requests tokens "
                             "(every prefill in a mixed step advances by at least one token)")
        self.token_budget = token_budget
        self.mixed = mixed
        self.mixed_chunk_tokens = mixed_chunk_tokens
        self.max_running_requests = max_running_requests
        self.kv_cache_manager = kv_cache_manager
        self.waiting: deque[RequestState] = deque()
        self.running: list[RequestState] = []
        self._free_slots = list(range(max_running_requests))
        self._last_phase: SchedulePhase | None = None

    @property
    def has_unfinished_requests(self) -> bool:
        return bool(self.waiting or self.running)

    def add_requests(self, states: Iterable[RequestState]) -> None:
        for state in states:
            state.status = RequestStatus.WAITING
            self.waiting.append(state)

    # -- decision ----------------------------------------------------------------------
    def _decoding(self) -> tuple[RequestState, ...]:
        return tuple(s for s in self.running if not s.is_prefilling)

    def _prefilling(self) -> tuple[RequestState, ...]:
        return tuple(s for s in self.running if s.is_prefilling)

    def _reserved_blocks(self) -> int:
        bs = self.kv_cache_manager.block_size
        return sum(num_blocks_for_tokens(s.request.prompt_len, bs) - num_blocks_for_tokens(s.cache_length, bs)
                   for s in self._prefilling())

    def _admission_candidates(self) -> tuple[RequestState, ...]:
        if not self._free_slots:
            return ()
        candidates = tuple(self.waiting)[:len(self._free_slots)]
        fits = self.kv_cache_manager.num_admissible([s.request.prompt_len for s in candidates],
                                                    self._reserved_blocks())
        return candidates[:fits]

    def _plan_chunks(self, budget: int) -> tuple[PrefillChunk, ...]:
        candidates = self._prefilling() + self._admission_candidates()
        if not candidates:
            return ()
        cap = budget // len(candidates)
        return tuple(PrefillChunk(s, s.cache_length, s.cache_length + min(s.request.prompt_len - s.cache_length, cap))
                     for s in candidates)

    def _decide(self) -> SchedulerOutput | None:
        decoding = self._decoding()
        if self.mixed:
            # token_budget >= max_running_requests, so every chunk still gets at least one token;
            # so does mixed_chunk_tokens (>= max_running_requests), which caps only MIXED steps
            budget = self.token_budget - len(decoding)
            if decoding and self.mixed_chunk_tokens is not None:
                budget = min(budget, self.mixed_chunk_tokens)
            chunks = self._plan_chunks(budget)
            if chunks and decoding:
                padded = len(chunks) * max(c.num_tokens for c in chunks)
                return SchedulerOutput(SchedulePhase.MIXED, decoding + tuple(c.state for c in chunks),
                                       len(decoding) + padded, chunks)
        elif decoding and self._last_phase is SchedulePhase.PREFILL:
            return SchedulerOutput(SchedulePhase.DECODE, decoding, len(decoding))
        else:
            chunks = self._plan_chunks(self.token_budget)
        if chunks:
            return SchedulerOutput(SchedulePhase.PREFILL, tuple(c.state for c in chunks),
                                   len(chunks) * max(c.num_tokens for c in chunks), chunks)
        if decoding:
            return SchedulerOutput(SchedulePhase.DECODE, decoding, len(decoding))
        return None

    # -- state transitions -------------------------------------------------------------
    def _allocate(self, state: RequestState, num_tokens: int) -> None:
        if not self.kv_cache_manager.allocate_slots(state.request.request_idx, num_tokens):
            raise RuntimeError("paged KV cache out of blocks (no preemption): enlarge num_blocks")

    def schedule(self, clock_ms: float) -> SchedulerOutput | None:
        """Plans one step and applies its admissions and block allocations; None when idle."""
        output = self._decide()
        if output is None:
            return None
        if output.phase is not SchedulePhase.DECODE:
            admitted = sum(1 for c in output.prefill_chunks if c.state.status is RequestStatus.WAITING)
            for _ in range(admitted):
                state = self.waiting.popleft()
                state.status = RequestStatus.RUNNING
                state.admitted_ms = clock_ms
                state.batch_slot_idx = heapq.heappop(self._free_slots)
                self.running.append(state)
            for chunk in output.prefill_chunks:
                self._allocate(chunk.state, chunk.num_tokens)
        for state in output.decode_requests:
            self._allocate(state, 1)
        self._last_phase = output.phase
        return output

    def update_from_output(self, output: SchedulerOutput, token_ids: Sequence[int], clock_ms: float,
                           eos_token_id: int | None = None, stop_on_eos: bool = True) -> list[RequestState]:
        """Advances the requests of a finished step; ``token_ids`` are the new tokens of every decode
        row, then of the prefill rows whose chunk completed the prompt.  Frees finished requests."""
        for state in output.decode_requests:
            state.cache_length += 1
        for chunk in output.prefill_chunks:
            chunk.state.cache_length = chunk.end
        producers = output.decode_requests + tuple(c.state for c in output.prefill_chunks if c.is_last)
        if len(token_ids) != len(producers):
            raise ValueError(f"{len(token_ids)} tokens for {len(producers)} producing requests")
        finished = [s for s, t in zip(producers, token_ids) if s.append_token(int(t), clock_ms, eos_token_id,
                                                                                stop_on_eos)]
        for state in finished:
            self.kv_cache_manager.free(state.request.request_idx)
            state.status = RequestStatus.FINISHED
            heapq.heappush(self._free_slots, state.batch_slot_idx)
        if finished:
            self.running = [s for s in self.running if s.status is RequestStatus.RUNNING]
        return finished


__all__ = [
    "ArrivalQueue",
    "IterationScheduler",
    "PrefillChunk",
    "RequestState",
    "RequestStatus",
    "SchedulePhase",
    "SchedulerOutput",
]
