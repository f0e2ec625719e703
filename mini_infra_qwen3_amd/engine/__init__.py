"""Continuous-batching driver of the paged path: scheduler loop, paged backend, metrics."""

from mini_infra_qwen3_amd.engine.paged_backend import PagedScheduleBackend, ScheduleStepOutput
from mini_infra_qwen3_amd.engine.scheduler_loop import ScheduleEvent, ScheduleResult, run_scheduler

__all__ = ["PagedScheduleBackend", "ScheduleEvent", "ScheduleResult", "ScheduleStepOutput", "run_scheduler"]
