"""Serving harness around the paged model: sequences, ragged batches, scheduler, engine."""

from mini_vllm.serve.batch import ForwardBatch
from mini_vllm.serve.engine import EngineStats, LLMEngine
from mini_vllm.serve.scheduler import Scheduler, SchedulerConfig, SchedulerOutput
from mini_vllm.serve.sequence import Sequence

__all__ = ["EngineStats", "ForwardBatch", "LLMEngine", "Scheduler", "SchedulerConfig",
           "SchedulerOutput", "Sequence"]
