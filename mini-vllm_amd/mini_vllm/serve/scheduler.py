"""Continuous batching with chunked prefill (reference serve/scheduler.py:50-433).

Each iteration fills a token budget in priority order: one token for every decoding
sequence, then prefill chunks (at most ``chunk_size`` each) for admitted sequences, then
admissions from the waiting queue (FCFS) while ``max_sequences`` allows. Pages are
allocated as tokens are scheduled; when a running sequence cannot get its pages, the
most recently admitted other sequence is preempted (its pages freed, recomputed later)
and goes back to the front of the queue.
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field

from mini_vllm.block.block_manager import BlockManager, OutOfBlocks
from mini_vllm.serve.sequence import Sequence

__all__ = ["Scheduler", "SchedulerConfig", "SchedulerOutput"]


@dataclass(frozen=True)
class SchedulerConfig:
    max_batched_tokens: int = 2048
    max_sequences: int = 32
    chunk_size: int = 512
    enable_chunked_prefill: bool = True


@dataclass
class SchedulerOutput:
    scheduled: list[tuple[Sequence, int]] = field(default_factory=list)
    preempted: list[Sequence] = field(default_factory=list)

    @property
    def total_tokens(self) -> int:
        return sum(n for _, n in self.scheduled)

    @property
    def num_decodes(self) -> int:
        return sum(1 for s, n in self.scheduled if n == 1 and s.output)


class Scheduler:
    def __init__(self, config: SchedulerConfig, manager: BlockManager) -> None:
        self.config = config
        self.manager = manager
        self.waiting: deque[Sequence] = deque()
        self.running: list[Sequence] = []
        self.finished: list[Sequence] = []

    def add(self, seq: Sequence) -> None:
        self.waiting.append(seq)

    @property
    def has_work(self) -> bool:
        return bool(self.waiting or self.running)

    def _chunk(self, seq: Sequence, budget: int) -> int:
        want = seq.num_uncomputed_tokens
        if not self.config.enable_chunked_prefill:
            return want if want <= budget else 0
        return min(want, self.config.chunk_size, max(budget, 0))

    def _preempt(self, victim: Sequence, out: SchedulerOutput) -> int:
        refund = sum(n for s, n in out.scheduled if s is victim)
        out.scheduled = [(s, n) for s, n in out.scheduled if s is not victim]
        self.running.remove(victim)
        self.manager.free(victim.seq_id)
        victim.reset_for_recompute()
        self.waiting.appendleft(victim)
        out.preempted.append(victim)
        return refund

    def _reserve(self, seq: Sequence, count: int, out: SchedulerOutput) -> int | None:
        """Allocate pages for ``count`` more tokens of a running sequence, preempting
        newer sequences if needed. Returns the token budget refunded by preemption, or
        None if even preempting everyone else cannot make room."""
        refund = 0
        while True:
            try:
                self.manager.allocate(seq.seq_id, seq.num_computed_tokens + count)
                return refund
            except OutOfBlocks:
                victim = next((s for s in reversed(self.running) if s is not seq), None)
                if victim is None:
                    return None
                refund += self._preempt(victim, out)

    def schedule(self) -> SchedulerOutput:
        out = SchedulerOutput()
        budget = self.config.max_batched_tokens
        decoding = [s for s in self.running if s.is_decoding()]
        prefilling = [s for s in self.running if not s.is_decoding()]
        for group in (decoding, prefilling):
            for seq in group:
                if seq not in self.running:
                    continue  # preempted by an earlier sequence this iteration
                n = 1 if seq.is_decoding() else self._chunk(seq, budget)
                if n == 0 or budget < n:
                    continue
                refund = self._reserve(seq, n, out)
                if refund is None:
                    raise OutOfBlocks(
                        f"sequence {seq.seq_id} cannot fit {seq.num_computed_tokens + n} tokens "
                        f"in a pool of {self.manager.num_blocks} blocks")
                budget += refund
                out.scheduled.append((seq, n))
                budget -= n
        while self.waiting and len(self.running) < self.config.max_sequences and budget > 0:
            seq = self.waiting[0]
            if seq in out.preempted:
                # Readmitting a victim in the iteration that evicted it lets two long
                # prompts evict each other forever (each restarting from token zero);
                # it waits one iteration while the sequence that evicted it advances.
                break
            n = self._chunk(seq, budget)
            if n == 0:
                break
            if self.manager.blocks_needed(seq.seq_id, seq.num_computed_tokens + n) > \
                    self.manager.num_free_blocks:
                break
            self.waiting.popleft()
            self.manager.allocate(seq.seq_id, seq.num_computed_tokens + n)
            self.running.append(seq)
            out.scheduled.append((seq, n))
            budget -= n
        if not out.scheduled and self.has_work:
            raise OutOfBlocks(
                f"nothing can run: {len(self.running)} running, {len(self.waiting)} waiting, "
                f"{self.manager.num_free_blocks} of {self.manager.num_blocks} blocks free")
        return out

    def commit(self, out: SchedulerOutput, tokens: list[int]) -> list[Sequence]:
        """Advance every scheduled sequence; those that reached the end of their tokens
        take their sampled token; finished ones free their pages."""
        if len(tokens) != len(out.scheduled):
            raise ValueError(f"{len(tokens)} tokens for {len(out.scheduled)} sequences")
        for (seq, n), token in zip(out.scheduled, tokens):
            seq.num_computed_tokens += n
            if seq.num_computed_tokens == len(seq):
                seq.output.append(int(token))
        done = [s for s in self.running if s.is_done()]
        for seq in done:
            self.running.remove(seq)
            self.manager.free(seq.seq_id)
            self.finished.append(seq)
        return done
