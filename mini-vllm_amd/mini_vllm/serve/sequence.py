"""One request's tokens and progress (reference serve/sequence.py).

``num_computed_tokens`` counts positions whose K/V are in the pool; the rest of
``token_ids`` is what the next passes compute. A pass that reaches the end of the
tokens yields a sampled token; a prefill chunk that stops mid-prompt yields none.
"""

from __future__ import annotations

from dataclasses import dataclass, field

from mini_vllm.sampler import GREEDY, SamplingParams

__all__ = ["Sequence"]


@dataclass(eq=False)
class Sequence:
    seq_id: int
    prompt: list[int]
    max_tokens: int
    output: list[int] = field(default_factory=list)
    num_computed_tokens: int = 0
    preemptions: int = 0
    params: SamplingParams = GREEDY  # how its tokens are drawn (reference sequence.py)

    @property
    def token_ids(self) -> list[int]:
        return self.prompt + self.output

    def __len__(self) -> int:
        return len(self.prompt) + len(self.output)

    def tokens(self, start: int, count: int) -> list[int]:
        """``token_ids[start:start + count]`` without building the whole list."""
        n = len(self.prompt)
        if start + count <= n:
            return self.prompt[start:start + count]
        if start >= n:
            return self.output[start - n:start - n + count]
        return self.prompt[start:] + self.output[:start + count - n]

    @property
    def num_uncomputed_tokens(self) -> int:
        return len(self) - self.num_computed_tokens

    def is_decoding(self) -> bool:
        """Past its prompt: one new token per pass."""
        return self.num_computed_tokens > 0 and self.num_uncomputed_tokens == 1 and bool(self.output)

    def is_done(self) -> bool:
        return len(self.output) >= self.max_tokens

    def reset_for_recompute(self) -> None:
        """Preempted: its pages are gone, so everything (prompt and output so far) is
        recomputed as a prefill when it is readmitted (reference sequence.py:198-217)."""
        self.num_computed_tokens = 0
        self.preemptions += 1
