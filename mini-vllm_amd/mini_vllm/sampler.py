"""Greedy, temperature, top-k and top-p sampling on the device (reference
mini_vllm/sampler.py:71-148: the same parameters, rules and order of operations).

Per-row parameters, one batched pass: row r may be greedy (``temperature == 0``)
beside a row with ``temperature=1.2, top_p=0.9``. The distribution a row is drawn
from, as the reference defines it:

  1. scale the logits by 1 / temperature (fp32);
  2. softmax;
  3. keep, in descending probability order, the ranks below top_k (0: all) whose
     probability mass strictly before them is below top_p (1: all), and always the
     first; both rules together keep the shorter prefix (the mass is summed in
     float64 here);
  4. renormalise; greedy rows are the one-hot of their argmax.

How it runs here: the whole batch stays on the device and nothing is read back by
the host. Greedy-only batches never build probabilities (the argmax kernel,
``ops.argmax``); batches without truncation take a softmax without sorting; only rows
that truncate pay for a sort of the vocabulary, which is stable, so equal
probabilities keep vocabulary order (lower token id first) and the kept set is
deterministic. Draws take a ``torch.Generator`` (on the logits' device) and are
reproducible under it.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import torch

from mini_vllm.kernels import ops

__all__ = ["SamplingParams", "sample", "sampling_probabilities"]


@dataclass(frozen=True)
class SamplingParams:
    """One request's sampling configuration (reference sampler.py:25-48).
    ``temperature=0`` is greedy; ``top_k=0`` and ``top_p=1.0`` disable truncation."""

    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 1.0

    def __post_init__(self) -> None:
        if self.temperature < 0:
            raise ValueError(f"temperature must be >= 0, got {self.temperature}")
        if self.top_k < 0:
            raise ValueError(f"top_k must be >= 0, got {self.top_k}")
        if not 0.0 < self.top_p <= 1.0:
            raise ValueError(f"top_p must be in (0, 1], got {self.top_p}")

    @property
    def is_greedy(self) -> bool:
        return self.temperature == 0.0

    @property
    def truncates(self) -> bool:
        return not self.is_greedy and (self.top_k > 0 or self.top_p < 1.0)


GREEDY = SamplingParams(temperature=0.0)


def _rows(params: SamplingParams | Sequence[SamplingParams], batch: int) -> list[SamplingParams]:
    rows = [params] * batch if isinstance(params, SamplingParams) else list(params)
    if len(rows) != batch:
        raise ValueError(f"got {len(rows)} sampling params for a batch of {batch}")
    return rows


def _columns(rows: list[SamplingParams], device) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Temperature (1 on greedy rows: those are replaced by their one-hot), top_k (the
    vocabulary size when disabled) and top_p as ``B x 1`` columns, one host-to-device
    copy."""
    host = torch.tensor([[r.temperature if r.temperature > 0 else 1.0, float(r.top_k), r.top_p]
                         for r in rows], dtype=torch.float64)
    cols = host.to(device, non_blocking=True)
    return cols[:, :1].float(), cols[:, 1:2].long(), cols[:, 2:3].float()


def _truncated(scaled: torch.Tensor, top_k: torch.Tensor, top_p: torch.Tensor) -> torch.Tensor:
    """Steps 2-4 on rows that truncate: probabilities in vocabulary order."""
    vocab = scaled.shape[1]
    descending, order = scaled.sort(dim=-1, descending=True, stable=True)
    probs = descending.softmax(dim=-1)
    rank = torch.arange(vocab, device=scaled.device).unsqueeze(0)
    k = torch.where(top_k == 0, torch.full_like(top_k, vocab), top_k)
    # the mass before each rank, accumulated in float64 (an fp32 running sum over a
    # 150K-entry vocabulary drifts by ~1e-5, the size of a tail token's probability)
    p64 = probs.double()
    keep = (rank < k) & (((p64.cumsum(dim=-1) - p64) < top_p.double()) | (top_p >= 1.0))
    keep[:, 0] = True
    kept = probs * keep
    kept = kept / kept.sum(dim=-1, keepdim=True)
    return torch.zeros_like(kept).scatter_(dim=-1, index=order, src=kept)


def sampling_probabilities(logits: torch.Tensor,
                           params: SamplingParams | Sequence[SamplingParams]) -> torch.Tensor:
    """``B x V`` logits -> the ``B x V`` fp32 distribution each row is drawn from (rows
    sum to 1; greedy rows one-hot). Reference sampler.py:71-124."""
    if logits.ndim != 2:
        raise ValueError(f"expected B x V logits, got shape {tuple(logits.shape)}")
    batch, _ = logits.shape
    rows = _rows(params, batch)
    use_cuda = logits.is_cuda
    greedy = [r.is_greedy for r in rows]
    result = torch.empty(logits.shape, dtype=torch.float32, device=logits.device)
    if not all(greedy):
        temperature, top_k, top_p = _columns(rows, logits.device)
        scaled = logits.float() / temperature
        trunc = [r.truncates for r in rows]
        if any(trunc):
            if all(trunc):
                result = _truncated(scaled, top_k, top_p)
            else:
                idx = torch.tensor([i for i, t in enumerate(trunc) if t], device=logits.device)
                result = scaled.softmax(dim=-1)
                result[idx] = _truncated(scaled[idx], top_k[idx], top_p[idx])
        else:
            result = scaled.softmax(dim=-1)
    if any(greedy):
        idx = torch.tensor([i for i, g in enumerate(greedy) if g], device=logits.device)
        best = ops.argmax(logits[idx], use_cuda=use_cuda)
        one_hot = torch.zeros(len(idx), logits.shape[1], dtype=torch.float32, device=logits.device)
        one_hot.scatter_(1, best.unsqueeze(1), 1.0)
        result[idx] = one_hot
    return result


def sample(logits: torch.Tensor,
           params: SamplingParams | Sequence[SamplingParams] = SamplingParams(),
           generator: torch.Generator | None = None) -> torch.Tensor:
    """One token per row (int64, on the logits' device). Greedy rows are their argmax
    and use no randomness; the others are one multinomial draw each from
    :func:`sampling_probabilities`, reproducible under ``generator``. Reference
    sampler.py:127-148."""
    if logits.ndim != 2:
        raise ValueError(f"expected B x V logits, got shape {tuple(logits.shape)}")
    rows = _rows(params, logits.shape[0])
    use_cuda = logits.is_cuda
    if all(r.is_greedy for r in rows):
        return ops.argmax(logits, use_cuda=use_cuda)
    probs = sampling_probabilities(logits, rows)
    tokens = torch.multinomial(probs, num_samples=1, generator=generator).squeeze(1)
    greedy = [i for i, r in enumerate(rows) if r.is_greedy]
    if greedy:
        idx = torch.tensor(greedy, device=logits.device)
        tokens[idx] = ops.argmax(logits[idx], use_cuda=use_cuda)
    return tokens
