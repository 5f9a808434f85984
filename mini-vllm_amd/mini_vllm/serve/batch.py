"""One ragged forward pass (reference serve/batch.py:100-347).

Sequences of different phases share one flattened token axis: ``cu_seqlens_q`` gives
each sequence's query rows, ``seq_lens`` (L) how many tokens it computes now,
``context_lens`` (S) how many it attends over, ``slot_mapping`` where each new K/V row
goes and ``block_tables`` its pages (right-padded with -1). ``max_query_len`` and
``max_context_len`` are host integers, so no kernel launch needs a device read.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

__all__ = ["ForwardBatch", "PADDING_BLOCK"]

PADDING_BLOCK = -1


@dataclass(frozen=True)
class ForwardBatch:
    input_ids: torch.Tensor      # int64 [T]
    positions: torch.Tensor      # int64 [T]
    cu_seqlens_q: torch.Tensor   # int32 [N + 1]
    seq_lens: torch.Tensor       # int32 [N]
    context_lens: torch.Tensor   # int32 [N]
    slot_mapping: torch.Tensor   # int32 [T]
    block_tables: torch.Tensor   # int32 [N, widest table]
    last_row_indices: torch.Tensor  # int64 [N], each sequence's last computed row
    max_query_len: int
    max_context_len: int
    seq_ids: tuple[int, ...]

    @property
    def num_sequences(self) -> int:
        return len(self.seq_ids)

    @property
    def total_tokens(self) -> int:
        return int(self.input_ids.shape[0])

    @classmethod
    def from_scheduled(cls, scheduled, manager, device: torch.device | str = "cpu") -> "ForwardBatch":
        """From ``(sequence, tokens to compute now)`` pairs whose blocks are allocated."""
        ids, positions, offsets, lens, contexts, slots, tables, seq_ids = [], [], [0], [], [], [], [], []
        for seq, count in scheduled:
            start = seq.num_computed_tokens
            if count < 1 or start + count > len(seq):
                raise ValueError(f"sequence {seq.seq_id}: cannot compute {count} tokens from {start}")
            ids.extend(seq.tokens(start, count))
            positions.extend(range(start, start + count))
            offsets.append(offsets[-1] + count)
            lens.append(count)
            contexts.append(start + count)
            slots.extend(manager.slots(seq.seq_id, start, count))
            tables.append(manager.table(seq.seq_id))
            seq_ids.append(seq.seq_id)
        widest = max(len(t) for t in tables)
        padded = [t + [PADDING_BLOCK] * (widest - len(t)) for t in tables]
        i32 = dict(dtype=torch.int32, device=device)
        i64 = dict(dtype=torch.int64, device=device)
        return cls(
            input_ids=torch.tensor(ids, **i64),
            positions=torch.tensor(positions, **i64),
            cu_seqlens_q=torch.tensor(offsets, **i32),
            seq_lens=torch.tensor(lens, **i32),
            context_lens=torch.tensor(contexts, **i32),
            slot_mapping=torch.tensor(slots, **i32),
            block_tables=torch.tensor(padded, **i32),
            last_row_indices=torch.tensor(offsets[1:], **i64) - 1,
            max_query_len=max(lens),
            max_context_len=max(contexts),
            seq_ids=tuple(seq_ids),
        )
