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

__all__ = ["BatchStager", "ForwardBatch", "PADDING_BLOCK"]

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
    # (ids, index, prev): row i's input token is prev[index[i]] where index[i] >= 0, else
    # ids[i] (a decode graph's: the previous replay's tokens still on the device, picked
    # in the embedding launch); None: input_ids.
    input_source: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None

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


class BatchStager:
    """Builds :class:`ForwardBatch` for a GPU without waiting for it.

    ``ForwardBatch.from_scheduled`` makes eight tensors from Python lists, and each
    blocking host-to-device copy waits for every kernel already queued, so the host could
    not prepare iteration i + 1 while the GPU runs iteration i. Here the metadata is
    written into pinned host memory (one int64 and one int32 block) and copied with two
    asynchronous copies into fresh device tensors that the batch's fields are views of.
    The pinned blocks are a small ring: a block is rewritten only after the event
    recorded behind its last copy has passed.

    A decode row whose input token was sampled by the previous iteration but not yet
    read by the host (``gather``: sequence id -> row of ``prev_tokens``) takes that token
    on the device.
    """

    RING = 3

    def __init__(self, device) -> None:
        self.device = torch.device(device)
        self._ring: list[list] = [[None, None, None] for _ in range(self.RING)]  # host64, host32, event
        self._turn = 0

    def _slot(self, n64: int, n32: int):
        slot = self._ring[self._turn]
        self._turn = (self._turn + 1) % self.RING
        if slot[2] is not None:
            slot[2].synchronize()
        if slot[0] is None or slot[0].numel() < n64:
            slot[0] = torch.empty(max(n64, 4096), dtype=torch.int64, pin_memory=True)
        if slot[1] is None or slot[1].numel() < n32:
            slot[1] = torch.empty(max(n32, 16384), dtype=torch.int32, pin_memory=True)
        return slot

    def build(self, scheduled, manager, prev_tokens: torch.Tensor | None = None,
              gather: dict[int, int] | None = None) -> ForwardBatch:
        n = len(scheduled)
        counts = [count for _, count in scheduled]
        total = sum(counts)
        tables = [manager.table(seq.seq_id) for seq, _ in scheduled]
        widest = max(len(t) for t in tables)
        # int64: ids | positions | gather rows | last rows; int32: cu | lens | context |
        # slots | tables
        n64 = 3 * total + n
        n32 = (n + 1) + 2 * n + total + n * widest
        slot = self._slot(n64, n32)
        h64 = slot[0][:n64].numpy()
        h32 = slot[1][:n32].numpy()
        ids, pos, rows, last = (h64[:total], h64[total:2 * total], h64[2 * total:3 * total],
                                h64[3 * total:])
        cu, lens, ctx = h32[:n + 1], h32[n + 1:2 * n + 1], h32[2 * n + 1:3 * n + 1]
        slots = h32[3 * n + 1:3 * n + 1 + total]
        tab = h32[3 * n + 1 + total:].reshape(n, widest)
        tab.fill(PADDING_BLOCK)
        rows.fill(-1)
        cu[0] = 0
        gathered = False
        at = 0
        for i, ((seq, count), table) in enumerate(zip(scheduled, tables)):
            start = seq.num_computed_tokens
            if count < 1 or start + count > len(seq):
                raise ValueError(f"sequence {seq.seq_id}: cannot compute {count} tokens from {start}")
            row = gather.get(seq.seq_id, -1) if gather else -1
            if row >= 0 and count == 1:
                ids[at] = 0
                rows[at] = row
                gathered = True
            else:
                ids[at:at + count] = seq.tokens(start, count)
            pos[at:at + count] = range(start, start + count)
            slots[at:at + count] = manager.slots(seq.seq_id, start, count)
            at += count
            cu[i + 1] = at
            lens[i] = count
            ctx[i] = start + count
            last[i] = at - 1
            tab[i, :len(table)] = table
        d64 = torch.empty(n64, dtype=torch.int64, device=self.device)
        d32 = torch.empty(n32, dtype=torch.int32, device=self.device)
        d64.copy_(slot[0][:n64], non_blocking=True)
        d32.copy_(slot[1][:n32], non_blocking=True)
        event = torch.cuda.Event()
        event.record()
        slot[2] = event
        input_ids = d64[:total]
        if gathered:
            if prev_tokens is None:
                raise ValueError("a gathered row needs prev_tokens")
            g = d64[2 * total:3 * total]
            input_ids = torch.where(g >= 0, prev_tokens.index_select(0, g.clamp(min=0)), input_ids)
        return ForwardBatch(
            input_ids=input_ids,
            positions=d64[total:2 * total],
            cu_seqlens_q=d32[:n + 1],
            seq_lens=d32[n + 1:2 * n + 1],
            context_lens=d32[2 * n + 1:3 * n + 1],
            slot_mapping=d32[3 * n + 1:3 * n + 1 + total],
            block_tables=d32[3 * n + 1 + total:].view(n, widest),
            last_row_indices=d64[3 * total:],
            max_query_len=max(counts),
            max_context_len=int(ctx.max()),
            seq_ids=tuple(seq.seq_id for seq, _ in scheduled),
        )
