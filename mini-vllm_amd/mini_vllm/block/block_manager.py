"""Host-side page bookkeeping (reference block/block_pool.py, block_table.py,
block_manager.py): a free list of physical blocks, one table of block ids per sequence,
and the slot arithmetic ``slot = table[j // P] * P + j % P``.

Everything here is host integers; nothing reads the GPU.
"""

from __future__ import annotations

from collections import deque

import torch

from mini_vllm.block.kv_pool import PagedKvPool

__all__ = ["BlockManager", "OutOfBlocks"]


class OutOfBlocks(RuntimeError):
    """The pool has too few free blocks for a request (reference block_pool.py:36-45)."""


class BlockManager:
    def __init__(self, num_blocks: int, block_size: int, num_layers: int, num_kv_heads: int,
                 head_dim: int, dtype: torch.dtype = torch.bfloat16,
                 device: torch.device | str = "cpu") -> None:
        if block_size < 1 or block_size & (block_size - 1):
            raise ValueError(f"block_size must be a power of two, got {block_size}")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.kv = PagedKvPool(num_layers, num_blocks, block_size, num_kv_heads, head_dim,
                              dtype, device)
        self._free: deque[int] = deque(range(num_blocks))
        self._tables: dict[int, list[int]] = {}
        self._changes = 0  # bumped on every table change: (seq_id, version) names a table
        self._versions: dict[int, int] = {}

    @property
    def num_free_blocks(self) -> int:
        return len(self._free)

    def table(self, seq_id: int) -> list[int]:
        return self._tables.get(seq_id, [])

    def blocks_needed(self, seq_id: int, context: int) -> int:
        """Extra blocks a sequence needs to hold ``context`` tokens."""
        have = len(self._tables.get(seq_id, ()))
        return max(0, -(-context // self.block_size) - have)

    def allocate(self, seq_id: int, context: int) -> None:
        """Grow the sequence's table to cover ``context`` tokens (FIFO free list)."""
        need = self.blocks_needed(seq_id, context)
        if need > len(self._free):
            raise OutOfBlocks(f"sequence {seq_id} needs {need} blocks, {len(self._free)} free")
        table = self._tables.setdefault(seq_id, [])
        for _ in range(need):
            table.append(self._free.popleft())
        if need:
            self._bump(seq_id)

    def _bump(self, seq_id: int) -> None:
        self._changes += 1
        self._versions[seq_id] = self._changes

    def version(self, seq_id: int) -> int:
        """A number that changes whenever the sequence's block table does (never reused),
        so a copy of the table can be kept until it changes."""
        return self._versions.get(seq_id, 0)

    def slots(self, seq_id: int, start: int, count: int) -> list[int]:
        """Physical slots of logical positions ``start .. start + count - 1``."""
        table = self._tables[seq_id]
        p = self.block_size
        if -(-(start + count) // p) > len(table):
            raise ValueError(f"sequence {seq_id}: positions up to {start + count} exceed its "
                             f"{len(table)} blocks")
        return [table[j // p] * p + j % p for j in range(start, start + count)]

    def free(self, seq_id: int) -> None:
        self._free.extend(self._tables.pop(seq_id, []))
        self._bump(seq_id)

    def check_no_leaks(self) -> None:
        held = sum(len(t) for t in self._tables.values())
        if held + len(self._free) != self.num_blocks or len(set(self._free)) != len(self._free):
            raise AssertionError(f"block leak: {held} held + {len(self._free)} free != "
                                 f"{self.num_blocks}")
