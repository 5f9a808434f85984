"""Paged KV memory: the pool the kernels read and the host bookkeeping that fills it."""

from mini_vllm.block.block_manager import BlockManager, OutOfBlocks
from mini_vllm.block.kv_pool import PagedKvPool

__all__ = ["BlockManager", "OutOfBlocks", "PagedKvPool"]
