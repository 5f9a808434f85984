"""The paged KV pool (reference block/kv_pool.py:50-155).

One tensor per K and V shaped ``num_layers x num_blocks x P x H_k x D``, so one layer's
view is exactly the ``num_blocks x P x H_k x D`` pool the paged-attention kernels walk
(``slot = block * P + offset``), and a flat ``num_slots x H_k x D`` view of it is free.
"""

from __future__ import annotations

import torch

__all__ = ["PagedKvPool"]


class PagedKvPool:
    def __init__(self, num_layers: int, num_blocks: int, block_size: int, num_kv_heads: int,
                 head_dim: int, dtype: torch.dtype = torch.bfloat16,
                 device: torch.device | str = "cpu") -> None:
        self.num_layers = num_layers
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        shape = (num_layers, num_blocks, block_size, num_kv_heads, head_dim)
        self.keys = torch.zeros(shape, dtype=dtype, device=device)
        self.values = torch.zeros(shape, dtype=dtype, device=device)

    @staticmethod
    def bytes_for(num_layers: int, num_blocks: int, block_size: int, num_kv_heads: int,
                  head_dim: int, dtype: torch.dtype) -> int:
        elt = torch.empty((), dtype=dtype).element_size()
        return 2 * num_layers * num_blocks * block_size * num_kv_heads * head_dim * elt

    def layer_keys(self, layer: int) -> torch.Tensor:
        return self.keys[layer]

    def layer_values(self, layer: int) -> torch.Tensor:
        return self.values[layer]

    def write(self, layer: int, slot_mapping: torch.Tensor, key: torch.Tensor,
              value: torch.Tensor) -> None:
        """Scatter ``T x H_k x D`` keys/values to their slots. Slot values are not read
        back (that would be a device-to-host sync per layer); the block manager bounded
        them on the host."""
        expected = (slot_mapping.shape[0], self.num_kv_heads, self.head_dim)
        if tuple(key.shape) != expected or key.shape != value.shape:
            raise ValueError(f"expected keys and values shaped {expected}, got "
                             f"{tuple(key.shape)} and {tuple(value.shape)}")
        slots = self.num_blocks * self.block_size
        flat_k = self.keys[layer].view(slots, self.num_kv_heads, self.head_dim)
        flat_v = self.values[layer].view(slots, self.num_kv_heads, self.head_dim)
        index = slot_mapping.to(device=flat_k.device, dtype=torch.int64)
        flat_k.index_copy_(0, index, key.to(self.dtype))
        flat_v.index_copy_(0, index, value.to(self.dtype))
