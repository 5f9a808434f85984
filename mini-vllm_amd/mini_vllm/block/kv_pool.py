"""The paged KV pool (reference block/kv_pool.py:50-155).

One tensor per K and V shaped ``num_layers x num_blocks x P x H_k x D``, so one layer's
view is exactly the ``num_blocks x P x H_k x D`` pool the paged-attention kernels walk
(``slot = block * P + offset``), and a flat ``num_slots x H_k x D`` view of it is free.
A ``float8_e4m3fn`` pool (not in the reference) also holds fp32 scales
``num_layers x num_blocks x H_k`` for K and for V, maintained by the quantising write.
"""

from __future__ import annotations

import torch

from mini_vllm.kernels import ops

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
        self.k_scales = self.v_scales = None
        if dtype == torch.float8_e4m3fn:
            scale_shape = (num_layers, num_blocks, num_kv_heads)
            self.k_scales = torch.zeros(scale_shape, dtype=torch.float32, device=device)
            self.v_scales = torch.zeros(scale_shape, dtype=torch.float32, device=device)

    @property
    def is_fp8(self) -> bool:
        return self.k_scales is not None

    def layer_scales(self, layer: int) -> tuple[torch.Tensor | None, torch.Tensor | None]:
        """(k_scale, v_scale) of one layer for a float8 pool, else (None, None)."""
        if not self.is_fp8:
            return None, None
        return self.k_scales[layer], self.v_scales[layer]

    @staticmethod
    def bytes_for(num_layers: int, num_blocks: int, block_size: int, num_kv_heads: int,
                  head_dim: int, dtype: torch.dtype) -> int:
        elt = torch.empty((), dtype=dtype).element_size()
        scales = 2 * num_layers * num_blocks * num_kv_heads * 4 if dtype == torch.float8_e4m3fn else 0
        return 2 * num_layers * num_blocks * block_size * num_kv_heads * head_dim * elt + scales

    def layer_keys(self, layer: int) -> torch.Tensor:
        return self.keys[layer]

    def layer_values(self, layer: int) -> torch.Tensor:
        return self.values[layer]

    def write(self, layer: int, slot_mapping: torch.Tensor, key: torch.Tensor,
              value: torch.Tensor, use_cuda: bool = False) -> None:
        """Scatter ``T x H_k x D`` keys/values to their slots (``ops.kv_write``: one
        kernel launch for K and V with ``use_cuda``, the reference's ``index_copy_``
        pair otherwise). Slot values are not read back (that would be a device-to-host
        sync per layer); the block manager bounded them on the host."""
        expected = (slot_mapping.shape[0], self.num_kv_heads, self.head_dim)
        if tuple(key.shape) != expected or key.shape != value.shape:
            raise ValueError(f"expected keys and values shaped {expected}, got "
                             f"{tuple(key.shape)} and {tuple(value.shape)}")
        k_scale, v_scale = self.layer_scales(layer)
        ops.kv_write(self.keys[layer], self.values[layer], key, value, slot_mapping,
                     use_cuda=use_cuda, k_scale=k_scale, v_scale=v_scale)
