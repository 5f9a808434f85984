"""Gather-then-dense paged attention on the CPU (test infrastructure only).

Restates the reference's oracle ``paged_attention_gathered``
(mini_vllm/paged_attention.py:36-110): per sequence, resolve the logical key
positions 0..S-1 to physical slots through the block table (slot = table[j // P] * P
+ j % P, csrc/paged_attention.cu:87-93), gather those keys and values, then run
grouped-query attention with the offset-causal mask ``j <= S - L + i``
(attention.py:68-92, 95-158) and a max-subtracted softmax (basics.py:44-65).

Everything is computed in ``compute_dtype`` (fp32 by default, fp64 on request) from
inputs upcast exactly, so for bf16/fp16/fp8 inputs this is the "fp32 oracle" the
tolerances are stated against. fp8 pools are dequantised first: value * scale of its
(block, kv head).

Pinned by: tests/golden/ (fixtures from brute.c in float64), and the known answers in
tests/test_oracle.py (one visible key returns that key's value exactly; a reversed
physical layout gives the same result; each sequence of a mixed batch equals its run
alone; padding is never read; closed-form two-key softmax).
"""

from __future__ import annotations

import math

import torch

__all__ = ["dequantize", "paged_attention", "slots_for"]


def slots_for(table_row: torch.Tensor, context_len: int, block_size: int) -> torch.Tensor:
    """Physical slot of each logical key position 0..context_len-1 of one sequence."""
    positions = torch.arange(context_len, dtype=torch.int64)
    needed = -(-context_len // block_size)
    if needed > table_row.shape[0]:
        raise ValueError(
            f"needs {needed} blocks for {context_len} tokens but the table holds "
            f"{table_row.shape[0]}: past the end of the table"
        )
    blocks = table_row.to(torch.int64)[positions // block_size]
    if context_len and int(blocks.min()) < 0:
        raise ValueError(
            f"needs {-(-context_len // block_size)} blocks for {context_len} tokens but the "
            "table is padded there"
        )
    return blocks * block_size + positions % block_size


def dequantize(pool: torch.Tensor, scales: torch.Tensor | None,
               compute_dtype: torch.dtype) -> torch.Tensor:
    """fp8 -> value * scale[block, kv_head]; other dtypes are upcast exactly."""
    x = pool.to(torch.float32).to(compute_dtype)
    if pool.dtype == torch.float8_e4m3fn:
        if scales is None:
            raise ValueError("an fp8 pool needs its per-(block, kv head) scales")
        x = x * scales.to(compute_dtype)[:, None, :, None]
    return x


def paged_attention(q: torch.Tensor, key_pool: torch.Tensor, value_pool: torch.Tensor,
                    block_tables: torch.Tensor, cu_seqlens_q: torch.Tensor,
                    context_lens: torch.Tensor, scale: float | None = None,
                    k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None,
                    compute_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """``T x H_q x D`` output in ``compute_dtype``; all inputs are read on the CPU.

    fp8 rows are dequantised after the gather: value * scale[block, kv head]
    (``rows * scales[slot // P]`` multiplies each row's H_k heads by their own scale).
    """
    q = q.detach().cpu()
    num_blocks, block_size, num_kv_heads, head_dim = key_pool.shape
    keys = key_pool.detach().cpu().reshape(num_blocks * block_size, num_kv_heads, head_dim)
    values = value_pool.detach().cpu().reshape(num_blocks * block_size, num_kv_heads, head_dim)
    ks = None if k_scale is None else k_scale.detach().cpu()
    vs = None if v_scale is None else v_scale.detach().cpu()
    tables = block_tables.detach().cpu()
    cu = [int(v) for v in cu_seqlens_q.cpu()]
    ctx = [int(v) for v in context_lens.cpu()]
    num_q_heads = q.shape[1]
    if num_q_heads % num_kv_heads:
        raise ValueError(f"H_q ({num_q_heads}) must be a multiple of H_k ({num_kv_heads})")
    group = num_q_heads // num_kv_heads
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)

    def gathered(pool: torch.Tensor, scales: torch.Tensor | None, slots: torch.Tensor):
        rows = pool.index_select(0, slots).to(torch.float32).to(compute_dtype)
        if pool.dtype == torch.float8_e4m3fn:
            if scales is None:
                raise ValueError("an fp8 pool needs its per-(block, kv head) scales")
            rows = rows * scales.to(compute_dtype)[slots // block_size].unsqueeze(-1)
        return rows

    out = torch.zeros(q.shape, dtype=compute_dtype)
    for s, S in enumerate(ctx):
        start, end = cu[s], cu[s + 1]
        L = end - start
        if L == 0:
            continue
        if S < L:
            raise ValueError(f"sequence {s} attends over {S} tokens but computes {L}")
        slots = slots_for(tables[s], S, block_size)
        k = gathered(keys, ks, slots).permute(1, 0, 2)                   # H_k x S x D
        v = gathered(values, vs, slots).permute(1, 0, 2)
        qs = q[start:end].to(compute_dtype).permute(1, 0, 2)             # H_q x L x D
        qs = qs.reshape(num_kv_heads, group, L, head_dim)
        scores = torch.matmul(qs, k.unsqueeze(1).transpose(-1, -2)) * scale  # H_k x G x L x S
        i = torch.arange(L).unsqueeze(1)
        j = torch.arange(S).unsqueeze(0)
        scores = scores.masked_fill(j > (S - L) + i, float("-inf"))
        scores = scores - scores.amax(dim=-1, keepdim=True)
        weights = torch.exp(scores)
        weights = weights / weights.sum(dim=-1, keepdim=True)
        attended = torch.matmul(weights, v.unsqueeze(1))                  # H_k x G x L x D
        out[start:end] = attended.reshape(num_q_heads, L, head_dim).permute(1, 0, 2)
    return out
