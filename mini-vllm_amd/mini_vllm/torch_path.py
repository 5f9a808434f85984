"""The readable PyTorch path of each hot-path op: what ``use_cuda=False`` selects.

These are the reference's PyTorch expressions, restated (they are also what its
kernels are specified against): ``rms_norm`` (layer_norm.py:18-46), ``apply_rope``
(positional_encoding.py:36-62), ``silu`` (basics.py:39-41), and gather-then-dense
paged attention (paged_attention.py:36-110 over attention.py:95-158, with the softmax
of basics.py:44-65: fp32 inside, returned in the input dtype).

They run on whatever device their inputs are on. They are not a fallback for the
kernels -- ``ops`` never routes a ``use_cuda=True`` call here -- and they are not the
test oracle either: parity tests compare the kernels with ``oracle/``, an independent
restatement.
"""

from __future__ import annotations

import math

import torch

__all__ = [
    "apply_rope",
    "dequantize_fp8_pool",
    "paged_attention_gathered",
    "rms_norm",
    "rope_tables",
    "silu",
    "softmax",
]


def silu(x: torch.Tensor) -> torch.Tensor:
    return x * torch.sigmoid(x)


def softmax(x: torch.Tensor, dim: int = -1) -> torch.Tensor:
    """Max-subtracted softmax computed in fp32, returned in ``x``'s dtype."""
    x32 = x.float()
    e = torch.exp(x32 - x32.amax(dim=dim, keepdim=True))
    return (e / e.sum(dim=dim, keepdim=True)).to(x.dtype)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``weight * T(x * rsqrt(mean(x^2) + eps))`` with the statistic in fp32."""
    x32 = x.float()
    inv = torch.rsqrt(x32.pow(2).mean(dim=-1, keepdim=True) + eps)
    return weight * (x32 * inv).to(x.dtype)


def rope_tables(head_dim: int, max_seq_len: int, theta: float = 1_000_000.0,
                device: torch.device | str | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 ``max_seq_len x D`` cos/sin tables, angles duplicated across the halves
    (positional_encoding.py:97-110)."""
    if head_dim % 2:
        raise ValueError(f"head_dim must be even for RoPE, got {head_dim}")
    exponents = torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim
    inv_freq = 1.0 / (theta**exponents)
    angles = torch.outer(torch.arange(max_seq_len, dtype=torch.float32, device=device), inv_freq)
    angles = torch.cat((angles, angles), dim=-1)
    return angles.cos(), angles.sin()


def apply_rope(x: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor,
               sin: torch.Tensor) -> torch.Tensor:
    """Rotate halves at ``positions``: ``x*cos + rotate_half(x)*sin`` in fp32."""
    c = cos.to(x.device)[positions].unsqueeze(-2)
    s = sin.to(x.device)[positions].unsqueeze(-2)
    x32 = x.float()
    half = x.shape[-1] // 2
    rotated = torch.cat((-x32[..., half:], x32[..., :half]), dim=-1)
    return (x32 * c + rotated * s).to(x.dtype)


def dequantize_fp8_pool(pool: torch.Tensor, scales: torch.Tensor,
                        dtype: torch.dtype) -> torch.Tensor:
    """``fp8 value * scale[block, kv_head]`` for a ``num_blocks x P x H_k x D`` pool."""
    return (pool.float() * scales.float()[:, None, :, None]).to(dtype)


def paged_attention_gathered(q: torch.Tensor, key_pool: torch.Tensor, value_pool: torch.Tensor,
                             block_tables: torch.Tensor, cu_seqlens_q: torch.Tensor,
                             context_lens: torch.Tensor, scale: float | None = None,
                             k_scale: torch.Tensor | None = None,
                             v_scale: torch.Tensor | None = None) -> torch.Tensor:
    """Per sequence: gather its pages, then dense causal GQA attention with offset S - L."""
    if q.dim() != 3:
        raise ValueError(f"expected q shaped T x H_q x D, got {tuple(q.shape)}")
    if key_pool.dim() != 4 or key_pool.shape != value_pool.shape:
        raise ValueError(
            "expected matching pools shaped num_blocks x P x H_k x D, got "
            f"{tuple(key_pool.shape)} and {tuple(value_pool.shape)}"
        )
    if key_pool.dtype == torch.float8_e4m3fn:
        key_pool = dequantize_fp8_pool(key_pool, k_scale, q.dtype)
        value_pool = dequantize_fp8_pool(value_pool, v_scale, q.dtype)
    num_seqs = context_lens.shape[0]
    if block_tables.shape[0] != num_seqs or cu_seqlens_q.shape[0] != num_seqs + 1:
        raise ValueError("metadata disagrees on the sequence count")
    if int(cu_seqlens_q[-1]) != q.shape[0]:
        raise ValueError(f"cu_seqlens_q ends at {int(cu_seqlens_q[-1])} but q has {q.shape[0]} rows")
    block_size, num_kv_heads, head_dim = key_pool.shape[1:]
    num_q_heads = q.shape[1]
    group = num_q_heads // num_kv_heads
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    out = torch.empty_like(q)
    for s in range(num_seqs):
        start, end = int(cu_seqlens_q[s]), int(cu_seqlens_q[s + 1])
        L, S = end - start, int(context_lens[s])
        if L == 0:
            continue
        if S < L:
            raise ValueError(f"sequence {s} attends over {S} tokens but computes {L}")
        used = -(-S // block_size)
        table = block_tables[s, :used]
        if int(table.min()) < 0:
            raise ValueError(
                f"sequence {s} needs {used} blocks for {S} tokens but its table is padded there"
            )
        ids = table.to(dtype=torch.int64, device=key_pool.device)
        k = key_pool.index_select(0, ids).reshape(-1, num_kv_heads, head_dim)[:S]
        v = value_pool.index_select(0, ids).reshape(-1, num_kv_heads, head_dim)[:S]
        k = k.permute(1, 0, 2).unsqueeze(1)                       # H_k x 1 x S x D
        v = v.permute(1, 0, 2).unsqueeze(1)
        qs = q[start:end].permute(1, 0, 2).reshape(num_kv_heads, group, L, head_dim)
        scores = (qs @ k.transpose(-2, -1).contiguous()) * scale   # H_k x G x L x S
        rows = torch.arange(L, device=q.device).unsqueeze(1)
        cols = torch.arange(S, device=q.device).unsqueeze(0)
        mask = torch.zeros(L, S, dtype=scores.dtype, device=q.device).masked_fill(
            cols > rows + (S - L), float("-inf"))
        probs = softmax(scores + mask, dim=-1)
        attended = (probs @ v).reshape(num_q_heads, L, head_dim)
        out[start:end] = attended.permute(1, 0, 2)
    return out
