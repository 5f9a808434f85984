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
    "kv_write",
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


def _pow2_ceil(t: torch.Tensor) -> torch.Tensor:
    """Least power of two >= t (float32, t >= 0; 0 stays 0)."""
    b = t.float().contiguous().view(torch.int32)
    up = torch.where((b & 0x7FFFFF) == 0, b, (b & 0x7F800000) + 0x800000)
    return up.view(torch.float32)


def kv_write(key_pool: torch.Tensor, value_pool: torch.Tensor, key: torch.Tensor,
             value: torch.Tensor, slot_mapping: torch.Tensor, *,
             k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None) -> None:
    """Scatter ``T x H_k x D`` keys/values into one layer's pools at ``slot_mapping``.

    Same dtype: the reference's ``index_copy_`` pair (block/kv_pool.py:148-155), with
    negative slots skipped. A ``float8_e4m3fn`` pool follows the library's quantising
    policy (include/minivllm_hip.h, ``mvllm_kv_write``) run by run in torch, reading
    the slots on the host (this path syncs; the kernel does not).
    """
    nb, bs, hk, d = key_pool.shape
    keep = slot_mapping >= 0
    if key_pool.dtype != torch.float8_e4m3fn:
        index = slot_mapping[keep].to(torch.int64)
        key_pool.view(nb * bs, hk, d).index_copy_(0, index, key[keep].to(key_pool.dtype))
        value_pool.view(nb * bs, hk, d).index_copy_(0, index, value[keep].to(value_pool.dtype))
        return
    slots = slot_mapping.tolist()
    t = 0
    while t < len(slots):
        if slots[t] < 0:
            t += 1
            continue
        block, row0 = divmod(slots[t], bs)
        n = 1
        while (t + n < len(slots) and slots[t + n] >= 0 and slots[t + n] // bs == block
               and slots[t + n] % bs == row0 + n):
            n += 1
        for pool, scales, x in ((key_pool, k_scale, key), (value_pool, v_scale, value)):
            rows = x[t:t + n].float()                                   # n x H_k x D
            amax = rows.abs().amax(dim=(0, 2))                          # H_k
            old = torch.zeros_like(amax) if row0 == 0 else scales[block].clone()
            s = torch.maximum(old, _pow2_ceil(amax / 448.0))
            grow = (old > 0) & (s > old)
            if row0 > 0 and bool(grow.any()):
                prev = pool[block, :row0].float()                       # row0 x H_k x D
                re = ((prev * old[None, :, None]) / s[None, :, None]).clamp(-448.0, 448.0)
                pool[block, :row0] = torch.where(grow[None, :, None],
                                                 re.to(torch.float8_e4m3fn), pool[block, :row0])
            safe = torch.where(s > 0, s, torch.ones_like(s))
            enc = (rows / safe[None, :, None]).clamp(-448.0, 448.0)
            enc = torch.where((s > 0)[None, :, None], enc, torch.zeros_like(enc))
            pool[block, row0:row0 + n] = enc.to(torch.float8_e4m3fn)
            scales[block] = s
        t += n


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
    fp8 = key_pool.dtype == torch.float8_e4m3fn
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
        k = key_pool.index_select(0, ids)
        v = value_pool.index_select(0, ids)
        if fp8:  # dequantised after the gather: only this sequence's pages
            k = dequantize_fp8_pool(k, k_scale.index_select(0, ids), q.dtype)
            v = dequantize_fp8_pool(v, v_scale.index_select(0, ids), q.dtype)
        k = k.reshape(-1, num_kv_heads, head_dim)[:S]
        v = v.reshape(-1, num_kv_heads, head_dim)[:S]
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


def interleave_gate_up(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """Gate and up projection weights (``I x E`` each) as one ``2I x E`` matrix with their
    rows interleaved in groups of 16: rows 32j .. 32j+15 are gate rows 16j .. 16j+15, the
    next 16 the same up rows (the layout of ``linear_swiglu``)."""
    i, e = gate.shape
    if up.shape != gate.shape or i % 16:
        raise ValueError("gate and up must share a shape with a multiple of 16 rows")
    return torch.stack((gate.view(i // 16, 16, e), up.view(i // 16, 16, e)), dim=1).reshape(2 * i, e)


def split_gate_up(y: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Undo the column interleave of ``x @ interleave_gate_up(gate, up).T``."""
    m, n = y.shape
    v = y.view(m, n // 32, 2, 16)
    return v[:, :, 0, :].reshape(m, n // 2), v[:, :, 1, :].reshape(m, n // 2)


def pack_fragments(w: torch.Tensor) -> torch.Tensor:
    """``w`` (N x K) in the skinny projection kernels' fragment order, flat: rows padded
    with zeros to a multiple of 32, then for each 32-row tile t and 16-element k-step s
    the 64 eight-element pieces l = 32 h + r holding w[32 t + r, 16 s + 8 h : 16 s + 8 h + 8]
    (piece index (t * K/16 + s) * 64 + l). The layout of ``mvllm_linear_pack``."""
    n, k = w.shape
    if k % 16:
        raise ValueError("K must be a multiple of 16")
    tiles = -(-n // 32)
    padded = torch.zeros((tiles * 32, k), dtype=w.dtype, device=w.device)
    padded[:n] = w
    return padded.view(tiles, 32, k // 16, 2, 8).permute(0, 2, 3, 1, 4).reshape(-1)
