"""Dense-cache grouped-query attention on the CPU (test infrastructure only).

Restates the reference's ``scaled_dot_product_attention_grouped``
(mini_vllm/attention.py:95-158) with its offset-causal mask (``causal_mask``,
attention.py:68-92: query i of L may see key j of S iff j <= S - L + i) and the
max-subtracted softmax (basics.py:44-65), for q ``B x H_q x L x D`` against k, v
``B x H_k x S x D`` (any strides), query head h reading kv head h // (H_q / H_k). This
is what the reference's dense kernels compute (csrc/decode_attention.cu: L = 1, every
key visible; csrc/flash_prefill.cu: L > 1, causal) and what ``ops.attention`` serves.

Computed in ``compute_dtype`` (fp64 by default) from inputs upcast exactly.

Pinned by tests/test_oracle.py: it equals the paged oracle (itself pinned by the
golden fixtures) on the same keys laid out as pages; one visible key returns that
key's value exactly; all-equal scores return the mean of the visible values.
"""

from __future__ import annotations

import math

import torch

__all__ = ["dense_attention"]


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = True,
                    scale: float | None = None,
                    compute_dtype: torch.dtype = torch.float64) -> torch.Tensor:
    """``B x H_q x L x D`` attention output in ``compute_dtype`` (on the CPU)."""
    b, hq, L, d = q.shape
    hk, s = k.shape[1], k.shape[2]
    if hq % hk:
        raise ValueError(f"H_q ({hq}) must be a multiple of H_k ({hk})")
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    qf = q.detach().cpu().to(compute_dtype)
    kf = k.detach().cpu().to(compute_dtype).repeat_interleave(hq // hk, dim=1)
    vf = v.detach().cpu().to(compute_dtype).repeat_interleave(hq // hk, dim=1)
    scores = (qf @ kf.transpose(-1, -2)) * scale
    if causal:
        rows = torch.arange(L).unsqueeze(1)
        cols = torch.arange(s).unsqueeze(0)
        scores = scores.masked_fill(cols > rows + (s - L), float("-inf"))
    scores = scores - scores.amax(dim=-1, keepdim=True)
    p = scores.exp()
    return (p / p.sum(dim=-1, keepdim=True)) @ vf
