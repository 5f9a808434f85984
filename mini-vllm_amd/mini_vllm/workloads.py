"""Seeded synthetic inputs for paged attention: the BASELINE configs and test cases.

A :class:`PagedBatch` is one call's worth of arguments to ``ops.paged_attention``:
a pool of pages, per-sequence block tables (right-padded with -1, as
``ForwardBatch`` builds them, reference serve/batch.py:122-132), ragged query rows
(``cu_seqlens_q``) and the host-side bounds ``max_query_len`` / ``max_context_len``.

Physical block ids are shuffled by default, so logical and physical order disagree
(the case the reference's kernel tests are built around,
tests/test_paged_attention_cuda.py:1-17, 44-129).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

__all__ = ["PagedBatch", "build_batch", "config_batch", "CONFIGS", "quantize_fp8_per_block"]


@dataclass
class PagedBatch:
    q: torch.Tensor
    key_pool: torch.Tensor
    value_pool: torch.Tensor
    block_tables: torch.Tensor
    cu_seqlens_q: torch.Tensor
    context_lens: torch.Tensor
    seq_lens: torch.Tensor
    max_query_len: int
    max_context_len: int
    scale: float
    k_scale: torch.Tensor | None = None
    v_scale: torch.Tensor | None = None
    contexts: list[int] = field(default_factory=list)
    query_lens: list[int] = field(default_factory=list)

    def args(self) -> tuple:
        return (self.q, self.key_pool, self.value_pool, self.block_tables, self.cu_seqlens_q,
                self.context_lens, self.seq_lens, self.max_query_len, self.max_context_len,
                self.scale)

    def kv_bytes(self) -> int:
        """Algorithmic K+V bytes of one call: every visible key row read once."""
        _, _, hk, d = self.key_pool.shape
        return 2 * sum(self.contexts) * hk * d * self.key_pool.element_size()

    def scale_bytes(self) -> int:
        if self.k_scale is None:
            return 0
        return 2 * self.k_scale.numel() * 4

    def to(self, device: torch.device | str) -> "PagedBatch":
        def mv(t):
            return None if t is None else t.to(device)
        return PagedBatch(mv(self.q), mv(self.key_pool), mv(self.value_pool),
                          mv(self.block_tables), mv(self.cu_seqlens_q), mv(self.context_lens),
                          mv(self.seq_lens), self.max_query_len, self.max_context_len, self.scale,
                          mv(self.k_scale), mv(self.v_scale), list(self.contexts),
                          list(self.query_lens))


def quantize_fp8_per_block(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``num_blocks x P x H_k x D`` float -> (float8_e4m3fn pool, ``num_blocks x H_k`` scales).

    One fp32 scale per (block, kv head), ``max|x| / 448`` over that page's rows of that
    head (448 = largest finite e4m3fn); stored value = e4m3fn(x / scale).
    """
    amax = x.abs().amax(dim=(1, 3)).float()                       # num_blocks x H_k
    scale = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    q = (x.float() / scale[:, None, :, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q, scale.contiguous()


def build_batch(contexts: list[int], query_lens: list[int], *, dtype: torch.dtype = torch.float32,
                kv_dtype: torch.dtype | None = None, num_q_heads: int = 16, num_kv_heads: int = 8,
                head_dim: int = 128, block_size: int = 16, spare_blocks: int = 3,
                shuffle: bool = True, seed: int = 0, pool_blocks: int | None = None,
                device: torch.device | str = "cpu", generator_device: str = "cpu") -> PagedBatch:
    """Pool, shuffled tables and ragged queries for the given per-sequence shapes.

    Draw order from one generator seeded with ``seed``: key pool, value pool, queries,
    block-id permutation. Values are N(0, 1) drawn in fp32 and cast to ``dtype``; an fp8
    ``kv_dtype`` quantises the fp32 draws per (block, kv head).
    """
    if len(contexts) != len(query_lens):
        raise ValueError("contexts and query_lens must have the same length")
    kv_dtype = kv_dtype or dtype
    blocks_each = [-(-c // block_size) for c in contexts]
    needed = sum(blocks_each)
    total = pool_blocks if pool_blocks is not None else needed + spare_blocks
    if total < needed:
        raise ValueError(f"pool of {total} blocks cannot hold {needed}")
    gen = torch.Generator(device=generator_device).manual_seed(seed)
    shape = (total, block_size, num_kv_heads, head_dim)
    keys = torch.randn(shape, generator=gen, dtype=torch.float32, device=generator_device)
    values = torch.randn(shape, generator=gen, dtype=torch.float32, device=generator_device)
    offsets = [0]
    for length in query_lens:
        offsets.append(offsets[-1] + length)
    q = torch.randn(offsets[-1], num_q_heads, head_dim, generator=gen, dtype=torch.float32,
                    device=generator_device)
    # The layout is drawn last, so shuffling changes only the layout, never the data.
    if shuffle:
        order = torch.randperm(total, generator=gen, device=generator_device).cpu().tolist()
    else:
        order = list(range(total))
    widest = max(blocks_each) if blocks_each else 1
    rows, cursor = [], 0
    for count in blocks_each:
        rows.append(order[cursor:cursor + count] + [-1] * (widest - count))
        cursor += count

    k_scale = v_scale = None
    if kv_dtype == torch.float8_e4m3fn:
        keys, k_scale = quantize_fp8_per_block(keys)
        values, v_scale = quantize_fp8_per_block(values)
        k_scale, v_scale = k_scale.to(device), v_scale.to(device)
    else:
        keys, values = keys.to(kv_dtype), values.to(kv_dtype)
    return PagedBatch(
        q=q.to(dtype).to(device),
        key_pool=keys.to(device),
        value_pool=values.to(device),
        block_tables=torch.tensor(rows, dtype=torch.int32, device=device),
        cu_seqlens_q=torch.tensor(offsets, dtype=torch.int32, device=device),
        context_lens=torch.tensor(contexts, dtype=torch.int32, device=device),
        seq_lens=torch.tensor(query_lens, dtype=torch.int32, device=device),
        max_query_len=max(query_lens) if query_lens else 1,
        max_context_len=max(contexts) if contexts else 1,
        scale=1.0 / math.sqrt(head_dim),
        k_scale=k_scale,
        v_scale=v_scale,
        contexts=list(contexts),
        query_lens=list(query_lens),
    )


def _draw_lengths(seed: int, n: int, low: int, high_inclusive: int) -> list[int]:
    gen = torch.Generator().manual_seed(seed)
    return torch.randint(low, high_inclusive + 1, (n,), generator=gen).tolist()


CONFIGS = {
    1: "paged decode, fp32, 4 seqs ctx {37,128,511,1000}, 512-block pool (CPU-runnable parity case)",
    2: "paged decode, bf16, batch 64, ctx U[512,4096] (bandwidth headline)",
    3: "chunked paged prefill, bf16, 8 seqs x (prefix U[0,1536] + 512-token chunk)",
    4: "paged decode, fp8-e4m3 KV with per-(block, kv head) scales, batch 128, ctx U[2048,8192]",
}


def config_batch(index: int, device: torch.device | str = "cpu", seed: int = 0,
                 generator_device: str = "cpu", kv_dtype: torch.dtype | None = None) -> PagedBatch:
    """The BASELINE.json config ``index`` (1-4), GQA 16q/8kv, D=128, 16-token pages.

    Lengths are drawn from their own generator (seed ``seed``) so the shapes do not
    depend on the tensor draws; pools for configs 2-4 hold the needed pages + 10%.
    ``kv_dtype=torch.float8_e4m3fn`` with config 3 gives its shape over an fp8 pool
    quantised per (block, kv head) as config 4's is.
    """
    common = dict(num_q_heads=16, num_kv_heads=8, head_dim=128, block_size=16, seed=seed,
                  device=device, generator_device=generator_device)
    if index == 1:
        contexts = [37, 128, 511, 1000]
        return build_batch(contexts, [1] * 4, dtype=torch.float32, pool_blocks=512, **common)
    if index == 2:
        contexts = _draw_lengths(seed, 64, 512, 4096)
        pages = sum(-(-c // 16) for c in contexts)
        return build_batch(contexts, [1] * 64, dtype=torch.bfloat16,
                           pool_blocks=math.ceil(1.1 * pages), **common)
    if index == 3:
        prefixes = _draw_lengths(seed, 8, 0, 1536)
        contexts = [p + 512 for p in prefixes]
        pages = sum(-(-c // 16) for c in contexts)
        return build_batch(contexts, [512] * 8, dtype=torch.bfloat16, kv_dtype=kv_dtype,
                           pool_blocks=math.ceil(1.1 * pages), **common)
    if index == 4:
        contexts = _draw_lengths(seed, 128, 2048, 8192)
        pages = sum(-(-c // 16) for c in contexts)
        return build_batch(contexts, [1] * 128, dtype=torch.bfloat16,
                           kv_dtype=torch.float8_e4m3fn, pool_blocks=math.ceil(1.1 * pages),
                           **common)
    raise ValueError(f"no config {index}")


def prefill_flops(batch: PagedBatch) -> int:
    """QK^T + PV flops over visible (query, key) pairs only: 4 * H_q * D per pair."""
    hq, d = batch.q.shape[1], batch.q.shape[2]
    pairs = 0
    for S, L in zip(batch.contexts, batch.query_lens):
        pairs += L * (S - L) + L * (L + 1) // 2
    return 4 * hq * d * pairs


# ----------------------------------------------------------------- config 5

CONFIG5_PROMPT_LEN = (64, 2048)   # inclusive bounds of the uniform prompt lengths
CONFIG5_BUDGET = 2048             # scheduled tokens per iteration
CONFIG5_CHUNK = 512               # prefill chunk


def config5_prompts(requests: int = 256, vocab_size: int = 151936, seed: int = 0) -> list[list[int]]:
    """BASELINE config 5's requests: prompt lengths U[64, 2048], token ids uniform in
    [0, vocab), drawn from one seeded CPU generator (lengths first, then each prompt)."""
    gen = torch.Generator().manual_seed(seed)
    lo, hi = CONFIG5_PROMPT_LEN
    lens = torch.randint(lo, hi + 1, (requests,), generator=gen).tolist()
    return [torch.randint(0, vocab_size, (n,), generator=gen).tolist() for n in lens]


def config5_pool_blocks(max_sequences: int = 32, max_tokens: int = 256, block_size: int = 16) -> int:
    """Pages for config 5's pool: every in-flight sequence at its longest, a margin, and
    the decode graphs' reserved dummy page (no preemption at this size)."""
    return max_sequences * -(-(CONFIG5_PROMPT_LEN[1] + max_tokens) // block_size) + 64 + 1
