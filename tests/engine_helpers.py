"""Shared pieces of the engine tests: the tiny model and a tie-aware token check."""

from __future__ import annotations

import torch

from mini_vllm.block import BlockManager
from mini_vllm.model import ModelConfig, Qwen3Paged, random_weights
from mini_vllm.serve import LLMEngine, SchedulerConfig

# Keeps two properties of Qwen3-0.6B that catch reshape bugs: H_q * D != E, and a
# GQA group of 2 (the reference's tiny model, tests/conftest.py:70-82).
TINY = dict(vocab_size=512, hidden_size=64, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, head_dim=32, intermediate_size=128,
            max_position_embeddings=256)


def tiny_config(dtype=torch.float32, **over) -> ModelConfig:
    return ModelConfig(**{**TINY, **over}, dtype=dtype)


def make_engine(config, weights, *, num_blocks=64, block_size=16, use_cuda=False,
                device="cpu", sched=None, use_graphs=False, kv_dtype=None) -> LLMEngine:
    manager = BlockManager(num_blocks, block_size, config.num_hidden_layers,
                           config.num_key_value_heads, config.head_dim,
                           kv_dtype or config.dtype, device)
    model = Qwen3Paged(config, weights, manager, use_cuda=use_cuda)
    return LLMEngine(model, sched or SchedulerConfig(), device=device, use_graphs=use_graphs)


def prompts(n, lo, hi, vocab, seed=0):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (n,), generator=g).tolist()
    return [torch.randint(0, vocab, (L,), generator=g).tolist() for L in lens]


def assert_tokens_match(got, want_tokens, want_logits, tie_tol, msg=""):
    """Equal token for token, except a genuine near-tie: where they first differ, the
    engine's token must be within ``tie_tol`` of the reference's best logit; the rest
    of the continuation then legitimately diverges and is not compared."""
    for i, (a, b) in enumerate(zip(got, want_tokens)):
        if a == b:
            continue
        gap = float(want_logits[i].max() - want_logits[i][a])
        assert gap <= tie_tol, f"{msg} step {i}: token {a} vs {b}, logit gap {gap:.3e} > {tie_tol}"
        return
    assert len(got) == len(want_tokens), msg
