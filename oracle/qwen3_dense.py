"""Dense, cache-free Qwen3 forward for greedy generation (test infrastructure only).

Each step recomputes the whole token sequence with full causal attention, in float64
by default, from the same weights dict as ``mini_vllm.model.qwen3_paged`` (the
reference's recompute model, model/qwen3.py, restated): no pages, no chunks, no
kernels, so a paged engine that agrees with it token for token got its batching,
slots, positions and masks right. Returns the tokens and each step's logits so a test
can tell a genuine near-tie from a bug.
"""

from __future__ import annotations

import math

import torch

__all__ = ["DenseQwen3", "generate_greedy", "generate_greedy_cached"]


def _rms(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def _rope(x, pos, theta, dtype):
    d = x.shape[-1]
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=dtype) / d))
    ang = torch.outer(pos.to(dtype), inv)
    cos = torch.cat([ang.cos(), ang.cos()], -1)[:, None, :]
    sin = torch.cat([ang.sin(), ang.sin()], -1)[:, None, :]
    half = d // 2
    rot = torch.cat([-x[..., half:], x[..., :half]], -1)
    return x * cos + rot * sin


def _forward_last(config, w, ids, dtype):
    c = config
    t = len(ids)
    h = w["embedding"].to(dtype)[torch.tensor(ids)]
    pos = torch.arange(t)
    g = c.num_attention_heads // c.num_key_value_heads
    mask = torch.full((t, t), float("-inf"), dtype=dtype).triu(1)
    for layer in range(c.num_hidden_layers):
        lw = {k.split(".", 2)[2]: v.to(dtype) for k, v in w.items() if k.startswith(f"layers.{layer}.")}
        x = _rms(h, lw["attn_norm"], c.rms_norm_eps)
        q = (x @ lw["wq"].t()).view(t, c.num_attention_heads, c.head_dim)
        k = (x @ lw["wk"].t()).view(t, c.num_key_value_heads, c.head_dim)
        v = (x @ lw["wv"].t()).view(t, c.num_key_value_heads, c.head_dim)
        q = _rope(_rms(q, lw["q_norm"], c.rms_norm_eps), pos, c.rope_theta, dtype)
        k = _rope(_rms(k, lw["k_norm"], c.rms_norm_eps), pos, c.rope_theta, dtype)
        k = k.repeat_interleave(g, dim=1)
        v = v.repeat_interleave(g, dim=1)
        scores = torch.einsum("qhd,khd->hqk", q, k) / math.sqrt(c.head_dim) + mask
        att = torch.einsum("hqk,khd->qhd", torch.softmax(scores, -1), v)
        h = h + att.reshape(t, -1) @ lw["wo"].t()
        x = _rms(h, lw["mlp_norm"], c.rms_norm_eps)
        gate = x @ lw["gate"].t()
        h = h + (gate * torch.sigmoid(gate) * (x @ lw["up"].t())) @ lw["down"].t()
    last = _rms(h[-1:], w["final_norm"].to(dtype), c.rms_norm_eps)
    return (last @ w["embedding"].to(dtype).t())[0]


def generate_greedy(config, weights, prompt, max_tokens, dtype=torch.float64):
    """Greedy continuation of ``prompt``: (tokens, per-step logits)."""
    w = {k: v.detach().cpu() for k, v in weights.items()}
    ids = list(prompt)
    tokens, logits = [], []
    for _ in range(max_tokens):
        out = _forward_last(config, w, ids, dtype)
        tok = int(out.argmax())
        tokens.append(tok)
        logits.append(out)
        ids.append(tok)
    return tokens, logits


def _layer_weights(config, weights, dtype):
    return [{k.split(".", 2)[2]: v.to(dtype) for k, v in weights.items()
             if k.startswith(f"layers.{layer}.")} for layer in range(config.num_hidden_layers)]


def _forward_cached(config, layers, emb, final_norm, ids, start, cache, dtype):
    """Rows ``start .. start + len(ids) - 1`` of the same dense forward, their K/V
    appended to ``cache`` (one [keys, values] pair per layer), attending causally over
    every cached position; returns the last row's logits."""
    c = config
    t = len(ids)
    h = emb[torch.tensor(ids)]
    pos = torch.arange(start, start + t)
    g = c.num_attention_heads // c.num_key_value_heads
    s = start + t
    mask = torch.full((t, s), float("-inf"), dtype=dtype).triu(start + 1)
    for layer, lw in enumerate(layers):
        x = _rms(h, lw["attn_norm"], c.rms_norm_eps)
        q = (x @ lw["wq"].t()).view(t, c.num_attention_heads, c.head_dim)
        k = (x @ lw["wk"].t()).view(t, c.num_key_value_heads, c.head_dim)
        v = (x @ lw["wv"].t()).view(t, c.num_key_value_heads, c.head_dim)
        q = _rope(_rms(q, lw["q_norm"], c.rms_norm_eps), pos, c.rope_theta, dtype)
        k = _rope(_rms(k, lw["k_norm"], c.rms_norm_eps), pos, c.rope_theta, dtype)
        if len(cache) <= layer:
            cache.append([k, v])
        else:
            cache[layer] = [torch.cat([cache[layer][0], k]), torch.cat([cache[layer][1], v])]
        keys = cache[layer][0].repeat_interleave(g, dim=1)
        vals = cache[layer][1].repeat_interleave(g, dim=1)
        scores = torch.einsum("qhd,khd->hqk", q, keys) / math.sqrt(c.head_dim) + mask
        att = torch.einsum("hqk,khd->qhd", torch.softmax(scores, -1), vals)
        h = h + att.reshape(t, -1) @ lw["wo"].t()
        x = _rms(h, lw["mlp_norm"], c.rms_norm_eps)
        gate = x @ lw["gate"].t()
        h = h + (gate * torch.sigmoid(gate) * (x @ lw["up"].t())) @ lw["down"].t()
    last = _rms(h[-1:], final_norm, c.rms_norm_eps)
    return (last @ emb.t())[0]


class DenseQwen3:
    """The dense model with its weights converted to ``dtype`` once, for several
    :meth:`generate` calls (the 0.6B shape's float64 weights take ~5 GB)."""

    def __init__(self, config, weights, dtype=torch.float64):
        w = {k: v.detach().cpu() for k, v in weights.items()}
        self.config, self.dtype = config, dtype
        self.layers = _layer_weights(config, w, dtype)
        self.emb, self.final_norm = w["embedding"].to(dtype), w["final_norm"].to(dtype)

    def generate(self, prompt, max_tokens):
        """Greedy continuation with each layer's K/V kept between steps: the prompt in
        one pass, then one token per step against the cache. The same dense causal math
        as :func:`generate_greedy` (no pages, no chunks, no kernels). Returns (tokens,
        per-step logits)."""
        args = (self.config, self.layers, self.emb, self.final_norm)
        cache: list = []
        tokens, logits = [], []
        out = _forward_cached(*args, list(prompt), 0, cache, self.dtype)
        pos = len(prompt)
        for _ in range(max_tokens):
            tok = int(out.argmax())
            tokens.append(tok)
            logits.append(out)
            if len(tokens) == max_tokens:
                break
            out = _forward_cached(*args, [tok], pos, cache, self.dtype)
            pos += 1
        return tokens, logits


def generate_greedy_cached(config, weights, prompt, max_tokens, dtype=torch.float64):
    """:func:`generate_greedy` through :class:`DenseQwen3`'s KV-cached loop."""
    return DenseQwen3(config, weights, dtype).generate(prompt, max_tokens)
