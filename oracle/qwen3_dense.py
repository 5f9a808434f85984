"""Dense, cache-free Qwen3 forward for greedy generation (test infrastructure only).

Each step recomputes the whole token sequence with full causal attention, in float64
by default, from the same weights dict as ``mini_vllm.model.qwen3_paged`` (the
reference's recompute model, model/qwen3.py, restated): no pages, no chunks, no
kernels, so a paged engine that agrees with it token for token got its batching,
slots, positions and masks right. Returns the tokens and each step's logits so a test
can tell a genuine near-tie from a bug.

``DenseQwen3(..., kv_fp8=True)`` is the same model with its K/V cache held the way an
fp8-e4m3 paged pool holds it (the reference has no fp8 cache): every K/V row written
through ``oracle.kv_write.kv_write_fp8`` (per-(page, kv head) power-of-two scales,
rows re-encoded when a scale grows) onto 16-row pages at slot = position, the prompt
in one write and each generated token in its own, and attention reading the
dequantised values. Everything else stays float64.
"""

from __future__ import annotations

import math

import numpy as np
import torch

__all__ = ["DenseQwen3", "Fp8Pages", "generate_greedy", "generate_greedy_cached"]


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


class Fp8Pages:
    """One sequence's K/V as fp8-e4m3 pages, per layer: positions on ``block_size``-row
    pages with slot = position, written through ``oracle.kv_write.kv_write_fp8`` (the
    values taken as float32, as the kernels receive them), read back dequantised
    (code x its page's scale) in float64."""

    def __init__(self, layers: int, kv_heads: int, head_dim: int, block_size: int = 16):
        self.bs, self.hk, self.d = block_size, kv_heads, head_dim
        shape = (0, block_size, kv_heads, head_dim)
        self.codes = [[np.zeros(shape, np.uint8), np.zeros(shape, np.uint8)] for _ in range(layers)]
        self.scales = [[np.zeros((0, kv_heads), np.float32), np.zeros((0, kv_heads), np.float32)]
                       for _ in range(layers)]
        self.values = [[torch.zeros(0, kv_heads, head_dim, dtype=torch.float64) for _ in range(2)]
                       for _ in range(layers)]

    def write(self, layer: int, start: int, k: torch.Tensor, v: torch.Tensor):
        """Write rows ``start ..`` of K and V (``t x H_k x D``); returns (keys, values)
        of every position so far, dequantised."""
        from oracle.elementwise import fp8_e4m3_decode
        from oracle.kv_write import kv_write_fp8

        t = k.shape[0]
        end = start + t
        blocks = -(-end // self.bs)
        slots = np.arange(start, end, dtype=np.int64)
        first = start // self.bs
        out = []
        for i, x in enumerate((k, v)):
            codes, scales = self.codes[layer][i], self.scales[layer][i]
            if codes.shape[0] < blocks:
                grow = blocks - codes.shape[0]
                codes = np.concatenate([codes, np.zeros((grow,) + codes.shape[1:], np.uint8)])
                scales = np.concatenate([scales, np.zeros((grow, self.hk), np.float32)])
            codes, scales = kv_write_fp8(codes, scales, slots,
                                         x.detach().to(torch.float32).cpu().numpy())
            self.codes[layer][i], self.scales[layer][i] = codes, scales
            # refresh the dequantised rows of the pages this write touched
            deq = fp8_e4m3_decode(codes[first:blocks]).astype(np.float64) * \
                scales[first:blocks][:, None, :, None].astype(np.float64)
            rows = torch.from_numpy(deq.reshape(-1, self.hk, self.d))
            kept = self.values[layer][i][:first * self.bs]
            self.values[layer][i] = torch.cat([kept, rows])[:end]
            out.append(self.values[layer][i])
        return out[0], out[1]


def _forward_cached(config, layers, emb, final_norm, ids, start, cache, dtype, pages=None):
    """Rows ``start .. start + len(ids) - 1`` of the same dense forward, their K/V
    appended to ``cache`` (one [keys, values] pair per layer) - or written to ``pages``
    (an :class:`Fp8Pages`) - attending causally over every cached position; returns
    the last row's logits."""
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
        if pages is not None:
            keys, vals = pages.write(layer, start, k, v)
            keys, vals = keys.to(dtype), vals.to(dtype)
        else:
            if len(cache) <= layer:
                cache.append([k, v])
            else:
                cache[layer] = [torch.cat([cache[layer][0], k]), torch.cat([cache[layer][1], v])]
            keys, vals = cache[layer]
        keys = keys.repeat_interleave(g, dim=1)
        vals = vals.repeat_interleave(g, dim=1)
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

    def __init__(self, config, weights, dtype=torch.float64, kv_fp8: bool = False):
        w = {k: v.detach().cpu() for k, v in weights.items()}
        self.config, self.dtype, self.kv_fp8 = config, dtype, kv_fp8
        self.layers = _layer_weights(config, w, dtype)
        self.emb, self.final_norm = w["embedding"].to(dtype), w["final_norm"].to(dtype)

    def generate(self, prompt, max_tokens):
        """Greedy continuation with each layer's K/V kept between steps: the prompt in
        one pass, then one token per step against the cache. The same dense causal math
        as :func:`generate_greedy` (no pages, no chunks, no kernels). Returns (tokens,
        per-step logits)."""
        c = self.config
        args = (c, self.layers, self.emb, self.final_norm)
        cache: list = []
        pages = (Fp8Pages(c.num_hidden_layers, c.num_key_value_heads, c.head_dim)
                 if self.kv_fp8 else None)
        tokens, logits = [], []
        out = _forward_cached(*args, list(prompt), 0, cache, self.dtype, pages)
        pos = len(prompt)
        for _ in range(max_tokens):
            tok = int(out.argmax())
            tokens.append(tok)
            logits.append(out)
            if len(tokens) == max_tokens:
                break
            out = _forward_cached(*args, [tok], pos, cache, self.dtype, pages)
            pos += 1
        return tokens, logits

    def forced(self, prompt, tokens):
        """Teacher forcing: the logits before each of ``tokens`` when the sequence
        continues with exactly them (row i predicts tokens[i] from prompt + tokens[:i]),
        so another model's whole continuation can be judged step by step, not only up to
        its first divergence."""
        return _forced(self, prompt, tokens)


def _forced(model: "DenseQwen3", prompt, tokens):
    c = model.config
    args = (c, model.layers, model.emb, model.final_norm)
    pages = (Fp8Pages(c.num_hidden_layers, c.num_key_value_heads, c.head_dim)
             if model.kv_fp8 else None)
    cache: list = []
    logits = [_forward_cached(*args, list(prompt), 0, cache, model.dtype, pages)]
    pos = len(prompt)
    for tok in list(tokens)[:-1]:
        logits.append(_forward_cached(*args, [int(tok)], pos, cache, model.dtype, pages))
        pos += 1
    return logits


def generate_greedy_cached(config, weights, prompt, max_tokens, dtype=torch.float64):
    """:func:`generate_greedy` through :class:`DenseQwen3`'s KV-cached loop."""
    return DenseQwen3(config, weights, dtype).generate(prompt, max_tokens)
