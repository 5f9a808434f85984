"""Qwen3 over a paged KV pool (reference model/qwen3_paged.py:40-228).

The per-layer sequence is the reference's, op for op, because it is the caller the
hot path has to serve unchanged:

    attn_norm -> q/k/v projections -> QK-norm (rmsnorm over D) -> RoPE at
    batch.positions -> write K/V to the pool -> paged attention -> wo -> residual ->
    mlp_norm -> gate/up -> SwiGLU -> down -> residual

(QK-norm + RoPE of q and k run as one fused op, bitwise equal to the unfused
rmsnorm/rope pair, which with a 16-bit pool also writes K and V to their slots; the
K/V write is otherwise one op for K and V; a decode step over a 16-bit pool runs the
QK-norm, RoPE and K/V write inside the attention launch, bitwise the same. Decode-sized
steps, at most
64 rows, also fuse the projections: q/k/v as one launch, gate/up with SwiGLU as one,
and the o and down projections with their residual add, each rounded as the unfused
ops round; larger steps run the same ops as one BLAS call each over the concatenated
weights.)

and the forward returns one logits row per sequence (its last computed position),
through the final norm and the tied embedding (reference qwen3_paged.py:211-228).
Every op, projections included (``ops.linear``: the skinny kernel for decode-sized
inputs over weights packed at load, BLAS otherwise), goes through
``mini_vllm.kernels.ops`` with the model's ``use_cuda`` flag.

Weights are random (there is no checkpoint download here): N(0, 0.02) for matrices
and the embedding, ones for norm weights, seeded.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from mini_vllm import torch_path
from mini_vllm.kernels import ops

__all__ = ["ModelConfig", "Qwen3Paged", "random_weights"]


@dataclass(frozen=True)
class ModelConfig:
    """Qwen3-0.6B's shape by default (reference model/loader.py:53-120 reads the same
    fields from config.json)."""

    vocab_size: int = 151936
    hidden_size: int = 1024
    num_hidden_layers: int = 28
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 3072
    max_position_embeddings: int = 40960
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    dtype: torch.dtype = torch.bfloat16

    @property
    def q_size(self) -> int:
        return self.num_attention_heads * self.head_dim

    @property
    def kv_size(self) -> int:
        return self.num_key_value_heads * self.head_dim

    def num_params(self) -> int:
        e, i, v = self.hidden_size, self.intermediate_size, self.vocab_size
        per_layer = e * (self.q_size + 2 * self.kv_size) + self.q_size * e + 3 * e * i
        per_layer += 2 * e + 2 * self.head_dim
        return v * e + self.num_hidden_layers * per_layer + e


def random_weights(config: ModelConfig, seed: int = 0, device: torch.device | str = "cpu",
                   std: float = 0.02) -> dict[str, torch.Tensor]:
    """Seeded N(0, std) matrices (fp32 draws cast to the model dtype), unit norms."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    dt = config.dtype

    def mat(rows: int, cols: int) -> torch.Tensor:
        return (torch.randn(rows, cols, generator=gen) * std).to(dt).to(device)

    def ones(n: int) -> torch.Tensor:
        return torch.ones(n, dtype=dt, device=device)

    e = config.hidden_size
    w = {"embedding": mat(config.vocab_size, e), "final_norm": ones(e)}
    for layer in range(config.num_hidden_layers):
        pre = f"layers.{layer}."
        w[pre + "wq"] = mat(config.q_size, e)
        w[pre + "wk"] = mat(config.kv_size, e)
        w[pre + "wv"] = mat(config.kv_size, e)
        w[pre + "wo"] = mat(e, config.q_size)
        w[pre + "q_norm"] = ones(config.head_dim)
        w[pre + "k_norm"] = ones(config.head_dim)
        w[pre + "attn_norm"] = ones(e)
        w[pre + "mlp_norm"] = ones(e)
        w[pre + "gate"] = mat(config.intermediate_size, e)
        w[pre + "up"] = mat(config.intermediate_size, e)
        w[pre + "down"] = mat(e, config.intermediate_size)
    return w


class Qwen3Paged:
    """``model(batch) -> N x V`` logits, one row per sequence of the ragged batch."""

    def __init__(self, config: ModelConfig, weights: dict[str, torch.Tensor], manager,
                 use_cuda: bool = True) -> None:
        self.config = config
        self.weights = weights
        self.manager = manager
        self.use_cuda = use_cuda
        device = weights["embedding"].device
        self.cos, self.sin = torch_path.rope_tables(config.head_dim,
                                                    config.max_position_embeddings,
                                                    config.rope_theta, device=device)
        self.layers = []
        self.packed = []
        for layer in range(config.num_hidden_layers):
            pre = f"layers.{layer}."
            w = {k[len(pre):]: v for k, v in weights.items() if k.startswith(pre)}
            p = {}
            if use_cuda:
                # Decode-sized steps run q/k/v as one projection over the concatenated
                # weights (wq, wk, wv become row views of it: no second dense copy) and
                # gate/up as one projection over their 16-row interleave, fused with
                # SwiGLU; each decode weight also kept in the skinny kernels' packed order.
                wqkv = torch.cat((w["wq"], w["wk"], w["wv"]))
                w["wq"], w["wk"], w["wv"] = wqkv.split(
                    [config.q_size, config.kv_size, config.kv_size])
                p["qkv"] = ops.pack_weight(wqkv, use_cuda=True)
                p["o"] = ops.pack_weight(w["wo"], use_cuda=True)
                p["down"] = ops.pack_weight(w["down"], use_cuda=True)
                if config.intermediate_size % 16 == 0:
                    p["gate_up"] = ops.pack_weight(
                        torch_path.interleave_gate_up(w["gate"], w["up"]), use_cuda=True)
            self.layers.append(w)
            self.packed.append(p)
        # The logits projection over the tied embedding (its rows are also the token
        # lookup table, so the dense matrix stays).
        self.lm_head = (ops.pack_weight(weights["embedding"], use_cuda=True) if use_cuda
                        else weights["embedding"])

    @torch.no_grad()
    def prepare_prefill_products(self, max_tokens: int, sweep: bool = True) -> int:
        """Choose the library's hipBLASLt algorithms for the prefill-sized projections
        now rather than during serving: with ``sweep``, every algorithm is timed once per
        projection shape at ``max_tokens`` rows (its fastest join every later choice);
        then each shape runs once for every row count class up to ``max_tokens``, so an
        algorithm is chosen (and timed) for each 128-row bucket and each whole multiple
        of 128. The layers share their shapes, so layer 0's weights stand for all.
        Returns the products run (0 on the PyTorch path, which keeps nothing)."""
        if not self.use_cuda or not self.packed:
            return 0
        w, p = self.layers[0], self.packed[0]
        weights = [p["qkv"], p["o"], p.get("gate_up", w["gate"]), p["down"]]
        device, dtype = self.weights["embedding"].device, self.config.dtype
        runs = 0
        if sweep and max_tokens > 64 and dtype in (torch.float16, torch.bfloat16):
            from mini_vllm.kernels.extension import load_extension

            ext = load_extension()
            for pw in weights:
                dense = pw.dense if isinstance(pw, ops.PackedWeight) else pw
                # random rows: constant operands time some kernels faster than real data
                x = torch.randn(max_tokens, dense.shape[1], device=device).to(dtype)
                if ext.blas_linear_supported(x, dense):
                    ext.blas_tune(x, dense)
                    runs += 1
        for j in range(max_tokens // 128 + 1):
            for m in (128 * j + 65, 128 * (j + 1)):
                if m > max_tokens or m <= 64:
                    continue
                for pw in weights:
                    k = pw.shape[1]
                    ops.linear(torch.randn(m, k, device=device).to(dtype), pw, use_cuda=True)
                    runs += 1
        return runs

    def _attention_block(self, layer: int, w: dict, p: dict, x: torch.Tensor, h: torch.Tensor,
                         batch, fused: bool) -> tuple[torch.Tensor, torch.Tensor]:
        """(h + wo(attention(x)), mlp_norm of that) for normed input x: the attention
        output, then the projection with its residual and norm."""
        out = self._attention(layer, w, p, x, batch, fused)
        return self._residual_norm(out, p.get("o"), w["wo"], h, w["mlp_norm"], fused)

    def _attention(self, layer: int, w: dict, p: dict, x: torch.Tensor, batch,
                   fused: bool) -> torch.Tensor:
        """The attention output (``T x H_q D``) of normed input x, before ``wo``."""
        c = self.config
        q, k, v = self._projections(w, p, x, fused)
        if fused and batch.max_query_len == 1:
            # A decode step: QK-norm, RoPE and the KV write inside the attention launch.
            kv = self.manager.kv
            out = ops.paged_decode_qk_norm_rope(
                q, k, v, w["q_norm"], w["k_norm"], self.cos, self.sin, c.rms_norm_eps,
                kv.layer_keys(layer), kv.layer_values(layer), batch.block_tables,
                batch.cu_seqlens_q, batch.context_lens, batch.seq_lens, batch.max_context_len,
                1.0 / math.sqrt(c.head_dim), use_cuda=self.use_cuda)
            if out is not None:
                return out.view(q.shape[0], c.q_size)
        return self._paged(layer, self._queries(layer, w, q, k, v, batch), batch)

    def _projections(self, w: dict, p: dict, x: torch.Tensor,
                     fused: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """q (``T x H_q x D``), k and v (``T x H_k x D``) of normed input x, before
        QK-norm and RoPE (with the fused projection, column views of its output)."""
        c = self.config
        t = x.shape[0]
        u = self.use_cuda
        if fused:
            q, k, v = ops.linear_split(x, p["qkv"], (c.q_size, c.kv_size, c.kv_size), use_cuda=u,
                                       views=True)
        else:
            q, k, v = (ops.linear(x, w[n], use_cuda=u) for n in ("wq", "wk", "wv"))
        return (q.view(t, c.num_attention_heads, c.head_dim),
                k.view(t, c.num_key_value_heads, c.head_dim),
                v.view(t, c.num_key_value_heads, c.head_dim))

    def _queries(self, layer: int, w: dict, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                 batch) -> torch.Tensor:
        """q (``T x H_q x D``, contiguous) after QK-norm and RoPE, with this step's K and
        V written to the layer's pages."""
        c = self.config
        u = self.use_cuda
        kv = self.manager.kv
        qr = ops.qk_norm_rope_kv_write(q, k, v, w["q_norm"], w["k_norm"], batch.positions,
                                       self.cos, self.sin, c.rms_norm_eps, kv.layer_keys(layer),
                                       kv.layer_values(layer), batch.slot_mapping, use_cuda=u)
        if qr is not None:
            q = qr
        else:
            q, k = ops.qk_norm_rope(q.contiguous(), k.contiguous(), w["q_norm"], w["k_norm"],
                                    batch.positions, self.cos, self.sin, c.rms_norm_eps, use_cuda=u)
            kv.write(layer, batch.slot_mapping, k, v.contiguous(), use_cuda=u)
        return q.contiguous()

    def _paged(self, layer: int, q: torch.Tensor, batch) -> torch.Tensor:
        """The paged attention of q over the layer's pages (``T x H_q D``)."""
        c = self.config
        kv = self.manager.kv
        k_scale, v_scale = kv.layer_scales(layer)
        out = ops.paged_attention(
            q, kv.layer_keys(layer), kv.layer_values(layer), batch.block_tables,
            batch.cu_seqlens_q, batch.context_lens, batch.seq_lens, batch.max_query_len,
            batch.max_context_len, 1.0 / math.sqrt(c.head_dim), use_cuda=self.use_cuda,
            k_scale=k_scale, v_scale=v_scale)
        return out.view(q.shape[0], c.q_size)

    def _residual_norm(self, x: torch.Tensor, pw, dense_w: torch.Tensor, h: torch.Tensor,
                       norm_w: torch.Tensor, fused: bool) -> tuple[torch.Tensor, torch.Tensor]:
        """(h + x w^T, rmsnorm of that): the o and down projections with the norm that
        follows each, fused into the projection's reduction when the kernels serve it."""
        c = self.config
        u = self.use_cuda
        if fused:
            both = ops.linear_residual_rmsnorm(x, pw, h, norm_w, c.rms_norm_eps, use_cuda=u)
            if both is not None:
                return both
            if not ops.skinny(x, use_cuda=u):
                # prefill-sized: the BLAS product, then the add and the norm in one pass
                return ops.add_rmsnorm(ops.linear(x, pw, use_cuda=u), h, norm_w,
                                       c.rms_norm_eps, use_cuda=u)
            h = ops.linear_residual(x, pw, h, use_cuda=u)
        else:
            h = h + ops.linear(x, dense_w, use_cuda=u)
        return h, ops.rmsnorm(h, norm_w, c.rms_norm_eps, use_cuda=u)

    @torch.no_grad()
    def __call__(self, batch) -> torch.Tensor:
        c = self.config
        u = self.use_cuda
        # The token embeddings and the first block's input norm (one launch with the
        # kernels on); a decode graph's batch names its input tokens by (ids, index, prev).
        ids, index, prev = batch.input_source or (batch.input_ids, None, None)
        h, normed = ops.embed_rmsnorm(self.weights["embedding"], ids, self.layers[0]["attn_norm"],
                                      c.rms_norm_eps, use_cuda=u, index=index, prev=prev)
        # With the kernels on, every step takes the fused ops: decode-sized ones run the
        # skinny kernels, larger ones (prefill chunks) one BLAS call over the
        # concatenated weights instead of three (q/k/v) or two (gate/up).
        fused = u
        n_layers = len(self.layers)
        for layer, (w, p) in enumerate(zip(self.layers, self.packed)):
            # normed = attn_norm(h) of this layer, computed by the previous layer's
            # down projection (or above, for the first layer).
            h, normed = self._attention_block(layer, w, p, normed, h, batch, fused)
            if fused and "gate_up" in p:
                gated = ops.linear_swiglu(normed, p["gate_up"], use_cuda=u)
            else:
                gated = ops.swiglu(ops.linear(normed, w["gate"], use_cuda=u),
                                   ops.linear(normed, w["up"], use_cuda=u), use_cuda=u)
            last = layer + 1 == n_layers
            next_norm = self.weights["final_norm"] if last else self.layers[layer + 1]["attn_norm"]
            if last and batch.total_tokens > batch.num_sequences:
                # Only each sequence's last row reaches the logits (reference
                # qwen3_paged.py:211-228), and everything after the attention is
                # row-wise: the last down projection, its residual and the final norm
                # run on those rows alone.
                rows = batch.last_row_indices
                gated, h = gated.index_select(0, rows), h.index_select(0, rows)
            h, normed = self._residual_norm(gated, p.get("down"), w["down"], h, next_norm, fused)
        # normed is now final_norm(h) of each sequence's last row.
        return ops.linear(normed, self.lm_head, use_cuda=u)
