"""Regenerate tests/golden/qwen3_tiny_hf.npz (test infrastructure).

An independent pin of the dense model oracle (oracle/qwen3_dense.py): the Hugging Face
``transformers`` Qwen3 implementation (``Qwen3ForCausalLM``, transformers 5.15.0 as
installed here; the reference pins its own model the same way, tests/test_qwen3.py)
run in float64 on the tiny test shape (vocab 512, hidden 64, 2 layers, 4 q heads over
2 kv heads, head_dim 32, SwiGLU 128, RoPE theta 1e6, tied embedding) with this
repository's seeded weights (``mini_vllm.model.random_weights(seed=3)``, float32 draws)
and seeded non-unit norm weights, so that every norm's wiring is visible.

Stored: the prompts, 8 greedy tokens per prompt and the next-token logits at each of
those steps (so the last position at 8 lengths), plus a SHA-256 of the weights so a
change in the weight generator is reported as such rather than read as a model bug.
transformers is imported here only; the test reads the fixture.

Run:  python tests/golden/make_qwen3_golden.py
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path[:0] = [str(REPO / "mini-vllm_amd"), str(REPO), str(REPO / "tests")]

from engine_helpers import prompts, tiny_config  # noqa: E402
from mini_vllm.model import random_weights  # noqa: E402

SEED = 3
STEPS = 8


def golden_weights() -> tuple[object, dict[str, torch.Tensor]]:
    """The tiny model's config and weights the fixture was made from: seeded matrices
    and seeded norm weights in [0.5, 1.5) (random_weights leaves norms at one)."""
    config = tiny_config(torch.float32)
    weights = random_weights(config, seed=SEED)
    gen = torch.Generator().manual_seed(SEED + 100)
    for name in sorted(weights):
        if name.endswith("norm"):
            weights[name] = torch.rand(weights[name].shape, generator=gen) + 0.5
    return config, weights


def weights_digest(weights: dict[str, torch.Tensor]) -> str:
    h = hashlib.sha256()
    for name in sorted(weights):
        h.update(name.encode() + weights[name].to(torch.float32).contiguous().numpy().tobytes())
    return h.hexdigest()


def hf_model(config, weights):
    from transformers import Qwen3Config, Qwen3ForCausalLM

    c = config
    hf = Qwen3Config(vocab_size=c.vocab_size, hidden_size=c.hidden_size,
                     num_hidden_layers=c.num_hidden_layers,
                     num_attention_heads=c.num_attention_heads,
                     num_key_value_heads=c.num_key_value_heads, head_dim=c.head_dim,
                     intermediate_size=c.intermediate_size,
                     max_position_embeddings=c.max_position_embeddings,
                     rms_norm_eps=c.rms_norm_eps, rope_theta=c.rope_theta,
                     tie_word_embeddings=True, attention_bias=False,
                     attn_implementation="eager")
    model = Qwen3ForCausalLM(hf).to(torch.float64).eval()
    names = {"wq": "self_attn.q_proj", "wk": "self_attn.k_proj", "wv": "self_attn.v_proj",
             "wo": "self_attn.o_proj", "q_norm": "self_attn.q_norm",
             "k_norm": "self_attn.k_norm", "attn_norm": "input_layernorm",
             "mlp_norm": "post_attention_layernorm", "gate": "mlp.gate_proj",
             "up": "mlp.up_proj", "down": "mlp.down_proj"}
    state = {"model.embed_tokens.weight": weights["embedding"],
             "model.norm.weight": weights["final_norm"],
             "lm_head.weight": weights["embedding"]}
    for layer in range(c.num_hidden_layers):
        for ours, theirs in names.items():
            state[f"model.layers.{layer}.{theirs}.weight"] = weights[f"layers.{layer}.{ours}"]
    missing, unexpected = model.load_state_dict({k: v.to(torch.float64) for k, v in state.items()},
                                                strict=False)
    if missing or unexpected:
        raise RuntimeError(f"weight mapping: missing {missing}, unexpected {unexpected}")
    return model


def main() -> None:
    config, weights = golden_weights()
    model = hf_model(config, weights)
    ps = prompts(3, 5, 40, config.vocab_size, seed=21)
    out = {"weights_sha256": np.array(weights_digest(weights)),
           "num_prompts": np.array(len(ps))}
    with torch.no_grad():
        for i, p in enumerate(ps):
            ids = torch.tensor([p])
            out[f"prompt_{i}"] = np.array(p, dtype=np.int64)
            tokens, steps = [], []
            for _ in range(STEPS):
                logits = model(ids).logits[0, -1]
                tok = int(logits.argmax())
                tokens.append(tok)
                steps.append(logits.numpy())
                ids = torch.cat([ids, torch.tensor([[tok]])], dim=1)
            out[f"tokens_{i}"] = np.array(tokens, dtype=np.int64)
            out[f"step_logits_{i}"] = np.stack(steps)
    np.savez_compressed(HERE / "qwen3_tiny_hf.npz", **out)
    print(f"wrote {HERE / 'qwen3_tiny_hf.npz'}")


if __name__ == "__main__":
    main()
