"""The paged Qwen3 model: the caller of every hot-path op."""

from mini_vllm.model.qwen3_paged import ModelConfig, Qwen3Paged, random_weights

__all__ = ["ModelConfig", "Qwen3Paged", "random_weights"]
