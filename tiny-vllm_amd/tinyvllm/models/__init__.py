"""Model families on the decode path."""
from tinyvllm.models.qwen3 import Qwen3Config, Qwen3ForCausalLM

__all__ = ["Qwen3Config", "Qwen3ForCausalLM"]
