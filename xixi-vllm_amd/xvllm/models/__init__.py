from .qwen3 import Qwen3ForCausalLM

__all__ = ["Qwen3ForCausalLM"]
