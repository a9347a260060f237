"""Model shape record for the Qwen3 dense family (the attributes the
reference reads from its HF config: src/compute/models/qwen3.py:131-185,
src/compute/kv_pool.py:9-15).  Any object with these attribute names (e.g. a
transformers Qwen3Config) is accepted where a config is expected."""
from __future__ import annotations

from dataclasses import dataclass


@dataclass
class Qwen3Shape:
    hidden_size: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    intermediate_size: int
    num_hidden_layers: int
    vocab_size: int = 151936
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    max_position_embeddings: int = 40960
    attention_bias: bool = False


QWEN3_0_6B = Qwen3Shape(1024, 16, 8, 128, 3072, 28)
QWEN3_8B = Qwen3Shape(4096, 32, 8, 128, 12288, 36)
QWEN3_32B = Qwen3Shape(5120, 64, 8, 128, 25600, 64)


def rope_theta(cfg) -> float:
    """rope_theta of a config (transformers >= 5 keeps it in rope_parameters)."""
    t = getattr(cfg, "rope_theta", None)
    if t is None:
        t = (getattr(cfg, "rope_parameters", None) or {}).get("rope_theta", 1e6)
    return float(t)


def head_dim(cfg) -> int:
    return getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
