from .attention import Attention, AttnInputs, AttnMetadata, attention_context
from .layernorm import RMSNorm
from .rotary import RotaryEmbedding, build_cos_sin_cache
from .activation import SiluAndMul

__all__ = [
    "Attention", "AttnInputs", "AttnMetadata", "attention_context", "RMSNorm",
    "RotaryEmbedding", "build_cos_sin_cache", "SiluAndMul",
]
